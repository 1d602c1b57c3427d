// MFMA kernels of the MoC hot path (gfx950).
//
// The K-contractions of MoC are GEMMs with K (<= 64 here) on one side:
//   forward  W[t, s, d]   = sum_k alpha[t,k] basis[k,s,d]        (tokens x K) . (K x channels)
//   dalpha   da[t, k]     = sum_{s,d} m_s[t,d] basis[k,s,d]     contraction over (s, d)
//   dbasis   db[k, s, d]  = sum_t alpha[t,k] m_s[t,d]           contraction over tokens
// with m_s[t,d] = g[t,d] x[t-(S-1-s), d] and g = dy * silu'(P) (or dy).  They run
// on the matrix cores (v_mfma_f32_16x16x16_bf16 for bf16 data, v_mfma_f32_16x16x4_f32
// for fp32 data); the per-channel convolution, SiLU and their gradients run on
// VALU in fp32 directly on the MFMA result registers.
//
// Register layout ("design A").  A 16x16 MFMA result block holds, in lane
// l = j + 16 q (j = l % 16, q = l / 16), column j and rows 4q..4q+3.  Columns are
// channels, rows are tokens.  A wave processes a super-block of TB = 16 NB tokens
// and CW = 16 NC channels:
//   * lane (j, q) owns channels d0 + NC j + c (c < NC, contiguous: one vector
//     load per token row) and tokens t0 + R q + r (r < R = 4 NB, contiguous: the
//     S-1 halo rows of the causal window are shared in registers);
//   * MFMA row i of token block b is token t0 + R (i/4) + 4 b + (i%4), which is
//     what makes the rows of a lane consecutive;
//   * every lane holds contraction entries k = 16 kc + 4 q + {0..3} of the K axis
//     for both A and B operands (bf16: one 16x16x16 MFMA; fp32: four 16x16x4).
// The forward never materialises W: one 16x16 block of W per (token block,
// channel block, tap) lives in 4 VGPRs between the MFMA and its FMAs.
#pragma once

#include <type_traits>

#include "moc_common.h"

namespace moc {
namespace mfma {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// compute-type traits: BF = bf16 operands (x is bf16), else fp32 operands.
template <bool BF>
struct CT;

template <>
struct CT<true> {
  using elem = uint16_t;
  using opnd = s16x4;
  static __device__ __forceinline__ f32x4 mma(opnd a, opnd b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(elem e) { return bf16_to_f32(e); }
  static __device__ __forceinline__ elem from_f(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ opnd make(elem a, elem b, elem c, elem d) {
    opnd o;
    o[0] = static_cast<short>(a);
    o[1] = static_cast<short>(b);
    o[2] = static_cast<short>(c);
    o[3] = static_cast<short>(d);
    return o;
  }
  static __device__ __forceinline__ opnd zero() { return opnd{0, 0, 0, 0}; }
};

template <>
struct CT<false> {
  using elem = float;
  using opnd = f32x4;
  static __device__ __forceinline__ f32x4 mma(opnd a, opnd b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
    return c;
  }
  static __device__ __forceinline__ float to_f(elem e) { return e; }
  static __device__ __forceinline__ elem from_f(float v) { return v; }
  static __device__ __forceinline__ opnd make(elem a, elem b, elem c, elem d) {
    return opnd{a, b, c, d};
  }
  static __device__ __forceinline__ opnd zero() { return opnd{0.f, 0.f, 0.f, 0.f}; }
};

// Vector of N elements moved with one load / store (N * sizeof(E) in {4, 8, 16}).
template <typename E, int N>
struct Vec {
  static constexpr int kBytes = N * static_cast<int>(sizeof(E));
  using raw = typename std::conditional<
      kBytes == 4, uint32_t,
      typename std::conditional<kBytes == 8, uint2,
                                typename std::conditional<kBytes == 16, uint4, void>::type>::type>::type;
  static __device__ __forceinline__ void load(const E* p, E (&out)[N]) {
    const raw r = *reinterpret_cast<const raw*>(p);
    __builtin_memcpy(out, &r, sizeof(r));
  }
  static __device__ __forceinline__ void store(E* p, const E (&in)[N]) {
    raw r;
    __builtin_memcpy(&r, in, sizeof(r));
    *reinterpret_cast<raw*>(p) = r;
  }
};

__device__ __forceinline__ float silu_f(float p) { return p * sigmoid_f(p); }

// Bit s set <=> tap s of token t reads a token of t's own sequence,
// i.e. S-1-s <= t - lo(t).  Tokens at or past n_tokens get no taps.
template <int S>
__device__ __forceinline__ uint32_t tap_bits(const SeqLayout& seq, int64_t t) {
  if (t >= seq.n_tokens || t < 0) return 0u;
  int64_t lo, hi;
  seq.bounds(t, lo, hi);
  const int64_t pos = t - lo;
  if (pos >= S - 1) return (1u << S) - 1u;
  // taps s >= S-1-pos are valid
  return ((1u << S) - 1u) & ~((1u << (S - 1 - pos)) - 1u);
}

// ---------------------------------------------------------------------------
// Forward.  Grid: x = channel groups of 4 waves (4 * CW channels), y = token
// ranges of n_sb super-blocks.  No LDS, no barriers.
template <int S, int KC, int NB, int NC, bool ACT, bool BF>
__global__ void __launch_bounds__(256)
fwd_kernel(const void* __restrict__ xv, const typename CT<BF>::elem* __restrict__ a_c,
           const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ yv, SeqLayout seq,
           int64_t D, int n_sb) {
  using C = CT<BF>;
  using E = typename C::elem;
  using Op = typename C::opnd;
  constexpr int R = 4 * NB, TB = 16 * NB, CW = 16 * NC, KP = 16 * KC, W = R + S - 1;
  const E* __restrict__ x = static_cast<const E*>(xv);
  E* __restrict__ y = static_cast<E*>(yv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int64_t N = seq.n_tokens;
  const int64_t d0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * CW;
  if (d0 >= D) return;  // whole wave past the channel axis; no barriers below
  const int64_t dl = d0 + NC * j;
  const bool ch_ok = dl < D;

  // basis B operands: bop[c][s][kc] = basis[16kc + 4q + v, s, dl + c], v = 0..3
  Op bop[NC][S][KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      E rows[4][NC];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * q + v;
        if (ch_ok) {
          Vec<E, NC>::load(b_c + (static_cast<int64_t>(k) * S + s) * D + dl, rows[v]);
        } else {
#pragma unroll
          for (int c = 0; c < NC; ++c) rows[v][c] = E(0);
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) bop[c][s][kc] = C::make(rows[0][c], rows[1][c], rows[2][c], rows[3][c]);
    }
  }

  const int64_t tbase = static_cast<int64_t>(blockIdx.y) * n_sb * TB;
  for (int sb = 0; sb < n_sb; ++sb) {
    const int64_t t0 = tbase + static_cast<int64_t>(sb) * TB;
    if (t0 >= N) break;
    const int64_t trun = t0 + R * q;

    // x window: rows trun-(S-1) .. trun+R-1
    float xw[W][NC];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int64_t t = trun - (S - 1) + w;
      E e[NC];
      if (ch_ok && t >= 0 && t < N) {
        Vec<E, NC>::load(x + t * D + dl, e);
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) e[c] = E(0);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) xw[w][c] = C::to_f(e[c]);
    }
    // alpha A operands: row i = j of block b is token t0 + R*(j/4) + 4b + j%4
    Op aop[NB][KC];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t tok = t0 + R * (j >> 2) + 4 * b + (j & 3);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        aop[b][kc] = (tok < N) ? *reinterpret_cast<const Op*>(a_c + tok * KP + 16 * kc + 4 * q)
                               : C::zero();
    }

    bool interior = true;
    if (trun < N) {
      int64_t lo, hi;
      seq.bounds(trun, lo, hi);
      const int64_t last = (trun + R < N ? trun + R : N);
      interior = (trun - lo >= S - 1) && (last <= hi);
    }

    auto body = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      uint32_t ok[R];
#pragma unroll
      for (int r = 0; r < R; ++r) ok[r] = MASK ? tap_bits<S>(seq, trun + r) : ((1u << S) - 1u);
      float acc[R][NC];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        f32x4 w[NB][NC];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) t = C::mma(aop[b][kc], bop[c][s][kc], t);
            w[b][c] = t;
          }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * b + v;
            if (!MASK || ((ok[r] >> s) & 1u)) {
#pragma unroll
              for (int c = 0; c < NC; ++c) acc[r][c] = fmaf(xw[r + s][c], w[b][c][v], acc[r][c]);
            }
          }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t t = trun + r;
        if (ch_ok && t < N) {
          E o[NC];
#pragma unroll
          for (int c = 0; c < NC; ++c) o[c] = C::from_f(ACT ? silu_f(acc[r][c]) : acc[r][c]);
          Vec<E, NC>::store(y + t * D + dl, o);
        }
      }
    };
    if (__all(interior)) body(std::false_type{});
    else body(std::true_type{});
  }
}

// ---------------------------------------------------------------------------
// Backward, stage 1.  A workgroup of WPG waves covers WPG * CW channels and a
// range of n_sb super-blocks; all its waves walk the same super-blocks.
// Super-block i covers rows [t0, t0 + TB) with t0 = i * EOWN, EOWN = TB - (S-1):
// its first EOWN rows are its own, the last S-1 rows only provide the future
// g / W the own rows' dx needs (they are recomputed as own rows of block i+1).
// Per super-block and lane:
//   P (SiLU only) from MFMA W and the register window; g = dy * silu'(P);
//   dx[u] = sum_s g[u+S-1-s] W_s[u+S-1-s]: W at the later token comes from an
//     MFMA on alpha rows shifted by S-1-s, g of the next lane group's first
//     S-1 rows by a cross-lane read;
//   m_s = g * x_shift_s  ->  dbasis MFMA (m^T . alpha, accumulated over the
//     whole range in registers) and, through LDS, dalpha MFMA (m . basis^T);
//   the WPG waves' dalpha tiles are summed in LDS in wave order.
// Outputs: dx (own rows), part_da[blockIdx.x][t][KP], part_db[blockIdx.y][KP][S][D].
template <int S, int KC, int NB, int NC, int WPG, bool ACT, bool BF>
__global__ void __launch_bounds__(64 * WPG)
bwd_kernel(const void* __restrict__ xv, const void* __restrict__ dyv,
           const typename CT<BF>::elem* __restrict__ a_c,
           const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ dxv,
           float* __restrict__ part_da, float* __restrict__ part_db, SeqLayout seq, int64_t D,
           int n_sb) {
  using C = CT<BF>;
  using E = typename C::elem;
  using Op = typename C::opnd;
  constexpr int R = 4 * NB, TB = 16 * NB, CW = 16 * NC, KP = 16 * KC, W = R + S - 1;
  constexpr int EOWN = TB - (S - 1);
  constexpr int MROW = S * CW + 4;  // padded LDS row: 8 / 16-byte aligned operand reads
  static_assert(S >= 2 && EOWN > 0, "super-block too small for the kernel size");

  __shared__ E m_lds[WPG][TB][MROW];
  __shared__ float da_lds[WPG][NB][KC][16][17];

  const E* __restrict__ x = static_cast<const E*>(xv);
  const E* __restrict__ dy = static_cast<const E*>(dyv);
  E* __restrict__ dx = static_cast<E*>(dxv);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int64_t N = seq.n_tokens;
  const int64_t d0 = (static_cast<int64_t>(blockIdx.x) * WPG + wave) * CW;
  const bool wave_on = d0 < D;
  const int64_t dl = d0 + NC * j;
  const bool ch_ok = wave_on && dl < D;

  // W operands: bop[c][s][kc] = basis[16kc + 4q + v, s, dl + c]
  Op bop[NC][S][KC];
  // dalpha B operands: bda[s][cg][kc] = basis[16kc + j, s, d0 + 16cg + 4q + v]
  Op bda[S][NC][KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      E rows[4][NC];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * q + v;
        if (ch_ok) {
          Vec<E, NC>::load(b_c + (static_cast<int64_t>(k) * S + s) * D + dl, rows[v]);
        } else {
#pragma unroll
          for (int c = 0; c < NC; ++c) rows[v][c] = E(0);
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) bop[c][s][kc] = C::make(rows[0][c], rows[1][c], rows[2][c], rows[3][c]);
#pragma unroll
      for (int cg = 0; cg < NC; ++cg) {
        const int64_t ch = d0 + 16 * cg + 4 * q;
        E e4[4];
        if (wave_on && ch < D) {
          Vec<E, 4>::load(b_c + (static_cast<int64_t>(16 * kc + j) * S + s) * D + ch, e4);
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) e4[v] = E(0);
        }
        bda[s][cg][kc] = C::make(e4[0], e4[1], e4[2], e4[3]);
      }
    }
  }

  f32x4 dbacc[NC][S][KC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) dbacc[c][s][kc] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int sb = 0; sb < n_sb; ++sb) {
    const int64_t t0 = (static_cast<int64_t>(blockIdx.y) * n_sb + sb) * EOWN;
    if (t0 >= N) break;  // uniform over the workgroup
    const int64_t own_end = (t0 + EOWN < N) ? t0 + EOWN : N;
    const int64_t trun = t0 + R * q;

    float xw[W][NC];
    float g[R][NC];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int64_t t = trun - (S - 1) + w;
      E e[NC];
      if (ch_ok && t >= 0 && t < N) {
        Vec<E, NC>::load(x + t * D + dl, e);
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) e[c] = E(0);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) xw[w][c] = C::to_f(e[c]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = trun + r;
      E e[NC];
      if (ch_ok && t < N) {
        Vec<E, NC>::load(dy + t * D + dl, e);
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) e[c] = E(0);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) g[r][c] = C::to_f(e[c]);
    }
    // alpha A operands, rows shifted by e = 0..S-1 tokens
    Op aop[S][NB][KC];
#pragma unroll
    for (int e = 0; e < S; ++e)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int64_t tok = t0 + R * (j >> 2) + 4 * b + (j & 3) + e;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
          aop[e][b][kc] = (tok < N) ? *reinterpret_cast<const Op*>(a_c + tok * KP + 16 * kc + 4 * q)
                                    : C::zero();
      }
    // alpha^T B operands of the dbasis MFMA: at[b][kc][v] = alpha[trun + 4b + v, 16kc + j],
    // zero for rows that are not this super-block's own
    Op at[NB][KC];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        E e4[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t tok = trun + 4 * b + v;
          e4[v] = (tok < own_end) ? a_c[tok * KP + 16 * kc + j] : E(0);
        }
        at[b][kc] = C::make(e4[0], e4[1], e4[2], e4[3]);
      }

    bool interior = true;
    if (trun < N) {
      int64_t lo, hi;
      seq.bounds(trun, lo, hi);
      const int64_t last = (trun + W < N ? trun + W : N);
      interior = (trun - lo >= S - 1) && (last <= hi);
    }

    auto body = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      // ok[r]: tap bits of row r of this lane's run extended by S-1 later rows
      uint32_t ok[R + S - 1];
#pragma unroll
      for (int r = 0; r < R + S - 1; ++r) ok[r] = MASK ? tap_bits<S>(seq, trun + r) : ((1u << S) - 1u);

      if (ACT) {
        float p[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) p[r][c] = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              f32x4 w4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kc = 0; kc < KC; ++kc) w4 = C::mma(aop[0][b][kc], bop[c][s][kc], w4);
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int r = 4 * b + v;
                if (!MASK || ((ok[r] >> s) & 1u)) p[r][c] = fmaf(xw[r + s][c], w4[v], p[r][c]);
              }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const float pv = p[r][c];
            const float sg = sigmoid_f(pv);
            g[r][c] = g[r][c] * (sg * (1.0f + pv * (1.0f - sg)));
          }
      }

      // g of the S-1 rows after this lane's run: first rows of lane group q+1
      float gf[S - 1][NC];
      const int src_lane = (lane + 16) & 63;
#pragma unroll
      for (int e = 0; e < S - 1; ++e)
#pragma unroll
        for (int c = 0; c < NC; ++c) gf[e][c] = __shfl(g[e][c], src_lane, 64);

      // dx: taps in ascending order
      if (dx != nullptr) {
        float dxa[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) dxa[r][c] = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int off = S - 1 - s;
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
              f32x4 w4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kc = 0; kc < KC; ++kc) w4 = C::mma(aop[off][b][kc], bop[c][s][kc], w4);
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int r = 4 * b + v;
                const int src = r + off;
                const float gs = (src < R) ? g[src < R ? src : 0][c] : gf[src >= R ? src - R : 0][c];
                if (!MASK || ((ok[src] >> s) & 1u)) dxa[r][c] = fmaf(gs, w4[v], dxa[r][c]);
              }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int64_t t = trun + r;
          if (ch_ok && t < own_end) {
            E o[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) o[c] = C::from_f(dxa[r][c]);
            Vec<E, NC>::store(dx + t * D + dl, o);
          }
        }
      }

      // m_s = g * x[t-(S-1-s)]: dbasis MFMA and the LDS copy for dalpha
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          E mv[4][NC];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * b + v;
            const bool on = !MASK || ((ok[r] >> s) & 1u);
#pragma unroll
            for (int c = 0; c < NC; ++c) mv[v][c] = C::from_f(on ? g[r][c] * xw[r + s][c] : 0.f);
            Vec<E, NC>::store(&m_lds[wave][R * q + r][s * CW + NC * j], mv[v]);
          }
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const Op am = C::make(mv[0][c], mv[1][c], mv[2][c], mv[3][c]);
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) dbacc[c][s][kc] = C::mma(am, at[b][kc], dbacc[c][s][kc]);
          }
        }
      }
    };
    if (__all(interior)) body(std::false_type{});
    else body(std::true_type{});

    __syncthreads();
    // dalpha over this wave's channels: D[t][k] = sum_(s,ch) m[t][(s,ch)] basis[k][(s,ch)]
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int cg = 0; cg < NC; ++cg) {
            const Op am = *reinterpret_cast<const Op*>(&m_lds[wave][16 * rb + j][s * CW + 16 * cg + 4 * q]);
            acc = C::mma(am, bda[s][cg][kc], acc);
          }
#pragma unroll
        for (int v = 0; v < 4; ++v) da_lds[wave][rb][kc][4 * q + v][j] = acc[v];
      }
    __syncthreads();
    // sum the WPG waves' tiles in wave order; own rows only
    for (int idx = tid; idx < NB * KC * 256; idx += 64 * WPG) {
      const int rb = idx / (KC * 256);
      const int kc = (idx / 256) % KC;
      const int row = (idx >> 4) & 15, col = idx & 15;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) sum += da_lds[w][rb][kc][row][col];
      const int64_t t = t0 + 16 * rb + row;
      if (t < own_end) part_da[(static_cast<int64_t>(blockIdx.x) * N + t) * KP + 16 * kc + col] = sum;
    }
  }

  // this workgroup's dbasis partial: dbacc[c][s][kc][v] is
  // (k = 16kc + j, s, channel d0 + NC (4q + v) + c)
  if (wave_on) {
    const int64_t base = static_cast<int64_t>(blockIdx.y) * KP;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int64_t ch = d0 + NC * (4 * q + v) + c;
            if (ch < D)
              part_db[((base + 16 * kc + j) * S + s) * D + ch] = dbacc[c][s][kc][v];
          }
  }
}

}  // namespace mfma
}  // namespace moc
