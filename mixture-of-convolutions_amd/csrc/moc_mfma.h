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
  // two route chunks in one v_mfma_f32_16x16x32_bf16: lane entries a0 ++ a1
  // against b0 ++ b1 (A and B list their entries in the same order)
  static __device__ __forceinline__ f32x4 mma2(opnd a0, opnd a1, opnd b0, opnd b1, f32x4 c) {
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
    const s16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
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

// Raw buffer resource over a byte range [base, base + bytes) (< 2 GiB).  Loads at
// offsets outside the range return zeros and stores there are dropped by the
// hardware, so rows before a sequence's first token, past the token axis or
// past the channel axis need no branches: they get an out-of-range offset.
constexpr uint32_t kOffNone = 0x80000000u;  // an offset no range here reaches

// Values of the kernels' ACT parameter: 0 (no activation), 1 (SiLU), or
// kActRuntime: the layers of a grouped launch each name theirs in the layer
// table (a uniform branch; the SiLU code is built in).
constexpr int kActRuntime = 2;

struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Buf(const void* base, int64_t bytes) {
    r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                          static_cast<int>(bytes > 0 ? bytes : 0), 0x00020000);
  }
  template <int BYTES>
  __device__ __forceinline__ void load(uint32_t off, void* dst) const {
    if constexpr (BYTES == 2) {
      const uint16_t v = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0);
      __builtin_memcpy(dst, &v, 2);
    } else if constexpr (BYTES == 4) {
      const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
      __builtin_memcpy(dst, &v, 4);
    } else if constexpr (BYTES == 8) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
      __builtin_memcpy(dst, &v, 8);
    } else {
      static_assert(BYTES == 16, "buffer load width");
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
      __builtin_memcpy(dst, &v, 16);
    }
  }
  template <int BYTES>
  __device__ __forceinline__ void store(uint32_t off, const void* src) const {
    if constexpr (BYTES == 2) {
      uint16_t v;
      __builtin_memcpy(&v, src, 2);
      __builtin_amdgcn_raw_buffer_store_b16(v, r, static_cast<int>(off), 0, 0);
    } else if constexpr (BYTES == 4) {
      uint32_t v;
      __builtin_memcpy(&v, src, 4);
      __builtin_amdgcn_raw_buffer_store_b32(v, r, static_cast<int>(off), 0, 0);
    } else if constexpr (BYTES == 8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      u32x2 v;
      __builtin_memcpy(&v, src, 8);
      __builtin_amdgcn_raw_buffer_store_b64(v, r, static_cast<int>(off), 0, 0);
    } else {
      static_assert(BYTES == 16, "buffer store width");
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      u32x4 v;
      __builtin_memcpy(&v, src, 16);
      __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(off), 0, 0);
    }
  }
};

// Byte offset of (row t, byte column col) relative to row `lo` of a row-major
// buffer, or kOffNone when `on` is false.  Negative rows give offsets >= 2^31.
__device__ __forceinline__ uint32_t row_off(int64_t t, int64_t lo, uint32_t row_bytes,
                                            uint32_t col, bool on = true) {
  const uint32_t o = static_cast<uint32_t>(static_cast<int32_t>(t - lo)) * row_bytes + col;
  return on ? o : kOffNone;
}

__device__ __forceinline__ float silu_f(float p) { return p * sigmoid_f(p); }

// Two fp32 rounded to bf16 (nearest even) in one dword, a in the low half: one
// v_cvt_pk_bf16_f32 (two scalar conversions compile to two conversions, a
// shift and an OR).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Sequence starts near a super-block.  A tap s of token t is valid when its
// source t-(S-1-s) is not before t's segment start.  All starts that can
// invalidate a tap of the rows [r0, r1] lie in [r0 - (S-2), r1]; `starts_in`
// tells (wave-uniformly) whether there is one, and `tap_bits_rows` gives the
// valid-tap bits of rows row0 + r (r < NROWS) by walking those starts.
__device__ __forceinline__ bool starts_in(const SeqLayout& seq, int64_t lo, int64_t hi) {
  return seq.next_start(lo) <= hi;
}

// starts_in for windows that move forward: `ns` caches the smallest segment
// start >= the previous window's lo and is searched again only once the
// window has passed it (about once per sequence), not for every super-block.
struct StartCursor {
  int64_t ns = -1;
  __device__ __forceinline__ bool starts_in(const SeqLayout& seq, int64_t lo, int64_t hi) {
    if (ns < lo) ns = seq.next_start(lo);
    return ns <= hi;
  }
};

template <int S, int NROWS>
__device__ __forceinline__ void tap_bits_rows(const SeqLayout& seq, int64_t row0, int64_t w_lo,
                                              int64_t w_hi, uint32_t (&ok)[NROWS]) {
  int64_t last[NROWS];
#pragma unroll
  for (int r = 0; r < NROWS; ++r) last[r] = INT64_MIN / 2;
  for (int64_t b = seq.next_start(w_lo); b <= w_hi && b < seq.n_tokens; b = seq.next_start(b + 1)) {
#pragma unroll
    for (int r = 0; r < NROWS; ++r)
      if (b <= row0 + r) last[r] = b;
  }
#pragma unroll
  for (int r = 0; r < NROWS; ++r) {
    const int64_t t = row0 + r;
    const int64_t pos = t - last[r];
    uint32_t bits = (1u << S) - 1u;
    if (pos < S - 1) bits &= ~((1u << (S - 1 - pos)) - 1u);  // taps s >= S-1-pos
    ok[r] = (t < seq.n_tokens && t >= 0) ? bits : 0u;
  }
}

// ---------------------------------------------------------------------------
// Prefill from a cache (moc/api.py:299-309, 218-227): fixed-length sequences of
// T = seq.seq_len tokens, T >= S-1, each continuing the S inputs its cache
// holds.  The reference prepends the cache to x with zero routing and drops
// those outputs; here the taps that reach before a sequence's first token read
// the cache where the plain kernels read nothing:
//   hist [n_seqs, D, S] (contiguous, slot S-1 the newest input), or null for a
//     zero history; tap s of the sequence's token pos < S-1-s reads slot
//     s + 1 + pos;
//   fin [n_seqs, D, S] (or null) receives each sequence's last S inputs (the
//     state a later call continues from), slot S-1 the last token; with T < S
//     its oldest S-T slots are the cache's newest ones (zeros without a cache).
//   g (backward, two passes with the activation): fp32 [N, D] g = dy silu'(P),
//     written by the dx pass (whose P reads the cache), read by the taps pass.
struct Pre {
  const void* hist;
  void* fin;
  float* g = nullptr;
};

// History value of window rows u0 + w (w < NW) for this lane's channels: with
// T >= S-1 the taps that reach row u from a later sequence all belong to the
// first sequence starting after u (at st, u >= st - (S-1)), and read its cache
// slot S - (st - u).  Rows that no masked tap reads get zero.
template <int S, int NW, int NC, typename E>
__device__ __forceinline__ void hist_window(const Buf& hb, int64_t u0, int64_t T, int64_t N,
                                            int64_t D, int64_t dl, bool ch_ok,
                                            float (&hx)[NW][NC]) {
  // sequence b starting at st = b T: the first start after u0 (token indices
  // stay below 2^31)
  int64_t b = 0;
  if (u0 >= 0) b = static_cast<int64_t>(static_cast<uint32_t>(u0) / static_cast<uint32_t>(T)) + 1;
  int64_t st = b * T;
  constexpr uint32_t ESZ = sizeof(E);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int64_t u = u0 + w;
    const int64_t m = st - u;  // >= 1
    const bool on = ch_ok && m <= S - 1 && st < N;
    const uint32_t off = static_cast<uint32_t>(((b * D + dl) * S + (S - m)) * ESZ);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      E v;
      hb.load<ESZ>(on ? off + c * S * ESZ : kOffNone, &v);
      if constexpr (sizeof(E) == 2) hx[w][c] = bf16_to_f32(v);
      else hx[w][c] = v;
    }
    if (u + 1 == st) {
      st += T;
      ++b;
    }
  }
}

// One value of hist_window: the cache entry standing for token u of channel
// dl + c (the tap of the first sequence starting after u), or 0.
template <int S, typename E>
__device__ __forceinline__ float hist_at(const Buf& hb, int64_t u, int64_t T, int64_t N, int64_t D,
                                         int64_t dl, bool ch_ok, int c) {
  int64_t b = 0;
  if (u >= 0) b = static_cast<int64_t>(static_cast<uint32_t>(u) / static_cast<uint32_t>(T)) + 1;
  const int64_t st = b * T;
  const int64_t m = st - u;  // >= 1
  const bool on = ch_ok && m <= S - 1 && st < N;
  constexpr uint32_t ESZ = sizeof(E);
  const uint32_t off = static_cast<uint32_t>(((b * D + dl) * S + (S - m) + c * S) * ESZ);
  E v;
  hb.load<ESZ>(on ? off : kOffNone, &v);
  if constexpr (sizeof(E) == 2) return bf16_to_f32(v);
  else return v;
}

// Final-state rows of a super-block [t0, t0 + TB): this lane's run trun + r
// (r < R) with x values xw[r + S - 1]; writes fin for the rows within S of
// their sequence's end, and the cache part of the state for T < S.
template <int S, int R, int NC, typename E>
__device__ __forceinline__ void fin_rows(const Pre& pre, const Buf& hb, int64_t trun, int64_t T,
                                         int64_t N, int64_t D, int64_t dl, bool ch_ok,
                                         const float (&xw)[R + S - 1][NC]) {
  constexpr uint32_t ESZ = sizeof(E);
  const Buf fb(pre.fin, N / T * D * S * ESZ);
  // sequence b and position pos of row trun (token indices stay below 2^31)
  int64_t b = static_cast<int64_t>(static_cast<uint32_t>(trun) / static_cast<uint32_t>(T));
  int64_t pos = trun - b * T;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = trun + r;
    const bool live = ch_ok && t < N;
    const int64_t slot = S - (T - pos);
    const uint32_t base = static_cast<uint32_t>((b * D + dl) * S * ESZ);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      E v;
      if constexpr (sizeof(E) == 2) v = f32_to_bf16(xw[r + S - 1][c]);
      else v = xw[r + S - 1][c];
      fb.store<ESZ>(live && slot >= 0 ? base + static_cast<uint32_t>((c * S + slot) * ESZ) : kOffNone, &v);
    }
    if (T < S && pos == 0) {
      // the oldest S - T slots: the cache's slots T.. (zero without a cache)
      for (int jj = 0; jj < S - T; ++jj)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          E v;
          hb.load<ESZ>(live && pre.hist ? base + static_cast<uint32_t>((c * S + jj + T) * ESZ) : kOffNone, &v);
          fb.store<ESZ>(live ? base + static_cast<uint32_t>((c * S + jj) * ESZ) : kOffNone, &v);
        }
    }
    if (++pos == T) {
      pos = 0;
      ++b;
    }
  }
}

// ---------------------------------------------------------------------------
// Layer tables of a grouped launch.  The MoC layers of one launch share the
// token axis (sequence layout), K, S, activation and compute dtype; each has its
// own tensors, channel count and the grid its own launch would use, and the
// launch is the concatenation of those grids: layer i owns the 1-D block ids
// [blk0, blk0 + its block count), mapped onto its grid as its own launch maps
// them (x fastest).  So each workgroup does exactly the work it does in the
// layer's own launch, and results equal those launches bit for bit.  A
// workgroup finds its layer with uniform selects (the table stays in scalar
// registers).
constexpr int kMaxLayers = 4;

struct FwdLayer {
  const void* x;
  const void* a;   // routing operands [n_tokens, KP] in the compute dtype
  const void* b;   // basis operands [KP, S, D] in the compute dtype
  void* y;
  int64_t D;
  int gx, n_sb, blk0;
  int act;         // this layer's activation (read where the kernel's ACT is kActRuntime)
  int kc;          // this layer's route chunks (1, 2 or 4)
};
struct FwdLayers {
  int n;
  FwdLayer l[kMaxLayers];
};

struct BwdLayer {
  const void* x;
  const void* dy;
  int64_t dys;     // dy row stride (elements): D, 0 for one broadcast row, -1 for one element
  const void* a;
  const void* b;
  void* dx;
  float* part_da;  // [gx, n_tokens, KP]
  float* part_db;  // [gy, KP, S, D]
  int64_t D;
  int gx, gy, gy1, n_old, n_total, blk0;
  int act;         // this layer's activation (read where the kernel's ACT is kActRuntime)
  float* gbuf;     // the two passes with the activation: g = dy silu'(P), fp32 [N, D]
};
struct BwdLayers {
  int n;
  BwdLayer l[kMaxLayers];
};

// Index of the layer owning 1-D block id blk of a grouped launch (uniform; the
// kernels then read that layer's fields from the kernel-argument table, where
// the compiler can reload them instead of keeping copies live).
template <typename LT>
__device__ __forceinline__ int layer_index(const LT& ly, int blk) {
  int li = 0;
#pragma unroll
  for (int i = 1; i < kMaxLayers; ++i)
    if (i < ly.n && blk >= ly.l[i].blk0) li = i;
  return __builtin_amdgcn_readfirstlane(li);
}

// ---------------------------------------------------------------------------
// Forward.  Grid: x = channel groups of 4 waves (4 * CW channels), y = token
// ranges of n_sb super-blocks.  No LDS, no barriers: every wave walks its
// super-blocks on its own, loading the rows of super-block i+1 (x window and
// routing weights, raw) before it computes super-block i.  fwd_tile is the
// work of workgroup (bx, by) of one layer.  PRE: prefill from a cache (Pre;
// fixed-length sequences).
template <int S, int KC, int NB, int NC, int ACT, bool BF, bool PRE = false>
__device__ __forceinline__ void fwd_tile(const void* __restrict__ xv,
                                         const typename CT<BF>::elem* __restrict__ a_c,
                                         const typename CT<BF>::elem* __restrict__ b_c,
                                         void* __restrict__ yv, SeqLayout seq, int64_t D, int n_sb,
                                         int bx, int by, Pre pre = Pre{nullptr, nullptr},
                                         bool act_rt = false) {
  using C = CT<BF>;
  const bool act = ACT == kActRuntime ? act_rt : ACT != 0;  // (uniform)
  using E = typename C::elem;
  using Op = typename C::opnd;
  constexpr int R = 4 * NB, TB = 16 * NB, CW = 16 * NC, KP = 16 * KC, W = R + S - 1;
  const E* __restrict__ x = static_cast<const E*>(xv);
  E* __restrict__ y = static_cast<E*>(yv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int64_t N = seq.n_tokens;
  const int64_t d0 = (static_cast<int64_t>(bx) * 4 + wave) * CW;
  if (d0 >= D) return;  // whole wave past the channel axis; no barriers below
  const int64_t dl = d0 + NC * j;
  const bool ch_ok = dl < D;

  constexpr int ESZ = static_cast<int>(sizeof(E));
  const int64_t tbase = static_cast<int64_t>(by) * n_sb * TB;
  // buffers over the rows this wave touches: x / y rows [row_lo, row_hi), alpha rows [tbase, row_hi)
  const int64_t row_lo = (tbase - (S - 1) > 0) ? tbase - (S - 1) : 0;
  const int64_t row_hi = (tbase + static_cast<int64_t>(n_sb) * TB < N) ? tbase + static_cast<int64_t>(n_sb) * TB : N;
  const uint32_t rb = static_cast<uint32_t>(D * ESZ);
  const uint32_t col = static_cast<uint32_t>(dl * ESZ);
  const Buf xb(x + row_lo * D, (row_hi - row_lo) * D * ESZ);
  const Buf yb(y + row_lo * D, (row_hi - row_lo) * D * ESZ);
  const Buf ab(a_c + tbase * KP, (row_hi - tbase) * KP * ESZ);
  const Buf bb(b_c, static_cast<int64_t>(KP) * S * D * ESZ);
  // PRE: the cache (n_seqs = N / T sequences)
  const int64_t T = seq.seq_len;
  const Buf hb(PRE ? pre.hist : nullptr, PRE && pre.hist ? N / T * D * S * ESZ : 0);

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
        bb.load<NC * ESZ>(row_off(k * S + s, 0, rb, col, ch_ok), rows[v]);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) bop[c][s][kc] = C::make(rows[0][c], rows[1][c], rows[2][c], rows[3][c]);
    }
  }

  // raw rows of one super-block: x window (trun-(S-1) .. trun+R-1) and the
  // alpha A operands (row i = j of block b is token t0 + R*(j/4) + 4b + j%4)
  E xr[W][NC];
  Op ar[NB][KC];
  // Window row w sits at base + w rb: rows before row_lo wrap to offsets
  // >= 2^31 and load zeros, and a lane past the channel axis starts at
  // kOffNone (row_off); the alpha rows of block b and route chunk kc sit a
  // constant (immediate) offset from the lane's first one.
  auto fetch = [&](int64_t t0) {
    const int64_t trun = t0 + R * q;
    const uint32_t base = row_off(trun - (S - 1), row_lo, rb, col, ch_ok);
#pragma unroll
    for (int w = 0; w < W; ++w) xb.load<NC * ESZ>(base + w * rb, xr[w]);
    const uint32_t abase = row_off(t0 + R * (j >> 2) + (j & 3), tbase, KP * ESZ, 4 * q * ESZ);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        ab.load<4 * ESZ>(abase + static_cast<uint32_t>((4 * b * KP + 16 * kc) * ESZ), &ar[b][kc]);
    }
  };

  if (tbase < N) fetch(tbase);
  StartCursor cursor;
  for (int sb = 0; sb < n_sb; ++sb) {
    const int64_t t0 = tbase + static_cast<int64_t>(sb) * TB;
    if (t0 >= N) break;
    const int64_t trun = t0 + R * q;

    float xw[W][NC];
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        xw[w][c] = C::to_f(xr[w][c]);
        asm volatile("" : "+v"(xw[w][c]));  // converted here, not sunk below the loads
      }
    Op aop[NB][KC];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) aop[b][kc] = ar[b][kc];
    // issue the next super-block's loads before computing this one; after the
    // last super-block they fall past the buffers and load zeros.  Issued
    // unconditionally and after the conversions above, they land in the
    // registers the rows just left, and the loop carries them without copies.
    __builtin_amdgcn_sched_barrier(0);
    fetch(t0 + TB);

    // uniform over the wave: does a sequence start fall where it masks a tap?
    const int64_t w_lo = t0 - (S - 2), w_hi = t0 + TB - 1;
    const bool interior = !cursor.starts_in(seq, w_lo, w_hi);

    auto body = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      uint32_t ok[R];
      if (MASK) {
        tap_bits_rows<S, R>(seq, trun, w_lo, w_hi, ok);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) ok[r] = (1u << S) - 1u;
      }
      // PRE: masked taps read the cache (uniform: is there one?)
      float hx[PRE && MASK ? W : 1][NC];
      bool use_h = false;
      if constexpr (PRE && MASK) {
        use_h = pre.hist != nullptr;
        if (use_h) hist_window<S, W, NC, E>(hb, trun - (S - 1), T, N, D, dl, ch_ok, hx);
      }
      float acc[R][NC];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            f32x4 w = {0.f, 0.f, 0.f, 0.f};
            if constexpr (BF && KC % 2 == 0) {
#pragma unroll
              for (int kp = 0; kp < KC; kp += 2)
                w = C::mma2(aop[b][kp], aop[b][kp + 1], bop[c][s][kp], bop[c][s][kp + 1], w);
            } else {
#pragma unroll
              for (int kc = 0; kc < KC; ++kc) w = C::mma(aop[b][kc], bop[c][s][kc], w);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int r = 4 * b + v;
              if (!MASK || ((ok[r] >> s) & 1u)) acc[r][c] = fmaf(xw[r + s][c], w[v], acc[r][c]);
              else if (PRE && MASK && use_h) acc[r][c] = fmaf(hx[PRE && MASK ? r + s : 0][c], w[v], acc[r][c]);
            }
          }
      }
      const uint32_t ybase = row_off(trun, row_lo, rb, col, ch_ok);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        E o[NC];
        if constexpr (BF && NC == 2) {
          const uint32_t pk = act ? pack2_bf16(silu_f(acc[r][0]), silu_f(acc[r][1]))
                                  : pack2_bf16(acc[r][0], acc[r][1]);
          __builtin_memcpy(o, &pk, 4);
        } else {
#pragma unroll
          for (int c = 0; c < NC; ++c) o[c] = C::from_f(act ? silu_f(acc[r][c]) : acc[r][c]);
        }
        yb.store<NC * ESZ>(ybase + r * rb, o);
      }
    };
    if (interior) body(std::false_type{});
    else body(std::true_type{});
    if constexpr (PRE) {
      // final state: does a sequence end within S rows after this super-block's rows?
      if (pre.fin != nullptr) {
        const int64_t e1 = (t0 / T + 1) * T;  // first sequence end after t0 (uniform)
        if (e1 - S <= t0 + TB - 1) fin_rows<S, R, NC, E>(pre, hb, trun, T, N, D, dl, ch_ok, xw);
      }
    }
  }
}

// Waves per SIMD the 8-tap, 32-route forward is built for (1: the compiler's
// choice, 169 VGPRs, two waves).
#ifndef MOC_FWD8_WAVES
#define MOC_FWD8_WAVES 1
#endif
template <int S, int KC, int NB, int NC, bool ACT, bool BF>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((S == 8 && KC == 2) ? MOC_FWD8_WAVES : 1)))
fwd_kernel(const void* __restrict__ xv, const typename CT<BF>::elem* __restrict__ a_c,
           const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ yv, SeqLayout seq,
           int64_t D, int n_sb) {
  fwd_tile<S, KC, NB, NC, ACT, BF>(xv, a_c, b_c, yv, seq, D, n_sb, static_cast<int>(blockIdx.x),
                                   static_cast<int>(blockIdx.y));
}

// Prefill from a cache (Pre), same grid as fwd_kernel.
template <int S, int KC, int NB, int NC, bool ACT, bool BF>
__global__ void __launch_bounds__(256)
fwd_pre_kernel(const void* __restrict__ xv, const typename CT<BF>::elem* __restrict__ a_c,
               const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ yv, SeqLayout seq,
               int64_t D, int n_sb, Pre pre) {
  fwd_tile<S, KC, NB, NC, ACT, BF, true>(xv, a_c, b_c, yv, seq, D, n_sb, static_cast<int>(blockIdx.x),
                                         static_cast<int>(blockIdx.y), pre);
}

// Several layers in one launch (1-D grid, the layers' grids one after another).
// KCM: the route-chunk counts present (bits 1, 2, 4); with more than one, each
// layer runs the tile of its own count (a uniform branch), so that a layer's y
// is that of its single launch.
template <int S, int KCM, int NB, int NC, int ACT, bool BF>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((S == 8 && KCM == 2) ? MOC_FWD8_WAVES : 1)))
fwd_layers_kernel(FwdLayers ly, SeqLayout seq) {
  using E = typename CT<BF>::elem;
  const int blk = static_cast<int>(blockIdx.x);
  const FwdLayer* Lp = &ly.l[layer_index(ly, blk)];
  int local = blk - Lp->blk0, row = 0;
  const int gxl = Lp->gx;
  while (local >= gxl) {  // scalar: local < gx gy, at most gy - 1 steps
    local -= gxl;
    ++row;
  }
  auto run = [&](auto kc) {
    fwd_tile<S, decltype(kc)::value, NB, NC, ACT, BF>(Lp->x, static_cast<const E*>(Lp->a),
                                                      static_cast<const E*>(Lp->b), Lp->y, seq, Lp->D,
                                                      Lp->n_sb, local, row, Pre{nullptr, nullptr},
                                                      Lp->act != 0);
  };
  if constexpr (KCM == 1 || KCM == 2 || KCM == 4) {
    run(std::integral_constant<int, KCM>{});
  } else {
    const int kc = __builtin_amdgcn_readfirstlane(Lp->kc);
    if constexpr ((KCM & 1) != 0) {
      if (kc == 1) {
        run(std::integral_constant<int, 1>{});
        return;
      }
    }
    if constexpr ((KCM & 2) != 0) {
      if (kc == 2 || (KCM & 4) == 0) {
        run(std::integral_constant<int, 2>{});
        return;
      }
    }
    if constexpr ((KCM & 4) != 0) run(std::integral_constant<int, 4>{});
  }
}

// ---------------------------------------------------------------------------
// m = g * x as an MFMA operand.  With bf16 operands m is split into a bf16 high
// part (its upper 16 bits) and a bf16 low part (round(m - high)), so that the
// products of the dalpha / dbasis MFMAs keep about 16 significant bits of m
// instead of 8: dbasis sums m over all tokens, and when g is close to constant
// (loss = y.sum(), small kernels) the part of m that varies with g is below
// bf16 resolution.  With fp32 operands m is used as is.
template <bool BF>
struct MSplit;

template <>
struct MSplit<true> {
  static constexpr int kParts = 2;
  static __device__ __forceinline__ void split(float m, uint16_t (&e)[2]) {
    const uint32_t u = __float_as_uint(m);
    e[0] = static_cast<uint16_t>(u >> 16);
    e[1] = f32_to_bf16(m - __uint_as_float(u & 0xffff0000u));
  }
};

template <>
struct MSplit<false> {
  static constexpr int kParts = 1;
  static __device__ __forceinline__ void split(float m, float (&e)[1]) { e[0] = m; }
};

// Four bf16 in MFMA operand order from the upper halves of four fp32 bit patterns
// (v_perm_b32 picks bytes 2-3 of each source).
__device__ __forceinline__ s16x4 pack4_hi(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 w = {__builtin_amdgcn_perm(b, a, 0x07060302u), __builtin_amdgcn_perm(d, c, 0x07060302u)};
  return __builtin_bit_cast(s16x4, w);
}

// Four fp32 rounded to bf16 (nearest even) in MFMA operand order.
__device__ __forceinline__ s16x4 pack4_bf16(float a, float b, float c, float d) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 w = {pack2_bf16(a, b), pack2_bf16(c, d)};
  return __builtin_bit_cast(s16x4, w);
}

// v_mfma_f32_16x16x32_bf16 on operand pairs: lane entries a0 ++ a1 against
// b0 ++ b1, i.e. two 16x16x16 products over disjoint halves of the contraction.
__device__ __forceinline__ f32x4 mma32(s16x4 a0, s16x4 a1, s16x4 b0, s16x4 b1, f32x4 c) {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
  const s16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Transposable LDS tile of one wave's m values for the dalpha MFMA (bf16).
//
// The writer lane (j, q) holds, per token block b and channel c, the 4 values of
// channel NC j + c at the super-block tokens 4 g + {0..3}, g = NB q + b: the
// dbasis operand, stored as one 8-byte slot.  The dalpha A operand wants, in
// lane i + 16 q', the 4 channels 16 cg + 4 q' + {0..3} of token 16 rb + i.
// ds_read_b64_tr_b16 returns, in lane i of each 16-lane group, element i % 4 of
// the slots read by lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4 of the group,
// so reader lane 4 e + a of group q' reads the slot of channel 16 cg + 4 q' + e,
// token group 4 rb + a.
// Slot (channel NC jj + c, token group g) lives at (c GB + g) * 16 +
// (jj ^ (2 c + 4 (g & 3))): 16 slots (128 bytes) per (c, g), and the 16 lanes
// of a writer group (16 channels) or of a reader group (4 channels x 4 token
// groups) touch 16 distinct slots modulo 16.
template <int NB, int NC>
struct TrTile {
  static_assert(NC == 2, "slot layout written for two channels per lane");
  static constexpr int GB = 4 * NB;          // token groups of 4 per super-block
  static constexpr int kSlots = NC * GB * 16;
  static __device__ __forceinline__ int wslot(int j, int q, int b, int c) {
    const int g = NB * q + b;
    return (c * GB + g) * 16 + (j ^ (2 * c + 4 * (g & 3)));
  }
  static __device__ __forceinline__ int rslot(int i, int q, int rb, int cg) {
    const int e = i >> 2, a = i & 3, c = e & 1;
    return (c * GB + a) * 16 + ((8 * cg + 2 * q + (e >> 1)) ^ (2 * c + 4 * a)) + 64 * rb;
  }
  template <typename T>
  static __device__ __forceinline__ s16x4 read(const T* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(const_cast<T*>(p)));
  }
};

// MFMA jobs issued ahead of the FMAs that consume them.
#ifndef MOC_BWD_LEAD
#define MOC_BWD_LEAD 2
#endif
constexpr int kLead = MOC_BWD_LEAD;

// Wave-local ordering of LDS traffic: LDS operations of one wave complete in
// issue order; this keeps the compiler from moving them across the point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Backward, stage 1.  A workgroup of WPG waves covers WPG * CW channels and a
// range of super-blocks (ranges by < gy1 share n_old of them, the later ones
// the rest: the launch may give the workgroups dispatched first longer ranges,
// as the SIMD favours their waves); all its waves walk the same super-blocks, one
// workgroup barrier per super-block.  Super-block i covers rows [t0, t0 + TB)
// with t0 = i * EOWN, EOWN = TB - (S-1): its first EOWN rows are its own, the
// last S-1 rows only provide the later g / W the own rows' dx needs (they are
// recomputed as own rows of block i+1).  The taps pass forms no dx: an m
// product needs dy (or g) of its own row and earlier x rows only, so there
// EOWN = TB and every row of a super-block is its own.  Per super-block and lane:
//   P (SiLU only) from MFMA W and the register window; g = dy * silu'(P);
//   dx[u] = sum_s g[u+S-1-s] W_s[u+S-1-s]: W at the later token from an MFMA on
//     alpha rows shifted by S-1-s, g of the next lane group's first S-1 rows by
//     a cross-lane read;
//   per tap s: m_s = g * x_shift_s -> dbasis MFMA (m^T . alpha, accumulated over
//     the whole range in registers) and, through a wave-private LDS tile, the
//     dalpha MFMA (m . basis^T) accumulated over taps;
//   the WPG waves' dalpha tiles are summed in LDS in wave order after the barrier.
// Routing weights of the super-block (TB + S - 1 rows) are staged in LDS,
// double buffered; x / dy rows of the next super-block are loaded before the
// current one is computed.
// dy rows are dys elements apart: D, or 0 when one row serves every token (the
// broadcast gradient of a sum), or -1 when one element serves every token and
// channel (the gradient of a sum to a scalar, expanded).
// Outputs: dx (own rows), part_da[bx][t][KP], part_db[by][KP][S][D] for channel
// group bx and token range by.
//
// MODE selects the work: kBwdFused does all of the above; kBwdDx only dx;
// kBwdTaps only the m products (dalpha / dbasis), its waves in two sets over
// the same channels, one per half of the taps.  The two partial modes (no
// activation) keep the working set of 8 taps x 32 routes within two waves per
// SIMD: the fused pass needs the W operands of every tap beside the dbasis
// accumulators.
constexpr int kBwdFused = 0, kBwdDx = 1, kBwdTaps = 2;
// Minimum waves per SIMD the backward is compiled for (register budget 512 / n).
// Two, except for the bf16 fused pass with 8 taps and 32 routes: there the
// working set exceeds 256 registers, and one wave per SIMD (spills to AGPRs
// instead of scratch memory) measured 9% faster than two with scratch spills.
// The fp32 fused pass (fp32 rows: twice the registers per window) spills at
// two waves from 3 taps up; at one wave, B4 T4096 D2048, 16 routes: 4 taps
// 262 -> 215 us, 8 taps 962 -> 447; 32 routes: 4 taps 607 -> 358, 8 taps
// 1790 -> 1039.  32 routes with 6 taps stays at two: LLVM's AGPR-copy rewrite
// crashes on its one-wave form.  16 routes below 4 taps gained nothing.  The
// bf16 pass at 16 routes, 6-7 taps spills 16-48 registers at two waves; one
// wave measured slower there (6 taps 136 -> 150 us, 7 with SiLU 174 -> 196).
#ifndef MOC_BWD_MIN_WAVES
#define MOC_BWD_MIN_WAVES 2
#endif
#ifndef MOC_BWD_TAPS_WAVES
#define MOC_BWD_TAPS_WAVES MOC_BWD_MIN_WAVES
#endif
template <int S, int KC, bool BF>
constexpr bool kBwdOneWaveFused = BF ? ((S >= 8 && KC >= 2) || KC >= 4)
                                     : ((KC == 1 && S >= 4) || (KC == 2 && S != 6));
// The dx pass over four route chunks (64 routes) holds the W operands of all
// four and spills at two waves from 7 taps up, and from 5 with SiLU (up to 141
// registers); at one wave, B4 T4096 D2048, 64 routes, backward entry: 8 taps
// 541 -> 427 us, with SiLU 926 -> 538.  Without SiLU at 6 taps one wave was
// slower (316 -> 333).
// The fp32 dx pass spills at two waves with 32 routes from 5 taps with SiLU
// (40-372 bytes) and from 7 without, with 16 routes at 8 taps with SiLU: one
// wave there (B4 T4096 D2048 with SiLU, 32 routes: 8 taps 982 -> 816 us, 6
// taps 638 -> 595).
template <int S, int KC, bool ACT>
constexpr bool kF32DxSpills = (KC >= 2 && S >= (ACT ? 5 : 7)) || (KC == 1 && ACT && S == 8);
template <int S, int KC, int MODE, bool BF, bool ACT = false>
constexpr int kBwdMinWaves = ((MODE == kBwdFused && kBwdOneWaveFused<S, KC, BF>) ||
                              (MODE == kBwdDx && KC >= 4 && (S >= 7 || (ACT && S >= 5))) ||
                              (MODE == kBwdDx && (KC >= 2 || !BF) && S > 8) ||
                              (MODE == kBwdDx && !BF && kF32DxSpills<S, KC, ACT>))
                                 ? 1
                                 : (MODE == kBwdTaps ? MOC_BWD_TAPS_WAVES : MOC_BWD_MIN_WAVES);

// bwd_tile is the work of workgroup (bx, by) (route chunk zh with SPLIT) of
// one layer; the __global__ wrappers below map the grid onto it.  PRE (fused
// pass only): prefill from a cache, whose values the masked taps read in P and
// in the m products (the cache gradient is not formed here).  gbuf (the partial
// passes with the activation): g = dy silu'(P) of every token and channel in
// fp32 [N, D], written by the dx pass, read by the taps pass in place of dy.
template <int S, int KC, int NB, int NC, int WPG, int ACT, bool BF, bool SPLIT, int MODE,
          bool PRE = false>
__device__ __forceinline__ void
bwd_tile(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
         const typename CT<BF>::elem* __restrict__ a_c,
         const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ dxv,
         float* __restrict__ part_da, float* __restrict__ part_db, SeqLayout seq, int64_t D,
         int bx, int by, int zh, int gy, int gy1, int n_old, int n_total,
         Pre pre = Pre{nullptr, nullptr}, float* __restrict__ gbuf = nullptr, bool act_rt = false) {
  using C = CT<BF>;
  using E = typename C::elem;
  using Op = typename C::opnd;
  using XV = Vec<E, NC>;
  using MS = MSplit<BF>;
  constexpr int R = 4 * NB, TB = 16 * NB, CW = 16 * NC, KP = 16 * KC, W = R + S - 1;
  // route chunks of dbasis / dalpha this workgroup accumulates: all KC, or with
  // SPLIT the single chunk kc0 = zh (W still uses every route; the taps pass of
  // 64 routes: the chunk pair kc0 = 2 zh)
  constexpr int KX = SPLIT ? (MODE == kBwdTaps ? 2 : 1) : KC;
  static_assert(!SPLIT || BF, "the route split is built for bf16 operands");
  static_assert(!SPLIT || KC % 2 == 0, "the route split takes an even number of route chunks");
  static_assert(!(SPLIT && MODE == kBwdTaps) || KC == 4, "the taps pass splits 64 routes in halves");
  const int kc0 = SPLIT ? zh * KX : 0;
  constexpr int EOWN = MODE == kBwdTaps ? TB : TB - (S - 1);
  constexpr int NP = MS::kParts;
  constexpr int AROWS = TB + S - 1;   // alpha rows a super-block touches
  constexpr int MROW = CW + 4;        // padded LDS row of one m tile (elements)
  static_assert(S >= 2 && EOWN > 0, "super-block too small for the kernel size");
  // work of this MODE: dx rows, m products of ST taps from tap s0
  constexpr bool DO_DX = MODE != kBwdTaps, DO_M = MODE != kBwdDx;
  // with the activation: P (and g) formed in this pass; g read from gbuf (taps
  // pass) or written there (dx pass)
  constexpr bool PACT = ACT != 0 && MODE != kBwdTaps;
  constexpr bool GIN = ACT != 0 && MODE == kBwdTaps, GOUT = ACT != 0 && MODE == kBwdDx;
  static_assert(ACT != kActRuntime || (MODE == kBwdFused && !PRE),
                "a per-layer activation is built for the fused pass of grouped launches");
  const bool act = ACT == kActRuntime ? act_rt : ACT != 0;  // (uniform)
  static_assert(MODE != kBwdDx || !SPLIT, "dx uses every route chunk");
  static_assert(!PRE || MODE != kBwdDx || ACT != 0,
                "without the activation the prefill dx pass is the plain one (it reads no cache)");
  constexpr int ST = MODE == kBwdTaps ? (S + 1) / 2 : S;
  constexpr bool kOneBody = MODE == kBwdTaps && BF;
  // kBwdTaps: waves w and w + WPG/2 cover the same channels, taps [0, ST) and
  // [ST, S): x and dy rows are read once per workgroup and the dalpha sum over
  // the workgroup's waves covers every tap (one partial per channel group).  With
  // S odd the second half's last tap (s0 + ST - 1 = S) does not exist: its m
  // values are zero, its dalpha operands zero rows, its dbasis never stored.
  static_assert(MODE != kBwdTaps || WPG % 2 == 0, "tap halves pair the waves");
  constexpr int WCH = MODE == kBwdTaps ? WPG / 2 : WPG;  // waves across channels
  // wave index as a scalar (uniform over the wave): the tap half and channel
  // offsets derived from it, and the x / dy row offsets of a window, then stay
  // in scalar registers (as vector values, hoisted out of the loop, they were
  // spilled, and each reload waited for the row loads just issued).  Not in the
  // prefill pass, whose one-wave forms then crash LLVM's AGPR-copy rewrite.
  constexpr bool kPreFused = PRE && MODE == kBwdFused;
  const int wave = kPreFused ? static_cast<int>(threadIdx.x) >> 6
                             : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int th = MODE == kBwdTaps ? wave / WCH : 0;
  const int s0 = th * ST;
  // whether tap s of this wave's half exists (uniform; false only for the last
  // tap of the second half with S odd)
  const bool last_tap_in = MODE != kBwdTaps || S % 2 == 0 || th == 0;
  auto tap_in = [&](int s) { return s + 1 < ST || last_tap_in; };
  // x window rows: every tap (P, or the fused m products), ST taps from s0, none
  constexpr bool NEED_X = DO_M || PACT;
  constexpr int WX = MODE == kBwdTaps ? R + ST - 1 : (NEED_X ? W : 1);

  // m tiles for the dalpha product.  fp32: [token][channel] tiles read as rows.
  // bf16: the dbasis operand of a (token group of 4, channel) is stored as is
  // (8 bytes) and read back transposed with ds_read_b64_tr_b16 (see TrTile).
  using TT = TrTile<NB, NC>;
  // routing-weight rows, unpadded.  bf16: the 8-byte chunk (4 routes) c of row r
  // is stored at chunk c ^ asw(r), so that the W operand reads of a 16-lane group
  // (one chunk of rows 8 (j/4) + j%4 + const) fall on 32 distinct banks; the
  // transposed reads and the staging writes stay conflict-free as well
  constexpr int AP = KP;
  __shared__ __align__(16) E a_lds[2][AROWS][AP];
  auto acol = [](int r, int col) -> int {
    if constexpr (!BF) return col;
    const int sw = KP == 16 ? ((r >> 3) & 3) : (((r >> 1) & 1) | (((r >> 3) & 3) << 1));
    return (col & 3) | (((col >> 2) ^ sw) << 2);
  };
  __shared__ __align__(16) E m_lds[BF ? 1 : WPG][NP][BF ? 1 : TB][BF ? 1 : MROW];
  __shared__ __align__(16) s16x4 m_tr[BF && DO_M ? WPG : 1][NP][BF && DO_M ? TT::kSlots : 1];
  // dalpha B operands of each wave's channels (bf16, one 16-route chunk): rows
  // (s, k), CW channels (with rows (k, s) the reads of a 16-lane group, rows k
  // = j at one s, hit each bank twice); with more routes they stay in registers
  // (the taps pass keeps them in LDS for both chunks, and its dalpha tiles
  // single-buffered, one more barrier per super-block, to stay within two
  // waves per SIMD without register spills)
  constexpr bool kBdaLds = BF && DO_M && (KX == 1 || MODE == kBwdTaps);
  constexpr int BROW = CW + 4;
  __shared__ __align__(16) E b_lds[kBdaLds ? WPG : 1][kBdaLds ? 16 * KX * ST : 1][kBdaLds ? BROW : 1];
  constexpr int DAB = MODE == kBwdTaps ? 1 : 2;  // dalpha tile buffers
  __shared__ float da_lds[DO_M ? DAB : 1][DO_M ? WPG : 1][NB][KX][16][17];

  const E* __restrict__ x = static_cast<const E*>(xv);
  const E* __restrict__ dy = static_cast<const E*>(dyv);
  E* __restrict__ dx = static_cast<E*>(dxv);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = lane & 15, q = lane >> 4;
  const int64_t N = seq.n_tokens;
  const int64_t d0 = (static_cast<int64_t>(bx) * WCH + wave % WCH) * CW;
  const bool wave_on = d0 < D;
  const int64_t dl = d0 + NC * j;
  const bool ch_ok = wave_on && dl < D;

  constexpr int ESZ = static_cast<int>(sizeof(E));
  // super-blocks [sb_lo, sb_hi) of this range: ranges by < gy1 share the first
  // n_old, the others the rest
  const int64_t sb_lo = by < gy1 ? static_cast<int64_t>(by) * n_old / gy1
                                 : n_old + static_cast<int64_t>(by - gy1) * (n_total - n_old) / (gy - gy1);
  const int64_t sb_hi = by < gy1 ? static_cast<int64_t>(by + 1) * n_old / gy1
                                 : n_old + static_cast<int64_t>(by + 1 - gy1) * (n_total - n_old) / (gy - gy1);
  const int nsb = static_cast<int>(sb_hi - sb_lo);
  const int64_t first = sb_lo * EOWN;
  // buffers over the rows this workgroup touches: x / dy / dx rows [row_lo, row_hi),
  // alpha rows [first, a_hi)
  const int64_t last_t0 = first + static_cast<int64_t>(nsb - 1) * EOWN;
  const int64_t row_lo = (first - (S - 1) > 0) ? first - (S - 1) : 0;
  const int64_t row_hi = (last_t0 + TB < N) ? last_t0 + TB : N;
  const int64_t a_hi = (last_t0 + AROWS < N) ? last_t0 + AROWS : N;
  const uint32_t rb = static_cast<uint32_t>(D * ESZ);
  const uint32_t col = static_cast<uint32_t>(dl * ESZ);
  const Buf xb(x + row_lo * D, (row_hi - row_lo) * D * ESZ);
  // dy rows [row_lo, row_hi): rows dys apart, the last one D elements long;
  // dys < 0: one element for every token and channel (not in the prefill
  // pass, whose entry takes rows only: the branch makes LLVM's AGPR-copy
  // rewrite crash on its one-wave forms)
  const bool dy_one = !PRE && dys < 0;
  const uint32_t drb = static_cast<uint32_t>((dy_one ? 0 : dys) * ESZ);
  const Buf dyb(dy_one ? dy : dy + row_lo * dys, dy_one ? ESZ : ((row_hi - row_lo - 1) * dys + D) * ESZ);
  // dy_one: the element's fp32 bits, OR-ed into every converted dy value while
  // the row loads read nothing (kOffNone gives zeros): the conversion stays one
  // instruction (v_lshl_or / v_and_or) and the loop has no branch on the form
  uint32_t dy_or = 0;
  if (dy_one) {
    E e;
    dyb.load<ESZ>(0, &e);
    dy_or = ch_ok ? __float_as_uint(C::to_f(e)) : 0u;
  }
  const bool dy_rows = ch_ok && !dy_one;
  const Buf ab(a_c + first * KP, (a_hi - first) * KP * ESZ);
  const Buf bb(b_c, static_cast<int64_t>(KP) * S * D * ESZ);
  // PRE: the cache (n_seqs = N / T sequences)
  const int64_t T = seq.seq_len;
  const Buf hb(PRE ? pre.hist : nullptr, PRE && pre.hist ? N / T * D * S * ESZ : 0);

  // W operands (P, dx): bop[c][s][kc] = basis[16kc + 4q + v, s, dl + c]
  Op bop[NC][S][KC];
  if constexpr (DO_DX || PACT)
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      E rows[4][NC];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * q + v;
        bb.load<NC * ESZ>(row_off(k * S + s, 0, rb, col, ch_ok), rows[v]);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) bop[c][s][kc] = C::make(rows[0][c], rows[1][c], rows[2][c], rows[3][c]);
    }
  }
  // dalpha B operands: bda[s][cg][kx] = basis[16 (kc0 + kx) + j, s0 + s, d0 + 16cg + 4q + v].
  // The fp32 taps pass loads them per tap where it uses them (from L2): held
  // through the super-block loop they spill past 8 taps
  constexpr bool kBdaMem = !BF && MODE == kBwdTaps;
  auto load_bda = [&](int s, int cg, int kx, E (&e4)[4]) {
    // (with D % 4 == 2 the last group's upper two channels read the next
    // row's first two: finite basis values that meet m products of zero, as
    // a channel pair past D loads x and dy as zeros)
    const int64_t ch = d0 + 16 * cg + 4 * q;
    bb.load<4 * ESZ>(row_off((16 * (kc0 + kx) + j) * S + s0 + s, 0, rb,
                             static_cast<uint32_t>(ch * ESZ), wave_on && ch < D && tap_in(s)),
                     e4);
  };
  Op bda[kBdaMem ? 1 : ST][NC][KX];
  if constexpr (DO_M && !kBdaMem)
#pragma unroll
  for (int kx = 0; kx < KX; ++kx) {
#pragma unroll
    for (int s = 0; s < ST; ++s) {
#pragma unroll
      for (int cg = 0; cg < NC; ++cg) {
        E e4[4];
        load_bda(s, cg, kx, e4);
        if constexpr (kBdaLds)  // read back per tap in the dalpha loop (wave-private rows)
          Vec<E, 4>::store(&b_lds[wave][s * 16 * KX + 16 * kx + j][16 * cg + 4 * q], e4);
        else
          bda[s][cg][kx] = C::make(e4[0], e4[1], e4[2], e4[3]);
      }
    }
  }

  f32x4 dbacc[NC][ST][KX];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int s = 0; s < ST; ++s)
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) dbacc[c][s][kx] = f32x4{0.f, 0.f, 0.f, 0.f};

  // raw rows of one super-block for this lane: x window, dy rows; alpha rows
  // (AROWS x KP elements, spread over the workgroup's threads) for LDS
  constexpr int AVEC = 4;                                  // elements per alpha load
  constexpr int ACHUNKS = AROWS * KP / AVEC;
  constexpr int APER = (ACHUNKS + 64 * WPG - 1) / (64 * WPG);
  E xr[WX][NC];
  E dr[GIN ? 1 : R][NC];
  float gr[GIN ? R : 1][NC];  // GIN: g rows (fp32)
  const uint32_t grb = static_cast<uint32_t>(D * 4), gcol = static_cast<uint32_t>(dl * 4);
  const Buf gib(GIN ? gbuf + row_lo * D : nullptr, GIN ? (row_hi - row_lo) * D * 4 : 0);
  E arw[APER][AVEC];
  auto fetch_xdy = [&](int64_t t0) {
    // offset of window row w = base + w rb: rows before row_lo wrap to >= 2^31
    // and load zeros; a lane past the channel axis starts at kOffNone.  The x
    // window of the taps from s0 starts s0 rows into the full one.  dy rows are
    // t0 + R q + r >= row_lo (never before the buffer, also with dys = 0)
    const uint32_t base = row_off(t0 + R * q - (S - 1), row_lo, rb, col, ch_ok);
    if constexpr (!kPreFused) {
      // both bases first: a value reloaded between the two groups of loads
      // would wait for the first group (the memory counter retires in issue
      // order).  The prefill pass keeps the plain order: its one-wave forms
      // crash LLVM's AGPR-copy rewrite with this one.
      const uint32_t dbase = row_off(t0 + R * q, row_lo, drb, col, dy_rows);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEED_X)
#pragma unroll
        for (int w = 0; w < WX; ++w) xb.load<NC * ESZ>(base + (w + s0) * rb, xr[w]);
      if constexpr (GIN) {
        const uint32_t gbase = row_off(t0 + R * q, row_lo, grb, gcol, ch_ok);
#pragma unroll
        for (int r = 0; r < R; ++r) gib.load<NC * 4>(gbase + r * grb, gr[r]);
      } else if (MODE != kBwdFused && dy_one) {
        // one dy element: the partial passes issue no row loads for it (they
        // would read nothing but take places in the memory queue behind the x
        // rows); the fused pass keeps them, a branch there cost it 3 us
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) dr[GIN ? 0 : r][c] = E(0);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) dyb.load<NC * ESZ>(dbase + r * drb, dr[r]);
      }
    } else {
      if constexpr (NEED_X)
#pragma unroll
        for (int w = 0; w < WX; ++w) xb.load<NC * ESZ>(base + (w + s0) * rb, xr[w]);
      const uint32_t dbase = row_off(t0 + R * q, row_lo, drb, col, dy_rows);
#pragma unroll
      for (int r = 0; r < R; ++r) dyb.load<NC * ESZ>(dbase + r * drb, dr[r]);
    }
  };
  auto fetch_a = [&](int64_t t0) {
    // taps pass: the per-lane terms are formed here each time (an opaque copy
    // of the thread id keeps them from being hoisted out of the loop, where
    // they were spilled and reloaded before every fetch)
    int tid_f = tid;
    if constexpr (MODE == kBwdTaps) asm volatile("" : "+v"(tid_f));
#pragma unroll
    for (int i = 0; i < APER; ++i) {
      const int chunk = tid_f + i * 64 * WPG;
      const int64_t tok = t0 + chunk / (KP / AVEC);
      ab.load<AVEC * ESZ>(row_off(tok, first, KP * ESZ, (chunk % (KP / AVEC)) * AVEC * ESZ,
                                  chunk < ACHUNKS),
                          arw[i]);
    }
  };
  auto fetch = [&](int64_t t0) {
    fetch_xdy(t0);
    fetch_a(t0);
  };
  auto stage_alpha = [&](int buf) {
    // taps pass: the LDS addresses formed here each time, as in fetch_a (a
    // hoisted copy was spilled, and its reload waited for the row loads)
    int tid_s = tid;
    if constexpr (MODE == kBwdTaps) asm volatile("" : "+v"(tid_s));
#pragma unroll
    for (int i = 0; i < APER; ++i) {
      const int chunk = tid_s + i * 64 * WPG;
      const int row = chunk / (KP / AVEC);
      if (chunk < ACHUNKS)
        Vec<E, AVEC>::store(&a_lds[buf][row][acol(row, (chunk % (KP / AVEC)) * AVEC)], arw[i]);
    }
  };

  if (first < N) {
    fetch(first);
    stage_alpha(0);
  }
  __syncthreads();

  // own-row masks of the dbasis alpha^T operands of a super-block with all
  // EOWN own rows (every one but possibly the last of the token axis)
  uint64_t keep_full[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int n_ok = min(max(EOWN - (R * q + 4 * b), 0), 4);
    keep_full[b] = n_ok >= 4 ? ~0ull : ((1ull << (16 * n_ok)) - 1ull);
  }

  StartCursor cursor;
  for (int sb = 0; sb < nsb; ++sb) {
    const int64_t t0 = first + static_cast<int64_t>(sb) * EOWN;
    if (t0 >= N) break;  // uniform over the workgroup
    const int buf = sb & 1;
    const int64_t own_end = (t0 + EOWN < N) ? t0 + EOWN : N;
    const int64_t trun = t0 + R * q;

    // without the activation, the fused and dx passes convert the rows here,
    // before the next super-block's loads (not sunk below them), so that those
    // loads land in the registers the rows just left and the loop carries them
    // without copies: configs[2] and configs[4] steps -1%; the SiLU pass
    // measured 1 us slower this way, and the prefill pass's one-wave forms
    // crash LLVM's AGPR-copy rewrite with it
    constexpr bool kPin = MODE != kBwdTaps && !PRE && ACT == 0;
    // the taps pass converts each x value where an m product uses it instead of
    // keeping an fp32 copy of the window (22 registers for about 40 more VALU:
    // the pass waits far more than it issues, and its spills waited on memory)
    constexpr bool kXOnUse = MODE == kBwdTaps;
    float xw[kXOnUse ? 1 : WX][NC];
    float g[R][NC];
    if constexpr (NEED_X && !kXOnUse)
#pragma unroll
      for (int w = 0; w < WX; ++w)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          xw[w][c] = C::to_f(xr[w][c]);
          if constexpr (kPin) asm volatile("" : "+v"(xw[w][c]));
        }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (GIN) g[r][c] = gr[r][c];
        else g[r][c] = __uint_as_float(__float_as_uint(C::to_f(dr[r][c])) | dy_or);
        if constexpr (kPin) asm volatile("" : "+v"(g[r][c]));
      }
    const bool more = (sb + 1 < nsb) && (t0 + EOWN < N);
    // the taps pass loads the next x / dy rows after its m products, where
    // fewer registers are live (issued here, they were spilled in the body);
    // the others load them here (kPin: also after the last super-block of the
    // range, whose next rows fall past the buffers or are never used)
    if constexpr (kPin) {
      __builtin_amdgcn_sched_barrier(0);
      fetch(t0 + EOWN);
    } else if (more) {
      // (the taps pass loads the next routing weights inside its products)
      if constexpr (MODE != kBwdTaps) fetch(t0 + EOWN);
    }

    // alpha operand of token-row block b shifted by e rows (row i = j)
    auto aop = [&](int e, int b, int kc) -> Op {
      const int r = R * (j >> 2) + 4 * b + (j & 3) + e;
      return *reinterpret_cast<const Op*>(&a_lds[buf][r][acol(r, 16 * kc + 4 * q)]);
    };

    // uniform: does a sequence start fall where it masks a tap of the rows
    // [t0, t0 + TB + S - 1) (own rows, their later rows, the lanes' extended runs)?
    const int64_t w_lo = t0 - (S - 2), w_hi = t0 + TB + S - 2;
    const bool interior = !cursor.starts_in(seq, w_lo, w_hi);

    f32x4 dacc[NB][KX];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) dacc[b][kx] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto body = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      // ok[r]: tap bits of row r of this lane's run extended by S-1 later rows
      // (the later rows only for dx)
      constexpr int NOK = DO_DX ? R + S - 1 : R;
      uint32_t ok[NOK];
      if (MASK && (!kOneBody || !interior)) {
        tap_bits_rows<S, NOK>(seq, trun, w_lo, w_hi, ok);
      } else {
#pragma unroll
        for (int r = 0; r < NOK; ++r) ok[r] = (1u << S) - 1u;
      }
      // PRE: masked taps read the cache (uniform: is there one?)
      // (the taps pass loads them where it forms an m product: a window held in
      // registers through its tap loop spills)
      constexpr bool HX = PRE && MASK;
      constexpr bool HXW = HX && MODE != kBwdTaps;
      float hx[HXW ? W : 1][NC];
      bool use_h = false;
      if constexpr (HX) {
        use_h = pre.hist != nullptr && (!kOneBody || !interior);
        if constexpr (HXW)
          if (use_h) hist_window<S, W, NC, E>(hb, trun - (S - 1), T, N, D, dl, ch_ok, hx);
      }

      if constexpr (PACT) if (act) {  // (act: uniform; always with a fixed ACT)
        float p[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) p[r][c] = 0.f;
        // jobs (s, b, c): W block by MFMA, then its 4 FMAs; the MFMA of job
        // i + kLead is issued before the FMAs of job i to cover its latency
        constexpr int NJ = S * NB * NC;
        f32x4 wq[NJ];
        auto issue = [&](int jb) {
          const int s = jb / (NB * NC), b = (jb / NC) % NB, c = jb % NC;
          f32x4 w4 = {0.f, 0.f, 0.f, 0.f};
          if constexpr (BF && KC % 2 == 0) {
#pragma unroll
            for (int kp = 0; kp < KC; kp += 2)
              w4 = C::mma2(aop(0, b, kp), aop(0, b, kp + 1), bop[c][s][kp], bop[c][s][kp + 1], w4);
          } else {
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) w4 = C::mma(aop(0, b, kc), bop[c][s][kc], w4);
          }
          wq[jb] = w4;
        };
#pragma unroll
        for (int jb = 0; jb < kLead && jb < NJ; ++jb) issue(jb);
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb) {
          if (jb + kLead < NJ) issue(jb + kLead);
          const int s = jb / (NB * NC), b = (jb / NC) % NB, c = jb % NC;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * b + v;
            if (!MASK || ((ok[r] >> s) & 1u)) p[r][c] = fmaf(xw[r + s][c], wq[jb][v], p[r][c]);
            else if (HXW && use_h) p[r][c] = fmaf(hx[HXW ? r + s : 0][c], wq[jb][v], p[r][c]);
          }
        }
        // g *= silu'(P) = sg (1 + P (1 - sg)), sg = sigmoid(P) as sigmoid_f forms
        // it, in stages over all R x NC values so that the latencies of their
        // independent transcendentals overlap
        float sg[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) sg[r][c] = __builtin_amdgcn_exp2f(-p[r][c] * 1.4426950408889634f);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) sg[r][c] = __builtin_amdgcn_rcpf(1.0f + sg[r][c]);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            // silu'(P) = sg + P sg (1 - sg): two FMAs on sg
            const float v = fmaf(-sg[r][c], sg[r][c], sg[r][c]);
            g[r][c] = g[r][c] * fmaf(p[r][c], v, sg[r][c]);
          }
      }
      // the dx pass with the activation: this super-block's own rows of g for
      // the taps pass (the buffer ends at the last own row)
      if constexpr (GOUT) {
        const Buf gob(gbuf + row_lo * D, (own_end - row_lo) * D * 4);
        const uint32_t gb0 = row_off(trun, row_lo, grb, gcol, ch_ok);
#pragma unroll
        for (int r = 0; r < R; ++r) gob.store<NC * 4>(gb0 + r * grb, g[r]);
      }

      // dx: taps in descending order, so that the first jobs (shift 0) need none
      // of the rows gf brings from the next lane group (with SPLIT, by the
      // kc0 = 0 workgroups only)
      if (DO_DX && dx != nullptr && kc0 == 0) {
        // g of the S-1 rows after this lane's run: first rows of lane group q+1
        // (row R + e of this lane's run is row e % R of lane group q + 1 + e / R:
        // past 9 taps the rows of two later groups)
        float gf[S - 1][NC];
#pragma unroll
        for (int e = 0; e < S - 1; ++e) {
          const int src_lane = (lane + 16 * (1 + e / R)) & 63;
#pragma unroll
          for (int c = 0; c < NC; ++c) gf[e][c] = __shfl(g[e % R][c], src_lane, 64);
        }
        float dxa[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int c = 0; c < NC; ++c) dxa[r][c] = 0.f;
        constexpr int NJ = S * NB * NC;
        f32x4 wq[NJ];
        auto issue = [&](int jb) {
          const int s = S - 1 - jb / (NB * NC), b = (jb / NC) % NB, c = jb % NC;
          f32x4 w4 = {0.f, 0.f, 0.f, 0.f};
          if constexpr (BF && KC % 2 == 0) {
#pragma unroll
            for (int kp = 0; kp < KC; kp += 2)
              w4 = C::mma2(aop(S - 1 - s, b, kp), aop(S - 1 - s, b, kp + 1), bop[c][s][kp],
                           bop[c][s][kp + 1], w4);
          } else {
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) w4 = C::mma(aop(S - 1 - s, b, kc), bop[c][s][kc], w4);
          }
          wq[jb] = w4;
        };
#pragma unroll
        for (int jb = 0; jb < kLead && jb < NJ; ++jb) issue(jb);
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb) {
          if (jb + kLead < NJ) issue(jb + kLead);
          const int s = S - 1 - jb / (NB * NC), b = (jb / NC) % NB, c = jb % NC;
          const int off = S - 1 - s;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * b + v;
            const int src = r + off;
            const float gs = (src < R) ? g[src < R ? src : 0][c] : gf[src >= R ? src - R : 0][c];
            if (!MASK || ((ok[src] >> s) & 1u)) dxa[r][c] = fmaf(gs, wq[jb][v], dxa[r][c]);
          }
        }
        // the buffer ends at this super-block's last own row: later rows drop
        const Buf dxb(dx + row_lo * D, (own_end - row_lo) * D * ESZ);
        const uint32_t base = row_off(trun, row_lo, rb, col, ch_ok);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          E o[NC];
          if constexpr (BF && NC == 2) {
            const uint32_t pk = pack2_bf16(dxa[r][0], dxa[r][1]);
            __builtin_memcpy(o, &pk, 4);
          } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) o[c] = C::from_f(dxa[r][c]);
          }
          dxb.store<NC * ESZ>(base + r * rb, o);
        }
      }

      if constexpr (DO_M) {
        // alpha^T operands of the dbasis MFMA (zero for rows that are not this
        // super-block's own): at[b][kx][v] = alpha[trun + 4b + v, 16 (kc0 + kx) + j]
        Op at[NB][KX];
        if constexpr (BF) {
          // transposed read: supplier lane 4e + a of each 16-lane group holds the
          // 4 routing weights 16kc + 4a.. of row R q + 4b + e (ds_read_b64_tr_b16)
          const int own_rows = static_cast<int>(own_end - t0);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            uint64_t keep = keep_full[b];
            if (own_rows != EOWN) {  // uniform: the last super-block of the token axis
              const int n_ok = min(max(own_rows - (R * q + 4 * b), 0), 4);
              keep = n_ok >= 4 ? ~0ull : ((1ull << (16 * n_ok)) - 1ull);
            }
#pragma unroll
            for (int kx = 0; kx < KX; ++kx) {
              const int r = R * q + 4 * b + (j >> 2);
              const Op v = TT::read(&a_lds[buf][r][acol(r, 16 * (kc0 + kx) + 4 * (j & 3))]);
              at[b][kx] = __builtin_bit_cast(Op, __builtin_bit_cast(uint64_t, v) & keep);
            }
          }
        } else {
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int kx = 0; kx < KX; ++kx) {
              E e4[4];
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int row = R * q + 4 * b + v;
                e4[v] = (t0 + row < own_end) ? a_lds[buf][row][16 * (kc0 + kx) + j] : E(0);
              }
              at[b][kx] = C::make(e4[0], e4[1], e4[2], e4[3]);
            }
        }
        // per tap: m_s = g * x[t-(S-1-s)] -> dbasis MFMA, wave-private LDS tile -> dalpha MFMA
        if constexpr (BF) {
          // both products contract 32 entries per v_mfma_f32_16x16x32_bf16: dbasis
          // the 8 rows of this lane's run (token blocks b, b+1), dalpha the 32
          // channels of the wave (channel groups 0, 1); A and B operands list
          // their entries in the same order
          static_assert(NB % 2 == 0 && NC == 2, "16x16x32 pairing");
          // tap s: m_s -> bf16 hi / lo operands -> the wave's LDS tile and the
          // dbasis MFMAs; the dalpha reads of tap s are issued before the m values
          // of tap s + 1 are computed and written, so that VALU work covers the
          // LDS latency (one tile suffices: a wave's LDS operations complete in
          // issue order, so the writes of tap s + 1 follow the reads of tap s)
          auto stage_m = [&](int s) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
#pragma unroll
              for (int b2 = 0; b2 < NB; b2 += 2) {
                Op mh[2], ml[2];
                // M: masked products (MASK, and with one body a super-block
                // that holds a sequence start)
                auto form = [&](auto mtag) {
                constexpr bool M = MASK && decltype(mtag)::value;
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                  const int b = b2 + bb;
                  // m of rows 4b..4b+3 of channel NC j + c, split into bf16 hi / lo
                  uint32_t hbits[4];
                  float lo[4];
#pragma unroll
                  for (int v = 0; v < 4; ++v) {
                    const int r = 4 * b + v;
                    // (the mask has no bit for a tap past S)
                    const bool on = !M ? tap_in(s) : static_cast<bool>((ok[r] >> (s0 + s)) & 1u);
                    float xv;
                    if constexpr (kXOnUse) xv = C::to_f(xr[r + s][c]);
                    else xv = xw[r + s][c];
                    float mval = on ? g[r][c] * xv : 0.f;
                    if constexpr (HXW && M) {
                      if (use_h && !on) mval = g[r][c] * hx[HXW ? r + s : 0][c];
                    } else if constexpr (HX && M) {
                      // every lane issues the cache load, with an out-of-range
                      // offset (zero) where its tap does not reach before the
                      // sequence, and selects: no divergent branch around a load
                      const bool want = use_h && !on && tap_in(s);
                      const float h = hist_at<S, E>(hb, trun - (S - 1) + s0 + r + s, T, N, D, dl,
                                                    ch_ok && want, c);
                      mval = want ? g[r][c] * h : mval;
                    }
                    hbits[v] = __float_as_uint(mval) & 0xffff0000u;
                    lo[v] = mval - __uint_as_float(hbits[v]);
                  }
                  mh[bb] = pack4_hi(hbits[0], hbits[1], hbits[2], hbits[3]);
                  ml[bb] = pack4_bf16(lo[0], lo[1], lo[2], lo[3]);
                  m_tr[wave][0][TT::wslot(j, q, b, c)] = mh[bb];
                  m_tr[wave][1][TT::wslot(j, q, b, c)] = ml[bb];
                }
                };
                if constexpr (kOneBody) {
                  if (interior) form(std::false_type{});
                  else form(std::true_type{});
                } else {
                  form(std::true_type{});
                }
#pragma unroll
                for (int kx = 0; kx < KX; ++kx) {
                  dbacc[c][s][kx] = mma32(mh[0], mh[1], at[b2][kx], at[b2 + 1][kx], dbacc[c][s][kx]);
                  dbacc[c][s][kx] = mma32(ml[0], ml[1], at[b2][kx], at[b2 + 1][kx], dbacc[c][s][kx]);
                }
              }
            }
          };
          stage_m(0);
          // taps pass: the next super-block's routing weights are loaded here,
          // after the first tap's products (where the fewest registers are
          // live), and go to LDS after the last tap, the loads covered by three
          // taps' work; loaded at the top of the super-block they were spilled
          // at once, the spill waiting for the loads to land.  The other half of
          // the double buffer has been free since the previous super-block's
          // closing barrier.
          if constexpr (MODE == kBwdTaps) {
            if (more) fetch_a(t0 + EOWN);
          }
#pragma unroll
          for (int s = 0; s < ST; ++s) {
            wave_lds_sync();
            Op ra[NB][NP][2];
#pragma unroll
            for (int rb = 0; rb < NB; ++rb)
#pragma unroll
              for (int h = 0; h < NP; ++h)
#pragma unroll
                for (int cg = 0; cg < 2; ++cg)
                  ra[rb][h][cg] = TT::read(&m_tr[wave][h][TT::rslot(j, q, rb, cg)]);
            // dalpha B operands of tap s: basis[16 kc + j][s][16 cg + 4 q + {0..3}]
            Op bs[KX][2];
#pragma unroll
            for (int kx = 0; kx < KX; ++kx)
#pragma unroll
              for (int cg = 0; cg < 2; ++cg) {
                if constexpr (kBdaLds)
                  bs[kx][cg] = *reinterpret_cast<const Op*>(&b_lds[wave][s * 16 * KX + 16 * kx + j][16 * cg + 4 * q]);
                else
                  bs[kx][cg] = bda[s][cg][kx];
              }
            // keep the reads ahead of the next tap's VALU work
            __builtin_amdgcn_sched_barrier(0);
            if (s + 1 < ST) stage_m(s + 1);
            // dalpha over this wave's channels for tap s: D[t][k] += sum_ch m[t][ch] basis[k][s][ch]
#pragma unroll
            for (int rb = 0; rb < NB; ++rb)
#pragma unroll
              for (int h = 0; h < NP; ++h)
#pragma unroll
                for (int kx = 0; kx < KX; ++kx)
                  dacc[rb][kx] = mma32(ra[rb][h][0], ra[rb][h][1], bs[kx][0], bs[kx][1], dacc[rb][kx]);
          }
          if constexpr (MODE == kBwdTaps) {
            if (more) stage_alpha(buf ^ 1);
          }
          wave_lds_sync();
        } else {
        // taps pass: the next super-block's routing weights are loaded before the
        // m products and go to LDS after them (the other half of the double
        // buffer has been free since the previous super-block's closing barrier)
        if constexpr (MODE == kBwdTaps) {
          if (more) fetch_a(t0 + EOWN);
        }
#pragma unroll
        for (int s = 0; s < ST; ++s) {
          Op bm[kBdaMem ? NC : 1][KX];
          if constexpr (kBdaMem)
#pragma unroll
            for (int cg = 0; cg < NC; ++cg)
#pragma unroll
              for (int kx = 0; kx < KX; ++kx) {
                E e4[4];
                load_bda(s, cg, kx, e4);
                bm[cg][kx] = C::make(e4[0], e4[1], e4[2], e4[3]);
              }
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            E mv[NP][4][NC];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int r = 4 * b + v;
              const bool on = !MASK ? tap_in(s) : static_cast<bool>((ok[r] >> (s0 + s)) & 1u);
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                E parts[NP];
                const float xv = kXOnUse ? C::to_f(xr[r + s][c]) : xw[kXOnUse ? 0 : r + s][c];
                float mval = on ? g[r][c] * xv : 0.f;
                if (HXW && use_h && !on && tap_in(s)) mval = g[r][c] * hx[HXW ? r + s : 0][c];
                MS::split(mval, parts);
#pragma unroll
                for (int h = 0; h < NP; ++h) mv[h][v][c] = parts[h];
              }
#pragma unroll
              for (int h = 0; h < NP; ++h) XV::store(&m_lds[wave][h][R * q + r][NC * j], mv[h][v]);
            }
#pragma unroll
            for (int h = 0; h < NP; ++h)
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                const Op am = C::make(mv[h][0][c], mv[h][1][c], mv[h][2][c], mv[h][3][c]);
#pragma unroll
                for (int kx = 0; kx < KX; ++kx) dbacc[c][s][kx] = C::mma(am, at[b][kx], dbacc[c][s][kx]);
              }
          }
          wave_lds_sync();
          // dalpha over this wave's channels for tap s: D[t][k] += sum_ch m[t][ch] basis[k][s][ch]
#pragma unroll
          for (int rb = 0; rb < NB; ++rb)
#pragma unroll
            for (int h = 0; h < NP; ++h)
#pragma unroll
              for (int cg = 0; cg < NC; ++cg) {
                const Op am = *reinterpret_cast<const Op*>(&m_lds[wave][h][16 * rb + j][16 * cg + 4 * q]);
#pragma unroll
                for (int kx = 0; kx < KX; ++kx)
                  dacc[rb][kx] = C::mma(am, kBdaMem ? bm[kBdaMem ? cg : 0][kx] : bda[kBdaMem ? 0 : s][cg][kx],
                                        dacc[rb][kx]);
              }
          wave_lds_sync();
        }
        if constexpr (MODE == kBwdTaps) {
          if (more) stage_alpha(buf ^ 1);
        }
        }
      }
    };
    // the bf16 taps pass runs one body, choosing masked or plain m products
    // inside it (a uniform branch per product group): with a body per form,
    // the dbasis accumulators met at the join in different registers and the
    // loop copied all of them twice per super-block (128 moves at 8 taps)
    if constexpr (kOneBody) body(std::true_type{});
    else if (interior) body(std::false_type{});
    else body(std::true_type{});
    if constexpr (MODE == kBwdTaps) {
      if (more) fetch_xdy(t0 + EOWN);
    }

    if constexpr (DO_M) {
      // one tile buffer: every wave has summed the previous super-block's tiles
      if constexpr (DAB == 1) __syncthreads();
#pragma unroll
      for (int rb = 0; rb < NB; ++rb)
#pragma unroll
        for (int kx = 0; kx < KX; ++kx)
#pragma unroll
          for (int v = 0; v < 4; ++v) da_lds[buf % DAB][wave][rb][kx][4 * q + v][j] = dacc[rb][kx][v];
    }
    if constexpr (MODE != kBwdTaps) {
      if (more) stage_alpha(buf ^ 1);
    }
    __syncthreads();
    // sum the WPG waves' dalpha tiles in wave order; own rows only
    if constexpr (DO_M && BF) {
      // unrolled (every thread sums the same number of elements), so that all
      // of its LDS reads are in flight together; fp32 keeps the loop below
      // (LLVM's AGPR rewrite fails on the unrolled form of its 8-tap kernel)
      constexpr int NSUM = NB * KX * 256 / (64 * WPG);
      static_assert(NB * KX * 256 % (64 * WPG) == 0, "dalpha tile elements per thread");
      float* __restrict__ pd = part_da + (static_cast<int64_t>(bx) * N + t0) * KP + 16 * kc0;
      const int n_own = static_cast<int>(own_end - t0);
      int tid_d = tid;  // taps pass: offsets formed here each time (see stage_alpha)
      if constexpr (MODE == kBwdTaps) asm volatile("" : "+v"(tid_d));
      // every tile value read first (all reads in flight together), then the
      // sums in wave order
      float tv[NSUM][WPG];
#pragma unroll
      for (int i = 0; i < NSUM; ++i) {
        const int idx = tid_d + i * 64 * WPG;
        const int rb = idx / (KX * 256);
        const int kx = (idx / 256) % KX;
        const int row = (idx >> 4) & 15, col = idx & 15;
#pragma unroll
        for (int w = 0; w < WPG; ++w) tv[i][w] = da_lds[buf % DAB][w][rb][kx][row][col];
      }
#pragma unroll
      for (int i = 0; i < NSUM; ++i) {
        const int idx = tid_d + i * 64 * WPG;
        const int rb = idx / (KX * 256);
        const int kx = (idx / 256) % KX;
        const int row = (idx >> 4) & 15, col = idx & 15;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < WPG; ++w) sum += tv[i][w];
        if (16 * rb + row < n_own) pd[(16 * rb + row) * KP + 16 * kx + col] = sum;
      }
    } else if constexpr (DO_M) {
      const int64_t pda = bx;
      for (int idx = tid; idx < NB * KX * 256; idx += 64 * WPG) {
        const int rb = idx / (KX * 256);
        const int kx = (idx / 256) % KX;
        const int row = (idx >> 4) & 15, col = idx & 15;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < WPG; ++w) sum += da_lds[buf % DAB][w][rb][kx][row][col];
        const int64_t t = t0 + 16 * rb + row;
        if (t < own_end) part_da[(pda * N + t) * KP + 16 * (kc0 + kx) + col] = sum;
      }
    }
  }

  // this workgroup's dbasis partial: dbacc[c][s][kx][v] is
  // (k = 16 (kc0 + kx) + j, s0 + s, channel d0 + NC (4q + v) + c)
  if (DO_M && wave_on) {
    const int64_t base = static_cast<int64_t>(by) * KP;
#pragma unroll
    for (int kx = 0; kx < KX; ++kx)
#pragma unroll
      for (int s = 0; s < ST; ++s)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int64_t ch = d0 + NC * (4 * q + v) + c;
            if (ch < D && tap_in(s))
              part_db[((base + 16 * (kc0 + kx) + j) * S + s0 + s) * D + ch] = dbacc[c][s][kx][v];
          }
  }
}

// Route parts of a split grid: one per route chunk, or route-chunk pairs for the
// taps pass.
template <int KC, bool SPLIT, int MODE>
constexpr int kRouteParts = SPLIT ? (MODE == kBwdTaps ? KC / 2 : KC) : 1;

// Workgroup -> (channel group bx, token range by, route chunk zh) over a grid of
// gx channel groups.  Split in NZ route chunks, the grid is 1-D and the NZ
// parts of a tile are 8 workgroup ids apart: ids go round-robin over the 8
// XCDs, so the parts run on one XCD at about the same time and the later ones
// find the tile's x / dy rows in that XCD's L2.  Returns false for the ids of
// the 1-D grid past the last tile.
// Block (x id, y id) of a 2-D grid (NZ = 1), or id L of the 1-D grid of a split one.
template <int NZ>
__device__ __forceinline__ bool bwd_block(int gx, int gy, int idx, int idy, int& bx, int& by,
                                          int& zh) {
  bx = idx;
  by = idy;
  zh = 0;
  if constexpr (NZ > 1) {
    const int L = idx;
    const int t = (L / (8 * NZ)) * 8 + (L & 7);
    if (t >= gx * gy) return false;
    zh = (L >> 3) % NZ;
    bx = t % gx;
    by = t / gx;
  }
  return true;
}

template <int S, int KC, int NB, int NC, int WPG, bool ACT, bool BF, bool SPLIT, int MODE>
__global__ void __launch_bounds__(64 * WPG)
__attribute__((amdgpu_waves_per_eu(kBwdMinWaves<S, KC, MODE, BF, ACT>)))
bwd_kernel(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
           const typename CT<BF>::elem* __restrict__ a_c,
           const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ dxv,
           float* __restrict__ part_da, float* __restrict__ part_db, SeqLayout seq, int64_t D,
           int gx, int gy, int gy1, int n_old, int n_total, float* __restrict__ gbuf = nullptr) {
  int bx, by, zh;
  if (!bwd_block<kRouteParts<KC, SPLIT, MODE>>(gx, gy, static_cast<int>(blockIdx.x),
                                               static_cast<int>(blockIdx.y), bx, by, zh))
    return;  // whole workgroup, before any barrier
  bwd_tile<S, KC, NB, NC, WPG, ACT, BF, SPLIT, MODE>(xv, dyv, dys, a_c, b_c, dxv, part_da, part_db,
                                                     seq, D, bx, by, zh, gy, gy1, n_old, n_total,
                                                     Pre{nullptr, nullptr}, gbuf);
}

// Prefill from a cache (Pre): the fused pass on a 2-D grid (bf16 with 32
// routes, which the plain backward splits, at one wave per SIMD: both route
// chunks' accumulators and operands stay in registers; with 64 routes at two,
// as LLVM's AGPR-copy rewrite crashes on that one-wave form).  bf16 with 6-8
// taps runs it at one wave too (at two it spilled up to 121 registers at 16
// routes and 440 at 32): B4 T4096 D2048 with SiLU, 16 routes: 6 taps
// 204 -> 182 us, 7 taps 387 -> 200, 8 taps 537 -> 237; 32 routes, 8 taps
// 1832 -> 973.
template <int S, int KC, bool BF>
constexpr int kBwdPreWaves = (BF && (KC == 2 || (KC == 1 && S >= 6))) ? 1
                             : (BF && KC >= 2) ? 2 : kBwdMinWaves<S, KC, kBwdFused, BF>;
// With 64 routes (SPLIT) it is split in route chunks like the plain pass.
template <int S, int KC, int NB, int NC, int WPG, bool ACT, bool BF, bool SPLIT>
__global__ void __launch_bounds__(64 * WPG)
__attribute__((amdgpu_waves_per_eu(SPLIT ? kBwdMinWaves<S, KC, kBwdFused, BF>
                                         : kBwdPreWaves<S, KC, BF>)))
bwd_pre_kernel(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
               const typename CT<BF>::elem* __restrict__ a_c,
               const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ dxv,
               float* __restrict__ part_da, float* __restrict__ part_db, SeqLayout seq, int64_t D,
               int gx, int gy, int gy1, int n_old, int n_total, Pre pre) {
  int bx, by, zh;
  if (!bwd_block<SPLIT ? KC : 1>(gx, gy, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y),
                                 bx, by, zh))
    return;  // whole workgroup, before any barrier
  bwd_tile<S, KC, NB, NC, WPG, ACT, BF, SPLIT, kBwdFused, true>(
      xv, dyv, dys, a_c, b_c, dxv, part_da, part_db, seq, D, bx, by, zh, gy, gy1, n_old, n_total,
      pre);
}

// Prefill from a cache in the two-pass form (bf16; the shapes of bwd_two_pass,
// and with the activation those of pre_two_pass_g): the m products of the taps pass,
// whose masked taps read the cache (with the activation from g = pre.g).
// Without the activation the dx pass is the plain one (dx reads no cache); with
// it, bwd_pre_dx_kernel, whose P reads the cache and which writes pre.g.
// With 64 routes (SPLIT) the taps pass runs in route halves on a 1-D grid, as
// the plain one does.
template <int S, int KC, int NB, int NC, int WPG, bool ACT, bool BF, bool SPLIT = false>
__global__ void __launch_bounds__(64 * WPG)
__attribute__((amdgpu_waves_per_eu(kBwdMinWaves<S, KC, kBwdTaps, BF>)))
bwd_pre_taps_kernel(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
                    const typename CT<BF>::elem* __restrict__ a_c,
                    const typename CT<BF>::elem* __restrict__ b_c, float* __restrict__ part_da,
                    float* __restrict__ part_db, SeqLayout seq, int64_t D, int gx, int gy,
                    int gy1, int n_old, int n_total, Pre pre) {
  int bx, by, zh;
  if (!bwd_block<kRouteParts<KC, SPLIT, kBwdTaps>>(gx, gy, static_cast<int>(blockIdx.x),
                                                   static_cast<int>(blockIdx.y), bx, by, zh))
    return;  // whole workgroup, before any barrier
  bwd_tile<S, KC, NB, NC, WPG, ACT, BF, SPLIT, kBwdTaps, true>(
      xv, dyv, dys, a_c, b_c, nullptr, part_da, part_db, seq, D, bx, by, zh, gy, gy1, n_old,
      n_total, pre, pre.g);
}

// (one wave per SIMD from 7 taps: at two it spilled 36 registers at 8 taps;
// 32 routes with SiLU, B4 T4096 D2048: 8 taps 427 -> 361 us per backward entry;
// with 64 routes from 5 taps, as the plain dx pass)
template <int S, int KC, int NB, int NC, int WPG, bool BF>
__global__ void __launch_bounds__(64 * WPG)
__attribute__((amdgpu_waves_per_eu((S >= 7 || (KC >= 4 && S >= 5)) ? 1 : 2)))
bwd_pre_dx_kernel(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
                  const typename CT<BF>::elem* __restrict__ a_c,
                  const typename CT<BF>::elem* __restrict__ b_c, void* __restrict__ dxv,
                  SeqLayout seq, int64_t D, int gx, int gy, int gy1, int n_old, int n_total,
                  Pre pre) {
  bwd_tile<S, KC, NB, NC, WPG, true, BF, false, kBwdDx, true>(
      xv, dyv, dys, a_c, b_c, dxv, nullptr, nullptr, seq, D, static_cast<int>(blockIdx.x),
      static_cast<int>(blockIdx.y), 0, gy, gy1, n_old, n_total, pre, pre.g);
}

// Several layers in one launch (1-D grid, the layers' grids one after another:
// gx gy blocks of layer i, or its split grid's ids).
template <int S, int KC, int NB, int NC, int WPG, int ACT, bool BF, bool SPLIT, int MODE>
__global__ void __launch_bounds__(64 * WPG)
__attribute__((amdgpu_waves_per_eu(kBwdMinWaves<S, KC, MODE, BF, ACT != 0>)))
bwd_layers_kernel(BwdLayers ly, SeqLayout seq) {
  using E = typename CT<BF>::elem;
  const int blk = static_cast<int>(blockIdx.x);
  const BwdLayer* Lp = &ly.l[layer_index(ly, blk)];
  int local = blk - Lp->blk0;
  int row = 0;
  if constexpr (!SPLIT) {
    const int gxl = Lp->gx;
    while (local >= gxl) {  // scalar: local < gx gy, at most gy - 1 steps
      local -= gxl;
      ++row;
    }
  }
  int bx, by, zh;
  if (!bwd_block<kRouteParts<KC, SPLIT, MODE>>(Lp->gx, Lp->gy, local, row, bx, by, zh))
    return;  // whole workgroup, before any barrier
  bwd_tile<S, KC, NB, NC, WPG, ACT, BF, SPLIT, MODE>(
      Lp->x, Lp->dy, Lp->dys, static_cast<const E*>(Lp->a), static_cast<const E*>(Lp->b), Lp->dx,
      Lp->part_da, Lp->part_db, seq, Lp->D, bx, by, zh, Lp->gy, Lp->gy1, Lp->n_old, Lp->n_total,
      Pre{nullptr, nullptr}, Lp->gbuf, Lp->act != 0);
}

}  // namespace mfma
}  // namespace moc
