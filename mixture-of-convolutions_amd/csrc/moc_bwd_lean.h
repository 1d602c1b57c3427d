// Fused backward (stage 1) at four waves per SIMD: bf16 operands, up to 16
// routes, 2 to 4 taps (the headline layer shape), the work of the fused pass of
// bwd_tile (moc_mfma.h) on a register budget of 128 VGPRs.
//
// Why a second form of the fused pass: the backward is VALU-issue bound, and
// one SIMD issues fp32 VALU work about 45% faster from four waves than from two
// (probe on this part: a wave64 v_fma_f32 every 1.7 cycles with four waves per
// SIMD, 2.5 with two, 5 with one; MFMA and VALU issue do not overlap).  The
// fused pass of bwd_tile holds 32 channels per wave and needs about 230 VGPRs,
// i.e. two waves per SIMD.  Here a wave holds 16 channels (one per lane, NC = 1)
// of the same 32-token super-block, so every per-lane array halves, and a
// workgroup of 8 waves covers the same 128 channels as bwd_tile's 4: the
// channel groups, token ranges and partial-sum layouts are those of bwd_tile's
// grid, and stage 2 is unchanged.
//
// Work per super-block and wave (rows t0 .. t0 + 31, own rows the first EOWN):
//   W_s = alpha . basis_s by MFMA (16x16x16, 16 routes), P = sum_s W_s x_s,
//   g = dy silu'(P); dx[u] = sum_s g[u+S-1-s] W_s[u+S-1-s] (W at shifted rows
//   by MFMA on shifted alpha rows, g of the next lane group's first rows by a
//   cross-lane read); m_s = g x_s split in bf16 hi / lo; dbasis += alpha^T m_s
//   (16x16x32 over the 32 tokens, accumulated over the whole range in
//   registers); dalpha += m . basis^T over (tap pair, 16 channels) (16x16x32,
//   m read back transposed from a wave-private LDS tile with
//   ds_read_b64_tr_b16); the 8 waves' dalpha tiles summed in LDS in wave order.
#pragma once

#include "moc_mfma.h"

namespace moc {
namespace mfma {

// m tile of one wave for the transposed dalpha reads, one channel per lane.
// Writer lane (j, q) holds, per token block b, m of channel j at the tokens
// 4 g + {0..3} of token group g = 2 q + b: one 8-byte slot.  The dalpha A
// operand wants, in lane i of 16-lane group qq, the channels 4 qq + {0..3} of
// token 16 rb + i; ds_read_b64_tr_b16 gives lane i element i % 4 of the slots
// read by lanes i / 4 + {0, 4, 8, 12} of its group, so reader lane 4 e + a
// reads the slot of channel 4 qq + e, token group 4 rb + a.  Slot (ch, g) sits
// at g 16 + (ch ^ 4 (g & 3)): a writer group covers 16 consecutive slots, a
// reader group 16 distinct slots modulo 16 (no bank conflicts).
struct TrTile1 {
  static constexpr int kSlots = 8 * 16;  // 8 token groups x 16 channels
  static __device__ __forceinline__ int wslot(int j, int q, int b) {
    const int g = 2 * q + b;
    return g * 16 + (j ^ (4 * (g & 3)));
  }
  static __device__ __forceinline__ int rslot(int i, int qq, int rb) {
    const int e = i >> 2, a = i & 3;
    const int g = 4 * rb + a;
    return g * 16 + ((4 * qq + e) ^ (4 * a));
  }
};

__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

#ifndef MOC_LEAN_WAVES
#define MOC_LEAN_WAVES 4
#endif
constexpr int kLeanWPG = 8;        // waves per workgroup (8 x 16 = 128 channels)
constexpr int kLeanCW = 16;        // channels per wave

// Shapes the lean pass serves (bf16 operands, single launches).
constexpr bool bwd_lean(int S, int KC, bool bf) { return bf && KC == 1 && S >= 2 && S <= 4; }

// The work of workgroup (bx, by) of one layer; the __global__ wrappers below
// map a single launch's 2-D grid or a grouped launch's 1-D grid onto it.
template <int S, int ACT, bool DY1>
__device__ __forceinline__ void
bwd_lean_tile(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
              const uint16_t* __restrict__ a_c, const uint16_t* __restrict__ b_c,
              void* __restrict__ dxv, float* __restrict__ part_da, float* __restrict__ part_db,
              SeqLayout seq, int64_t D, int bx, int by, int gy, int gy1, int n_old, int n_total,
              bool act_rt = false) {
  const bool act = ACT == kActRuntime ? act_rt : ACT != 0;  // (uniform)
  using E = uint16_t;
  using Op = s16x4;
  constexpr int NB = 2, R = 8, TB = 32, W = R + S - 1, EOWN = TB - (S - 1);
  constexpr int KP = 16, AROWS = TB + S - 1, WPG = kLeanWPG, CW = kLeanCW;
  constexpr int ESZ = 2;
  static_assert(S >= 2 && S <= 4, "lean backward: 2 to 4 taps");

  // routing-weight rows of a super-block, twice: copy b holds rows 4 b .. (row
  // rho of copy b is super-block row rho + 4 b), so that the W operand reads of
  // token block b at shift e (rows 8 (i / 4) + (i % 4) + e of the copy, e < 4)
  // never cross an 8-row boundary and sit one immediate apart; unpadded, the
  // 8-byte chunk c of copy row rho at chunk c ^ ((rho >> 3) & 3) (W operand,
  // transposed and staging accesses without bank conflicts)
  constexpr int CROWS = AROWS;
  __shared__ __align__(16) E a_lds[2][NB][CROWS][KP];
  __shared__ __align__(16) Op m_tr[WPG][2][2][TrTile1::kSlots];  // [wave][tap of a pair][hi / lo]
  __shared__ float da_lds[2][WPG][NB][16][17];
  auto acol = [](int r, int col) -> int { return (col & 3) | (((col >> 2) ^ ((r >> 3) & 3)) << 2); };

  const E* __restrict__ x = static_cast<const E*>(xv);
  const E* __restrict__ dy = static_cast<const E*>(dyv);
  E* __restrict__ dx = static_cast<E*>(dxv);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int64_t N = seq.n_tokens;
  const int64_t d0 = (static_cast<int64_t>(bx) * WPG + wave) * CW;
  const bool wave_on = d0 < D;
  const int64_t dl = d0 + j;
  const bool ch_ok = wave_on && dl < D;

  // super-blocks [sb_lo, sb_hi) of this range (ranges by < gy1 share the first n_old)
  const int64_t sb_lo = by < gy1 ? static_cast<int64_t>(by) * n_old / gy1
                                 : n_old + static_cast<int64_t>(by - gy1) * (n_total - n_old) / (gy - gy1);
  const int64_t sb_hi = by < gy1 ? static_cast<int64_t>(by + 1) * n_old / gy1
                                 : n_old + static_cast<int64_t>(by + 1 - gy1) * (n_total - n_old) / (gy - gy1);
  const int nsb = static_cast<int>(sb_hi - sb_lo);
  const int64_t first = sb_lo * EOWN;
  const int64_t last_t0 = first + static_cast<int64_t>(nsb - 1) * EOWN;
  const int64_t row_lo = (first - (S - 1) > 0) ? first - (S - 1) : 0;
  const int64_t row_hi = (last_t0 + TB < N) ? last_t0 + TB : N;
  const int64_t a_hi = (last_t0 + AROWS < N) ? last_t0 + AROWS : N;
  const uint32_t rb = static_cast<uint32_t>(D * ESZ);
  const uint32_t col = static_cast<uint32_t>(dl * ESZ);
  const Buf xb(x + row_lo * D, (row_hi - row_lo) * D * ESZ);
  // dy rows dys elements apart (D; 0: one row for all tokens; -1: one element
  // for every token and channel, the expanded gradient of a sum to a scalar).
  // DY1 (dys = -1 in every layer of the launch): the element is read once here,
  // no row loads and no conversions in the loop.  Otherwise a -1 of one layer
  // is served by OR-ing the element's fp32 bits into every converted dy value
  // while the row loads read nothing (no branch in the loop)
  const bool dy_one = DY1 || dys < 0;
  const uint32_t drb = static_cast<uint32_t>((dy_one ? 0 : dys) * ESZ);
  const Buf dyb(dy_one ? dy : dy + row_lo * dys, dy_one ? ESZ : ((row_hi - row_lo - 1) * dys + D) * ESZ);
  uint32_t dy_or = 0;
  if (dy_one) {
    E e;
    dyb.load<ESZ>(0, &e);
    dy_or = ch_ok ? __float_as_uint(bf16_to_f32(e)) : 0u;
  }
  const bool dy_rows = ch_ok && !dy_one;
  const Buf ab(a_c + first * KP, (a_hi - first) * KP * ESZ);
  const Buf bb(b_c, static_cast<int64_t>(KP) * S * D * ESZ);

  // W operands: bop[s] = basis[4 q + v, s, dl] (B operand, column = this lane's channel)
  Op bop[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    E e[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) bb.load<ESZ>(row_off((4 * q + v) * S + s, 0, rb, col, ch_ok), &e[v]);
    bop[s] = CT<true>::make(e[0], e[1], e[2], e[3]);
  }
  // dalpha B operands: bda[s] = basis[j, s, d0 + 4 q + {0..3}] (channels past D,
  // with D % 4 == 2 the last two of the final group, zero: the load reaches into
  // the next row)
  Op bda[S];
  {
    const int64_t ch = d0 + 4 * q;
    const bool on = wave_on && ch < D;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      bb.load<8>(row_off(j * S + s, 0, rb, static_cast<uint32_t>(ch * ESZ), on), &bda[s]);
      if (ch + 2 >= D) {
        bda[s][2] = 0;
        bda[s][3] = 0;
      }
    }
  }
  f32x4 dbacc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) dbacc[s] = f32x4{0.f, 0.f, 0.f, 0.f};

  // raw rows of one super-block: x window (trun - (S-1) .. trun + R - 1), dy rows
  E xr[W], dr[DY1 ? 1 : R];
  auto fetch_xdy = [&](int64_t t0) {
    const uint32_t base = row_off(t0 + R * q - (S - 1), row_lo, rb, col, ch_ok);
#pragma unroll
    for (int w = 0; w < W; ++w) xb.load<ESZ>(base + w * rb, &xr[w]);
    if constexpr (!DY1) {
      const uint32_t dbase = row_off(t0 + R * q, row_lo, drb, col, dy_rows);
#pragma unroll
      for (int r = 0; r < R; ++r) dyb.load<ESZ>(dbase + r * drb, &dr[r]);
    }
  };
  // routing-weight rows of a super-block: AROWS x 16 elements, 8 bytes per thread
  constexpr int ACHUNKS = AROWS * KP / 4;
  static_assert(ACHUNKS <= 64 * WPG, "one routing-weight chunk per thread");
  E arw[4];
  // (the per-lane terms are formed where they are used, from an opaque copy of
  // the thread id: hoisted out of the loop they outgrew the register budget)
  auto opaque_tid = [&]() {
    int t = tid;
    asm volatile("" : "+v"(t));
    return t;
  };
  auto fetch_a = [&](int64_t t0) {
    const int tt = opaque_tid();
    ab.load<8>(row_off(t0 + (tt >> 2), first, KP * ESZ, (tt & 3) * 8, tt < ACHUNKS), arw);
  };
  auto stage_alpha = [&](int buf) {
    const int tt = opaque_tid();
    const int row = tt >> 2, c4 = (tt & 3) * 4;
    if (tt < ACHUNKS) {
      Vec<E, 4>::store(&a_lds[buf][0][row][acol(row, c4)], arw);
      if (row >= 4) Vec<E, 4>::store(&a_lds[buf][1][row - 4][acol(row - 4, c4)], arw);
    }
  };

  if (first < N) {
    fetch_xdy(first);
    fetch_a(first);
    stage_alpha(0);
  }
  __syncthreads();

  StartCursor cursor;
  // dalpha partials of this channel group from row `first` on (rows
  // [first, row_hi), 16 routes; 32-bit offsets within the range)
  const Buf pdab(part_da + (static_cast<int64_t>(bx) * N + first) * KP, (row_hi - first) * KP * 4);
  for (int sb = 0; sb < nsb; ++sb) {
    const int64_t t0 = first + static_cast<int64_t>(sb) * EOWN;
    if (t0 >= N) break;  // uniform over the workgroup
    const int buf = sb & 1;
    const int64_t own_end = (t0 + EOWN < N) ? t0 + EOWN : N;
    // the lane's terms formed here each time (see opaque_tid); they shadow the
    // function-scope ones in the loop body
    const int tl = opaque_tid();
    const int lane = tl & 63;
    const int j = lane & 15, q = lane >> 4;
    const int64_t trun = t0 + R * q;
    const bool more = (sb + 1 < nsb) && (t0 + EOWN < N);

    float xw[W], g[R];
#pragma unroll
    for (int w = 0; w < W; ++w) xw[w] = bf16_to_f32(xr[w]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      g[r] = DY1 ? __uint_as_float(dy_or) : __uint_as_float(__float_as_uint(bf16_to_f32(dr[DY1 ? 0 : r])) | dy_or);
    // the next super-block's routing weights (unconditionally: after the last
    // super-block of the range they fall past the buffer and load zeros, and
    // the rows just converted are dead, so the loop carries no copies)
    fetch_a(t0 + EOWN);

    // alpha operand of token block b shifted by e < 4 rows (row i = j): row
    // r = R (j / 4) + j % 4 + e of copy b, chunk q ^ (r >> 3) = q ^ (j / 4)
    // (j % 4 + e < 8): one lane offset plus immediates
    const char* a_base = reinterpret_cast<const char*>(&a_lds[buf][0][0][0]) +
                         ((R * (j >> 2) + (j & 3)) * KP + ((q ^ (j >> 2)) << 2)) * ESZ;
    auto aop = [&](int e, int b) -> Op {
      return *reinterpret_cast<const Op*>(a_base + ((b * CROWS + e) * KP) * ESZ);
    };

    const int64_t w_lo = t0 - (S - 2), w_hi = t0 + TB + S - 2;
    const bool interior = !cursor.starts_in(seq, w_lo, w_hi);

    f32x4 dacc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) dacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto body = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      // masks of this lane's run extended by S-1 later rows (rows r < R + S - 1),
      // packed in two registers: bit k of `sb` is set when window row
      // trun - (S-1) + k starts a segment, bit r of `rv` when row trun + r is a
      // token (< N); tap s of row r is valid when the row is a token and no
      // segment starts in window rows r + s + 1 .. r + S - 1
      uint32_t sbm = 0, rv = 0;
      if constexpr (MASK) {
        const int64_t u0 = trun - (S - 1);
        for (int64_t st = seq.next_start(w_lo); st <= w_hi && st < N; st = seq.next_start(st + 1)) {
          const int64_t k = st - u0;
          if (k > 0 && k < 32) sbm |= 1u << k;
        }
        const int64_t nrow = N - trun;  // rows r < nrow are tokens
        rv = nrow >= 32 ? ~0u : (nrow <= 0 ? 0u : ((1u << nrow) - 1u));
      }
      auto tap_ok = [&](int r, int s) -> bool {
        if constexpr (MASK) {
          constexpr uint32_t kNone = 0;
          const uint32_t span = ((1u << (S - 1 - s)) - 1u) << (r + s + 1);
          return ((rv >> r) & 1u) && (sbm & span) == kNone;
        } else {
          return true;
        }
      };

      if constexpr (ACT != 0) if (act) {  // (act: uniform; always with a fixed ACT)
        float p[R];
#pragma unroll
        for (int r = 0; r < R; ++r) p[r] = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const f32x4 w4 = mma16(aop(0, b), bop[s], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int r = 4 * b + v;
              if (tap_ok(r, s)) p[r] = fmaf(xw[r + s], w4[v], p[r]);
            }
          }
        // g *= silu'(P) = sg (1 + P (1 - sg)), sg = sigmoid(P) as sigmoid_f forms it
        float sg[R];
#pragma unroll
        for (int r = 0; r < R; ++r) sg[r] = __builtin_amdgcn_exp2f(-p[r] * 1.4426950408889634f);
#pragma unroll
        for (int r = 0; r < R; ++r) sg[r] = __builtin_amdgcn_rcpf(1.0f + sg[r]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float v = fmaf(-sg[r], sg[r], sg[r]);
          g[r] = g[r] * fmaf(p[r], v, sg[r]);
        }
      }

      // dx, taps in descending order (the first need none of the next lane
      // group's rows)
      if (dx != nullptr) {
        float gf[S - 1];
        const int src_lane = (lane + 16) & 63;
#pragma unroll
        for (int e = 0; e < S - 1; ++e) gf[e] = __shfl(g[e], src_lane, 64);
        float dxa[R];
#pragma unroll
        for (int r = 0; r < R; ++r) dxa[r] = 0.f;
#pragma unroll
        for (int si = 0; si < S; ++si) {
          const int s = S - 1 - si, off = S - 1 - s;
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const f32x4 w4 = mma16(aop(off, b), bop[s], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int r = 4 * b + v, src = r + off;
              const float gs = (src < R) ? g[src < R ? src : 0] : gf[src >= R ? src - R : 0];
              if (tap_ok(src, s)) dxa[r] = fmaf(gs, w4[v], dxa[r]);
            }
          }
        }
        // the buffer ends at this super-block's last own row: later rows drop
        const Buf dxb(dx + row_lo * D, (own_end - row_lo) * D * ESZ);
        const uint32_t base = row_off(trun, row_lo, rb, col, ch_ok);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const E o = f32_to_bf16(dxa[r]);
          dxb.store<ESZ>(base + r * rb, &o);
        }
      }

      // alpha^T operands of the dbasis MFMA, own rows only:
      // at[b] = alpha[trun + 4 b + v, j] (transposed read of the staged rows)
      Op at[NB];
      {
        const int own_rows = static_cast<int>(own_end - t0);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          uint64_t keep;
          if (own_rows == EOWN) {
            // (uniform) every super-block but the token axis's last: rows
            // R q + 4 b + v < EOWN hold for all but the last block of group 3,
            // which keeps its first EOWN - (TB - 4) rows
            keep = (b == NB - 1 && q == 3) ? ((1ull << (16 * (EOWN - (TB - 4)))) - 1ull) : ~0ull;
          } else {
            const int n_ok = min(max(own_rows - (R * q + 4 * b), 0), 4);
            keep = n_ok >= 4 ? ~0ull : ((1ull << (16 * n_ok)) - 1ull);
          }
          const int r = R * q + 4 * b + (j >> 2);
          const Op v = TrTile<NB, 2>::read(&a_lds[buf][0][r][acol(r, 4 * (j & 3))]);
          at[b] = __builtin_bit_cast(Op, __builtin_bit_cast(uint64_t, v) & keep);
        }
      }
      // m of tap s -> hi / lo operands -> this wave's tile slot p, dbasis MFMAs
      auto stage_m = [&](int s, int p) {
        Op mh[NB], ml[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          uint32_t hbits[4];
          float lo[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 4 * b + v;
            const float mval = tap_ok(r, s) ? g[r] * xw[r + s] : 0.f;
            hbits[v] = __float_as_uint(mval) & 0xffff0000u;
            lo[v] = mval - __uint_as_float(hbits[v]);
          }
          mh[b] = pack4_hi(hbits[0], hbits[1], hbits[2], hbits[3]);
          ml[b] = pack4_bf16(lo[0], lo[1], lo[2], lo[3]);
          m_tr[wave][p][0][TrTile1::wslot(j, q, b)] = mh[b];
          m_tr[wave][p][1][TrTile1::wslot(j, q, b)] = ml[b];
        }
        dbacc[s] = mma32(mh[0], mh[1], at[0], at[1], dbacc[s]);
        dbacc[s] = mma32(ml[0], ml[1], at[0], at[1], dbacc[s]);
      };
      // transposed reads of tile slot p: ra[rb][h] = m[16 rb + i][4 qq + {0..3}]
      auto read_m = [&](int p, Op (&ra)[NB][2]) {
#pragma unroll
        for (int r2 = 0; r2 < NB; ++r2)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            ra[r2][h] = TrTile<NB, 2>::read(&m_tr[wave][p][h][TrTile1::rslot(j, q, r2)]);
      };
      // tap pairs (s, s + 1): dalpha contracts (tap, 16 channels) pairs in one
      // 16x16x32 MFMA; an odd last tap alone in a 16x16x16 one.  The reads of a
      // pair are issued before the next pair's m values are formed and written
      // (a wave's LDS operations complete in issue order, so one tile serves).
      constexpr int NPAIR = (S + 1) / 2;
      Op ra0[NB][2], ra1[NB][2];
#pragma unroll
      for (int pi = 0; pi < NPAIR; ++pi) {
        const int s0 = 2 * pi;
        const bool two = s0 + 1 < S;
        if (pi == 0) {
          stage_m(s0, 0);
          if (two) stage_m(s0 + 1, 1);
        }
        wave_lds_sync();
        read_m(0, ra0);
        if (two) read_m(1, ra1);
        __builtin_amdgcn_sched_barrier(0);
        if (pi + 1 < NPAIR) {
          stage_m(s0 + 2, 0);
          if (s0 + 3 < S) stage_m(s0 + 3, 1);
        }
#pragma unroll
        for (int r2 = 0; r2 < NB; ++r2)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if (two) dacc[r2] = mma32(ra0[r2][h], ra1[r2][h], bda[s0], bda[two ? s0 + 1 : s0], dacc[r2]);
            else dacc[r2] = mma16(ra0[r2][h], bda[s0], dacc[r2]);
          }
      }
      wave_lds_sync();
    };
    if (interior) body(std::false_type{});
    else body(std::true_type{});
    // the next super-block's rows, into the registers the raw rows left
    // (unconditionally, as fetch_a above); issued after the m products, where
    // the fewest registers are live, and covered by the other waves of the SIMD
    fetch_xdy(t0 + EOWN);

#pragma unroll
    for (int r2 = 0; r2 < NB; ++r2)
#pragma unroll
      for (int v = 0; v < 4; ++v) da_lds[buf][wave][r2][4 * q + v][j] = dacc[r2][v];
    if (more) stage_alpha(buf ^ 1);
    __syncthreads();
    // sum the 8 waves' dalpha tiles in wave order; own rows only
    {
      const int r2 = tl >> 8, row = (tl >> 4) & 15, c = tl & 15;
      float tv[WPG];
#pragma unroll
      for (int w = 0; w < WPG; ++w) tv[w] = da_lds[buf][w][r2][row][c];
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) sum += tv[w];
      const int n_own = static_cast<int>(own_end - t0);
      const uint32_t off = static_cast<uint32_t>(((t0 - first + 16 * r2 + row) * KP + c) * 4);
      pdab.store<4>(16 * r2 + row < n_own ? off : kOffNone, &sum);
    }
  }

  // this workgroup's dbasis partial: dbacc[s][v] is (k = j, s, channel d0 + 4 q + v);
  // with D % 4 == 2 the rows are 8-byte aligned and the last group of 4 half past D
  if (wave_on && d0 + 4 * q < D) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float* dst = part_db + ((static_cast<int64_t>(by) * KP + j) * S + s) * D + d0 + 4 * q;
      if (D % 4 == 0) {
        *reinterpret_cast<f32x4*>(dst) = dbacc[s];
      } else {
        *reinterpret_cast<f32x2*>(dst) = f32x2{dbacc[s][0], dbacc[s][1]};
        if (d0 + 4 * q + 2 < D) *reinterpret_cast<f32x2*>(dst + 2) = f32x2{dbacc[s][2], dbacc[s][3]};
      }
    }
  }
}

template <int S, bool ACT, bool DY1>
__global__ void __launch_bounds__(64 * kLeanWPG) __attribute__((amdgpu_waves_per_eu(MOC_LEAN_WAVES)))
bwd_lean_kernel(const void* __restrict__ xv, const void* __restrict__ dyv, int64_t dys,
                const uint16_t* __restrict__ a_c, const uint16_t* __restrict__ b_c,
                void* __restrict__ dxv, float* __restrict__ part_da, float* __restrict__ part_db,
                SeqLayout seq, int64_t D, int gy, int gy1, int n_old, int n_total) {
  bwd_lean_tile<S, ACT, DY1>(xv, dyv, dys, a_c, b_c, dxv, part_da, part_db, seq, D,
                        static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y), gy, gy1, n_old,
                        n_total);
}

// Several layers in one launch (1-D grid, the layers' grids one after another,
// as bwd_layers_kernel maps them), so that a grouped launch returns the
// per-layer calls' results bit for bit.
template <int S, int ACT, bool DY1>
__global__ void __launch_bounds__(64 * kLeanWPG) __attribute__((amdgpu_waves_per_eu(MOC_LEAN_WAVES)))
bwd_lean_layers_kernel(BwdLayers ly, SeqLayout seq) {
  const int blk = static_cast<int>(blockIdx.x);
  const BwdLayer* Lp = &ly.l[layer_index(ly, blk)];
  int local = blk - Lp->blk0, row = 0;
  const int gxl = Lp->gx;
  while (local >= gxl) {  // scalar: local < gx gy, at most gy - 1 steps
    local -= gxl;
    ++row;
  }
  bwd_lean_tile<S, ACT, DY1>(Lp->x, Lp->dy, Lp->dys, static_cast<const uint16_t*>(Lp->a),
                        static_cast<const uint16_t*>(Lp->b), Lp->dx, Lp->part_da, Lp->part_db, seq,
                        Lp->D, local, row, Lp->gy, Lp->gy1, Lp->n_old, Lp->n_total, Lp->act != 0);
}

}  // namespace mfma
}  // namespace moc
