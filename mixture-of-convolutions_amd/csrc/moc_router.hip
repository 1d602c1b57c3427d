// Router GEMMs of the MoC layer (moc/api.py:383-388 of the reference: logits =
// F.linear(z, router) and its autograd): logits = z . router^T, and in the
// backward dz = dlogits . router and drouter = dlogits^T . z.
//
// All three products have the K (<= 32) routes on one side and the [N, Z]
// routing input on the other, so they are bound by streaming z (or writing dz)
// through HBM once.  The kernels read and write [N, Z] with 16-byte accesses and
// run the products on the matrix cores (v_mfma_f32_16x16x32_bf16, 16x16x16 for
// dz with K = 16); accumulation is fp32, results are rounded to bf16 once.
// drouter is reduced in a fixed order (per-range partials, then one sum), so it
// is bitwise reproducible.  bf16 data only; K % 4 == 0, K <= 96 (the fused
// activation K <= 32), Z % 64 == 0.

#include "moc_kernels.h"
#include "moc_mfma.h"

namespace moc {
namespace router {

using mfma::Buf;
using mfma::f32x4;
using mfma::kOffNone;
using mfma::s16x4;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 load16(const Buf& b, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(b.r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ u32x2 load8(const Buf& b, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(b.r, static_cast<int>(off), 0, 0);
}

// Wave index, known to the compiler as uniform over the wave (so that loops
// and branches on it compile as scalar control flow, not exec-masked).
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// 16 x 16 x 32 product of 8-element bf16 operands held as 16 bytes.
__device__ __forceinline__ f32x4 mma8(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Transposed LDS read (ds_read_b64_tr_b16): lane i of each 16-lane group gets
// element i % 4 of the 8-byte rows read by lanes i / 4 + {0, 4, 8, 12}.
__device__ __forceinline__ s16x4 tr_read(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<void*>(p)));
}

// ---------------------------------------------------------------------------
// logits[t, k] = sum_z z[t, z] router[k, z].  Workgroup: 32 tokens (two blocks
// of 16), 4 waves.  Wave w sums the 64-wide z chunks c = w, w + 4, ...: lane
// (i, qq) loads columns 64 c + 8 qq + [0, 8) and 64 c + 32 + 8 qq + [0, 8) of
// tokens t0 + i, t0 + 16 + i (A operands) and of route 16 kc + i (B operands),
// so that each load instruction reads 64 contiguous bytes per row and the
// router operands serve both token blocks.  The 4 partial tiles are summed in
// LDS in wave order.
// Chunks whose loads are issued together: four up to 32 routes, fewer above
// (the router operands of a chunk take 8 KC registers per lane).
template <int KC>
constexpr int kFwdBatch = KC <= 2 ? 4 : (KC <= 4 ? 2 : 1);

// Weights of one token of a route group from its bf16 logits l[0, kn): the
// softmax sum in the order of router_fwd_kernel's lane tree over KPg = 16 or
// 32 lanes (pairs k ^ 16, then k ^ 8, k ^ 4, k ^ 2, k ^ 1), so that a group
// gets the weights a single router of kn routes gets, bit for bit.
__device__ __forceinline__ void route_group(float (&l)[32], int kn, int routing) {
  if (routing == ROUTE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (k < kn) m = fmaxf(m, l[k]);
    float e[32], sm[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      e[k] = (k < kn) ? __expf(l[k] - m) : 0.f;
      sm[k] = e[k];
    }
    if (kn > 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) sm[k] = sm[k] + sm[k + 16];
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1)
#pragma unroll
      for (int k = 0; k < o; ++k) sm[k] = sm[k] + sm[k + o];
    const float inv = 1.0f / sm[0];
#pragma unroll
    for (int k = 0; k < 32; ++k) l[k] = round_to(e[k] * inv, DT_BF16);
  } else if (routing == ROUTE_EXP) {
#pragma unroll
    for (int k = 0; k < 32; ++k) l[k] = round_to(__expf(l[k]), DT_BF16);
  }
}

template <int KC, bool GROUPED>
__global__ void __launch_bounds__(256) router_fwd_kernel(const uint16_t* __restrict__ z,
                                                         const uint16_t* __restrict__ r,
                                                         uint16_t* __restrict__ logits,
                                                         int64_t N, int Z, int K, int routing,
                                                         RouteGroups grp) {
  constexpr int KP = 16 * KC;
  constexpr int UB = kFwdBatch<KC>;
  __shared__ float red[4][2][KP][17];
  const int lane = threadIdx.x & 63, w = wave_id();
  const int i = lane & 15, qq = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t rows = (N - t0 < 32) ? N - t0 : 32;
  // rows past N and routes past K lie outside the buffers and load zeros
  const Buf zb(z + t0 * Z, rows * Z * 2);
  const Buf rb(r, static_cast<int64_t>(K) * Z * 2);
  f32x4 acc[2][KC];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) acc[h][kc] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nchunk = Z / 64;
  // UB chunks per round (4 + 2 KC loads per chunk and lane).  Above 32 routes
  // (rounds of one or two chunks) two rounds are in flight: the loads of round
  // r + 1 are issued before the MFMAs of round r (two register sets, the loop
  // unrolled by two so that neither is copied; grouped router of configs[4]:
  // 89 -> 81 us).  Chunks past the row end load zeros instead of branching.
  typedef u32x4 ZOps[UB][2][2];
  typedef u32x4 ROps[UB][KC][2];
  auto load_round = [&](int c0, ZOps& za, ROps& ra) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int c = c0 + 4 * u;
      const bool on = c < nchunk;
      const uint32_t col0 = static_cast<uint32_t>((64 * c + 8 * qq) * 2), col1 = col0 + 64;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t zrow = static_cast<uint32_t>((16 * h + i) * Z * 2);
        za[u][h][0] = load16(zb, on ? zrow + col0 : kOffNone);
        za[u][h][1] = load16(zb, on ? zrow + col1 : kOffNone);
      }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const uint32_t rrow = static_cast<uint32_t>((16 * kc + i) * Z * 2);
        ra[u][kc][0] = load16(rb, on ? rrow + col0 : kOffNone);
        ra[u][kc][1] = load16(rb, on ? rrow + col1 : kOffNone);
      }
    }
  };
  auto mma_round = [&](const ZOps& za, const ROps& ra) {
#pragma unroll
    for (int u = 0; u < UB; ++u)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[h][kc] = mma8(za[u][h][0], ra[u][kc][0], acc[h][kc]);
          acc[h][kc] = mma8(za[u][h][1], ra[u][kc][1], acc[h][kc]);
        }
  };
  constexpr int kRound = 4 * UB;  // chunks between a wave's rounds
  ZOps zA, zB;
  ROps rA, rB;
  if constexpr (UB >= 4) {
    // up to 32 routes: rounds of four chunks, one in flight (measured faster
    // than two, whose registers cost the second workgroup on a SIMD its slot)
    for (int c0 = w; c0 < nchunk; c0 += kRound) {
      load_round(c0, zA, rA);
      mma_round(zA, rA);
    }
  } else {
    int c0 = w;
    if (c0 < nchunk) load_round(c0, zA, rA);
    while (c0 < nchunk) {
      load_round(c0 + kRound, zB, rB);
      mma_round(zA, rA);
      c0 += kRound;
      if (c0 >= nchunk) break;
      load_round(c0 + kRound, zA, rA);
      mma_round(zB, rB);
      c0 += kRound;
    }
  }
  // D lane (j, q): route 16 kc + j, tokens 16 h + 4 q + v
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[w][h][16 * kc + i][4 * qq + v] = acc[h][kc][v];
  __syncthreads();
  if constexpr (GROUPED) {
    // route groups: one thread per (group, token) forms the group's weights
    for (int idx = threadIdx.x; idx < 32 * grp.n; idx += 256) {
      const int tok = idx & 31, gi = idx >> 5, h = tok >> 4, tr = tok & 15;
      if (tok >= rows) continue;
      const int k0 = grp.k0[gi], kn = grp.kn[gi];
      float l[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const int kk = k0 + ((k < kn) ? k : 0);
        const float sm =
            ((red[0][h][kk][tr] + red[1][h][kk][tr]) + red[2][h][kk][tr]) + red[3][h][kk][tr];
        l[k] = round_to(sm, DT_BF16);
      }
      route_group(l, kn, grp.routing[gi]);
      // kn % 4 == 0: 8-byte stores
      uint2* o = reinterpret_cast<uint2*>(grp.out[gi] + (t0 + tok) * kn);
#pragma unroll
      for (int k = 0; k < 32; k += 4)
        if (k < kn)
          o[k / 4] = make_uint2(static_cast<uint32_t>(f32_to_bf16(l[k])) |
                                    (static_cast<uint32_t>(f32_to_bf16(l[k + 1])) << 16),
                                static_cast<uint32_t>(f32_to_bf16(l[k + 2])) |
                                    (static_cast<uint32_t>(f32_to_bf16(l[k + 3])) << 16));
    }
    return;
  }
  // KP consecutive lanes hold one token's routes; every lane runs every pass
  // (the shuffles of the routing need all of them; routing needs KC <= 2)
#pragma unroll
  for (int pass = 0; pass < 32 * KP / 256; ++pass) {
    const int idx = threadIdx.x + 256 * pass;
    const int tok = idx / KP, k = idx % KP, h = tok >> 4, tr = tok & 15;
    const float s = ((red[0][h][k][tr] + red[1][h][k][tr]) + red[2][h][k][tr]) + red[3][h][k][tr];
    float v = round_to(s, DT_BF16);
    if (KC <= 2 && routing == ROUTE_SOFTMAX) {
      // softmax of the bf16 logits over the token's KP lanes (routes >= K
      // excluded), rounded to bf16
      const float l = (k < K) ? v : -INFINITY;
      float m = l;
#pragma unroll
      for (int o = KP / 2; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      const float e = (k < K) ? __expf(l - m) : 0.f;
      float sum = e;
#pragma unroll
      for (int o = KP / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      v = round_to(e * (1.0f / sum), DT_BF16);
    } else if (KC <= 2 && routing == ROUTE_EXP) {
      v = round_to(__expf(v), DT_BF16);
    }
    if (k < K && tok < rows) logits[(t0 + tok) * K + k] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// dz[t, zc] = sum_k dl[t, k] router[k, zc].  A wave owns 64 columns and kDzBlocks
// blocks of 16 tokens.  D[zc][t] = router^T . dl^T with A lane (i, qq) holding
// router[16 kc + 4 qq + {0..3}][zc] (kept in registers) and B lane (j, qq)
// holding dl[t_j][16 kc + 4 qq + {0..3}].  Row r = 4 q + v of tile tl stands for
// column zs + zcol(tl, r), zcol = 32 (tl >> 1) + 8 q + 4 (tl & 1) + v, so that
// the result lane (j, q) holds columns 8 q + {0..7} (tiles 0, 1) and
// 32 + 8 q + {0..7} (tiles 2, 3) of token t_j: two 16-byte stores, and each
// store instruction writes 64 contiguous bytes of every token row.
// token blocks per wave: 8 up to 32 routes, 16 above (the router operands,
// 4 KC gathered loads per lane, are loaded once per wave; the dl operands one
// block ahead)
template <int KC>
constexpr int kDzBlocks = KC <= 2 ? 8 : 16;

__device__ __forceinline__ int dz_col(int tl, int r) {
  return 32 * (tl >> 1) + 8 * (r >> 2) + 4 * (tl & 1) + (r & 3);
}

// One 16 x 16 tile of router^T . dl^T over KC route chunks.  One route chunk:
// a 16x16x16 MFMA.  More: chunk pairs in 16x16x32 MFMAs, an odd last chunk
// paired with zeros, so that the accumulator chain never mixes MFMA shapes (a
// 16x16x16 accumulating onto a 16x16x32 result gave wrong rows here).
template <int KC>
__device__ __forceinline__ f32x4 dz_tile(const s16x4 (&a)[KC], const s16x4 (&b)[KC]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (KC == 1) {
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a[0], b[0], acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int kc = 0; kc + 1 < KC; kc += 2)
      acc = mfma::mma32(a[kc], a[kc + 1], b[kc], b[kc + 1], acc);
    if constexpr (KC % 2 == 1) {
      const s16x4 zero = {0, 0, 0, 0};
      acc = mfma::mma32(a[KC - 1], zero, b[KC - 1], zero, acc);
    }
  }
  return acc;
}

template <int KC>
__global__ void __launch_bounds__(256) router_dz_kernel(const uint16_t* __restrict__ dl,
                                                        const uint16_t* __restrict__ r,
                                                        uint16_t* __restrict__ dz, int64_t N,
                                                        int Z, int K) {
  const int lane = threadIdx.x & 63, w = wave_id();
  const int i = lane & 15, qq = lane >> 4;
  const int zs = (blockIdx.x * 4 + w) * 64;
  if (zs >= Z) return;  // whole wave; the kernel has no barrier
  const Buf rb(r, static_cast<int64_t>(K) * Z * 2);
  const Buf db(dl, N * K * 2);
  const Buf ob(dz, N * Z * 2);
  constexpr int NBLK = kDzBlocks<KC>;
  const int64_t tb = static_cast<int64_t>(blockIdx.y) * NBLK * 16;
  // B operands (dl) of block b, rows past N load zeros: block 0 now, each
  // next block while the current one is multiplied
  auto load_b = [&](s16x4 (&bo)[KC], int b) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = 16 * kc + 4 * qq;
      const int64_t t = tb + 16 * b + i;
      const uint32_t off = (k < K) ? static_cast<uint32_t>((t * K + k) * 2) : kOffNone;
      bo[kc] = __builtin_bit_cast(s16x4, load8(db, off));
    }
  };
  s16x4 bop[2][KC];
  load_b(bop[0], 0);
  s16x4 aop[4][KC];
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      uint16_t e[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        const uint32_t off = static_cast<uint32_t>((k * Z + zs + dz_col(tl, i)) * 2);
        e[v] = __builtin_amdgcn_raw_buffer_load_b16(rb.r, static_cast<int>(off), 0, 0);
      }
      aop[tl][kc] = s16x4{static_cast<short>(e[0]), static_cast<short>(e[1]),
                          static_cast<short>(e[2]), static_cast<short>(e[3])};
    }
#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + 1 < NBLK) load_b(bop[(b + 1) & 1], b + 1);
    const int64_t t = tb + 16 * b + i;
    f32x4 acc[4];
#pragma unroll
    for (int tl = 0; tl < 4; ++tl) acc[tl] = dz_tile<KC>(aop[tl], bop[b & 1]);
    // rows past N lie outside the buffer: their stores are dropped
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f32x4 a0 = acc[2 * half], a1 = acc[2 * half + 1];
      const u32x4 pk = {mfma::pack2_bf16(a0[0], a0[1]), mfma::pack2_bf16(a0[2], a0[3]),
                        mfma::pack2_bf16(a1[0], a1[1]), mfma::pack2_bf16(a1[2], a1[3])};
      const uint32_t off = static_cast<uint32_t>((t * Z + zs + 32 * half + 8 * qq) * 2);
      __builtin_amdgcn_raw_buffer_store_b128(pk, ob.r, static_cast<int>(off), 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Partial drouter over a token range: D[k][zc] = sum_t dl[t][k] z[t][zc].
// Workgroup: 64 columns and one token range, 4 waves taking 32-token blocks in
// turn.  Each block of z (32 x 64) and of dl (32 x KP) is loaded with 16- and
// 8-byte accesses into a wave-private LDS tile and read back transposed: A lane
// (i, qq) = dl[8 qq + {0..7}][16 kc + i], B lane (j, qq) = z[8 qq + {0..7}][16 tl
// + j].  The waves' tiles are summed in LDS in wave order and written as
// part[range][k][zc] (fp32).
constexpr int kZRow = 64 + 8;   // padded LDS row of a z tile (bf16)

template <int KC>
__global__ void __launch_bounds__(256) router_dr_kernel(const uint16_t* __restrict__ dl,
                                                        const uint16_t* __restrict__ z,
                                                        float* __restrict__ part, int64_t N,
                                                        int Z, int K, int blocks_per_range) {
  constexpr int KP = 16 * KC;
  constexpr int KROW = KP + 4;  // padded LDS row of a dl tile (bf16)
  __shared__ __align__(16) uint16_t zt[4][32][kZRow];
  __shared__ __align__(16) uint16_t dt[4][32][KROW];
  __shared__ float red[KP][65];
  const int lane = threadIdx.x & 63, w = wave_id();
  const int i = lane & 15, qq = lane >> 4;
  const int zs = blockIdx.x * 64;
  const Buf zb(z, N * Z * 2);
  const Buf db(dl, N * K * 2);
  f32x4 acc[4][KC];
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) acc[tl][kc] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t blk0 = static_cast<int64_t>(blockIdx.y) * blocks_per_range;
  // registers of one block: z rows t0 + lane / 8 + 8 ld, columns zs + 8 (lane % 8)
  // .. + 7; dl rows of the block in KP / 4 chunks of 4 routes.  Two register
  // sets: the loads of blocks b + 4 and b + 8 are in flight while block b is
  // multiplied.  Blocks past the range or past N load zeros (no branches).
  struct Regs {
    u32x4 z[4];
    u32x2 d[KP / 8];
  };
  auto load_block = [&](Regs& rg, int bb) {
    const int64_t t0 = (blk0 + bb) * 32;
    const bool on = bb < blocks_per_range && t0 < N;
#pragma unroll
    for (int ld = 0; ld < 4; ++ld) {
      const int row = lane / 8 + 8 * ld;
      rg.z[ld] = load16(zb, on ? static_cast<uint32_t>(((t0 + row) * Z + zs + 8 * (lane % 8)) * 2)
                               : kOffNone);
    }
#pragma unroll
    for (int ld = 0; ld < KP / 8; ++ld) {
      const int chunk = lane + 64 * ld;
      const int row = chunk / (KP / 4), k = 4 * (chunk % (KP / 4));
      rg.d[ld] = load8(db, (on && k < K) ? static_cast<uint32_t>(((t0 + row) * K + k) * 2) : kOffNone);
    }
  };
  auto mult_block = [&](const Regs& rg) {
#pragma unroll
    for (int ld = 0; ld < 4; ++ld)
      *reinterpret_cast<u32x4*>(&zt[w][lane / 8 + 8 * ld][8 * (lane % 8)]) = rg.z[ld];
#pragma unroll
    for (int ld = 0; ld < KP / 8; ++ld) {
      const int chunk = lane + 64 * ld;
      *reinterpret_cast<u32x2*>(&dt[w][chunk / (KP / 4)][4 * (chunk % (KP / 4))]) = rg.d[ld];
    }
    mfma::wave_lds_sync();
    // supplier lane 4 e + a of group qq reads row 8 qq + 4 h + e, columns 4 a..
    const int e = i >> 2, a = i & 3;
    s16x4 bz[4][2], ad[KC][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 8 * qq + 4 * h + e;
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) bz[tl][h] = tr_read(&zt[w][row][16 * tl + 4 * a]);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) ad[kc][h] = tr_read(&dt[w][row][16 * kc + 4 * a]);
    }
#pragma unroll
    for (int tl = 0; tl < 4; ++tl)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc[tl][kc] = mfma::mma32(ad[kc][0], ad[kc][1], bz[tl][0], bz[tl][1], acc[tl][kc]);
    mfma::wave_lds_sync();
  };
  // the wave's blocks are w, w + 4, ...: nb of them; straight-line loop body
  // (single exit, so both sets stay in flight across the back edge), one
  // block left over runs after it
  const int nb = (blocks_per_range - w + 3) / 4;
  Regs ra, rb2;
  load_block(ra, w);
  load_block(rb2, w + 4);
  int it = 0;
  for (; it + 2 <= nb; it += 2) {  // per wave; no barrier inside
    const int b = w + 4 * it;
    mult_block(ra);
    load_block(ra, b + 8);
    mult_block(rb2);
    load_block(rb2, b + 12);
  }
  if (it < nb) mult_block(ra);
  // D lane (j, q): column 16 tl + j, routes 16 kc + 4 q + v.  The waves' tiles
  // are summed in wave order, ((w0 + w1) + w2) + w3, one wave at a time.
#pragma unroll
  for (int ww = 0; ww < 4; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int tl = 0; tl < 4; ++tl)
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float& cell = red[16 * kc + 4 * qq + v][16 * tl + i];
            cell = (ww == 0) ? acc[tl][kc][v] : cell + acc[tl][kc][v];
          }
    }
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < K * 64; idx += 256) {
    const int k = idx / 64, col = idx % 64;
    part[(static_cast<int64_t>(blockIdx.y) * K + k) * Z + zs + col] = red[k][col];
  }
}

// dz and the partial drouter in one pass (both requested): the workgroup of
// router_dr_kernel (64 columns, one token range, 4 waves taking 32-token blocks
// in turn, the same block order, so the partials are the same bit for bit)
// also writes dz for its columns and tokens, D[zc][t] = router^T . dl^T as in
// router_dz_kernel, with the dl B operands read from the block's LDS tile.
// Three blocks' loads are in flight per wave.
template <int KC>
__global__ void __launch_bounds__(256) router_bwd_kernel(const uint16_t* __restrict__ dl,
                                                         const uint16_t* __restrict__ z,
                                                         const uint16_t* __restrict__ r,
                                                         uint16_t* __restrict__ dz,
                                                         float* __restrict__ part, int64_t N,
                                                         int Z, int K, int blocks_per_range) {
  constexpr int KP = 16 * KC;
  constexpr int KROW = KP + 4;  // padded LDS row of a dl tile (bf16)
  __shared__ __align__(16) uint16_t zt[4][32][kZRow];
  __shared__ __align__(16) uint16_t dt[4][32][KROW];
  __shared__ float red[4][KP][65];
  const int lane = threadIdx.x & 63, w = wave_id();
  const int i = lane & 15, qq = lane >> 4;
  const int zs = blockIdx.x * 64;
  const Buf zb(z, N * Z * 2);
  const Buf db(dl, N * K * 2);
  const Buf rb(r, static_cast<int64_t>(K) * Z * 2);
  const Buf ob(dz, N * Z * 2);
  f32x4 acc[4][KC];
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) acc[tl][kc] = f32x4{0.f, 0.f, 0.f, 0.f};
  // dz A operands: router[16 kc + 4 qq + v][zs + dz_col(tl, i)] (routes >= K load 0)
  s16x4 aop[4][KC];
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      uint16_t e[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        const uint32_t off = static_cast<uint32_t>((k * Z + zs + dz_col(tl, i)) * 2);
        e[v] = __builtin_amdgcn_raw_buffer_load_b16(rb.r, static_cast<int>(off), 0, 0);
      }
      aop[tl][kc] = s16x4{static_cast<short>(e[0]), static_cast<short>(e[1]),
                          static_cast<short>(e[2]), static_cast<short>(e[3])};
    }

  const int64_t blk0 = static_cast<int64_t>(blockIdx.y) * blocks_per_range;
  struct Regs {
    u32x4 z[4];
    u32x2 d[KP / 8];
  };
  // as router_dr_kernel: blocks past the range or past N load zeros
  auto load_block = [&](Regs& rg, int bb) {
    const int64_t t0 = (blk0 + bb) * 32;
    const bool on = bb < blocks_per_range && t0 < N;
#pragma unroll
    for (int ld = 0; ld < 4; ++ld) {
      const int row = lane / 8 + 8 * ld;
      rg.z[ld] = load16(zb, on ? static_cast<uint32_t>(((t0 + row) * Z + zs + 8 * (lane % 8)) * 2)
                               : kOffNone);
    }
#pragma unroll
    for (int ld = 0; ld < KP / 8; ++ld) {
      const int chunk = lane + 64 * ld;
      const int row = chunk / (KP / 4), k = 4 * (chunk % (KP / 4));
      rg.d[ld] = load8(db, (on && k < K) ? static_cast<uint32_t>(((t0 + row) * K + k) * 2) : kOffNone);
    }
  };
  // block bb is in the range; rows past N are dropped by the dz buffer's bound
  auto mult_block = [&](const Regs& rg, int bb) {
#pragma unroll
    for (int ld = 0; ld < 4; ++ld)
      *reinterpret_cast<u32x4*>(&zt[w][lane / 8 + 8 * ld][8 * (lane % 8)]) = rg.z[ld];
#pragma unroll
    for (int ld = 0; ld < KP / 8; ++ld) {
      const int chunk = lane + 64 * ld;
      *reinterpret_cast<u32x2*>(&dt[w][chunk / (KP / 4)][4 * (chunk % (KP / 4))]) = rg.d[ld];
    }
    mfma::wave_lds_sync();
    const int e = i >> 2, a = i & 3;
    s16x4 bz[4][2], ad[KC][2], bd[2][KC];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 8 * qq + 4 * h + e;
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) bz[tl][h] = tr_read(&zt[w][row][16 * tl + 4 * a]);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) ad[kc][h] = tr_read(&dt[w][row][16 * kc + 4 * a]);
    }
    // dz B operands: dl[t0 + 16 hb + i][16 kc + 4 qq + {0..3}]
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        bd[hb][kc] = *reinterpret_cast<const s16x4*>(&dt[w][16 * hb + i][16 * kc + 4 * qq]);
#pragma unroll
    for (int tl = 0; tl < 4; ++tl)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc[tl][kc] = mfma::mma32(ad[kc][0], ad[kc][1], bz[tl][0], bz[tl][1], acc[tl][kc]);
    const int64_t t0 = (blk0 + bb) * 32;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      f32x4 o[4];
#pragma unroll
      for (int tl = 0; tl < 4; ++tl) o[tl] = dz_tile<KC>(aop[tl], bd[hb]);
      const int64_t t = t0 + 16 * hb + i;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const f32x4 a0 = o[2 * half], a1 = o[2 * half + 1];
        const u32x4 pk = {mfma::pack2_bf16(a0[0], a0[1]), mfma::pack2_bf16(a0[2], a0[3]),
                          mfma::pack2_bf16(a1[0], a1[1]), mfma::pack2_bf16(a1[2], a1[3])};
        const uint32_t off = static_cast<uint32_t>((t * Z + zs + 32 * half + 8 * qq) * 2);
        __builtin_amdgcn_raw_buffer_store_b128(pk, ob.r, static_cast<int>(off), 0, 0);
      }
    }
    mfma::wave_lds_sync();
  };
  // the wave's blocks are w, w + 4, ...: nb of them.  The loop body is
  // straight-line (three blocks, each set reloaded right after use) and the
  // zero to two blocks left run after it, so the loop has a single exit and
  // the three sets stay in flight across its back edge.
  const int nb = (blocks_per_range - w + 3) / 4;
  Regs r0, r1, r2;
  load_block(r0, w);
  load_block(r1, w + 4);
  load_block(r2, w + 8);
  int it = 0;
  for (; it + 3 <= nb; it += 3) {  // per wave; no barrier inside
    const int b = w + 4 * it;
    mult_block(r0, b);
    load_block(r0, b + 12);
    mult_block(r1, b + 4);
    load_block(r1, b + 16);
    mult_block(r2, b + 8);
    load_block(r2, b + 20);
  }
  if (it < nb) mult_block(r0, w + 4 * it);
  if (it + 1 < nb) mult_block(r1, w + 4 * it + 4);
#pragma unroll
  for (int tl = 0; tl < 4; ++tl)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[w][16 * kc + 4 * qq + v][16 * tl + i] = acc[tl][kc][v];
  __syncthreads();
  for (int idx = threadIdx.x; idx < K * 64; idx += 256) {
    const int k = idx / 64, col = idx % 64;
    const float sm = ((red[0][k][col] + red[1][k][col]) + red[2][k][col]) + red[3][k][col];
    part[(static_cast<int64_t>(blockIdx.y) * K + k) * Z + zs + col] = sm;
  }
}

// drouter[k, zc] = sum over ranges of part[range][k][zc], in range order.
__global__ void __launch_bounds__(256) router_dr_reduce_kernel(const float* __restrict__ part,
                                                               uint16_t* __restrict__ dr,
                                                               int64_t KZ, int n_ranges) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= KZ) return;
  // loads four at a time, sums in range order
  float s = 0.f;
  int p = 0;
  for (; p + 4 <= n_ranges; p += 4) {
    const float a = part[p * KZ + idx], b = part[(p + 1) * KZ + idx];
    const float c = part[(p + 2) * KZ + idx], d = part[(p + 3) * KZ + idx];
    s += a;
    s += b;
    s += c;
    s += d;
  }
  for (; p < n_ranges; ++p) s += part[p * KZ + idx];
  dr[idx] = f32_to_bf16(s);
}

// ---------------------------------------------------------------------------
// host side

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct BwdPlan {
  int64_t ranges, blocks_per_range;
};

#ifndef MOC_RB_TARGET_WG
#define MOC_RB_TARGET_WG 512
#endif

BwdPlan bwd_plan(int64_t N, int64_t Z) {
  const int64_t nblk = cdiv(N, 32);
  const int64_t slices = Z / 64;
  int64_t ranges = cdiv(MOC_RB_TARGET_WG, slices);  // about MOC_RB_TARGET_WG workgroups
  if (ranges > cdiv(nblk, 4)) ranges = cdiv(nblk, 4);
  if (ranges < 1) ranges = 1;
  const int64_t bpr = cdiv(nblk, ranges);
  return BwdPlan{cdiv(nblk, bpr), bpr};
}

}  // namespace router

bool router_supported(int64_t N, int64_t Z, int64_t K, int dt) {
  // buffer resources address [N, Z] bf16 with 32-bit byte offsets; the dz grid
  // (N / 64 token blocks at most) stays within the 65535 limit of grid.y
  return dt == DT_BF16 && K > 0 && K <= kRouterMaxK && K % 4 == 0 && Z >= 64 && Z % 64 == 0 &&
         N > 0 && N * Z * 2 < (int64_t(1) << 31) && N <= int64_t(65535) * 64;
}

size_t router_backward_workspace(int64_t N, int64_t Z, int64_t K) {
  const router::BwdPlan pl = router::bwd_plan(N, Z);
  return static_cast<size_t>(pl.ranges * K * Z) * 4;
}

namespace router {

// Launch F<KC> with KC = ceil(K / 16) (1..6).
template <template <int> class F, typename... A>
void with_kc(int64_t K, A&&... a) {
  switch ((K + 15) / 16) {
    case 1: F<1>::run(a...); break;
    case 2: F<2>::run(a...); break;
    case 3: F<3>::run(a...); break;
    case 4: F<4>::run(a...); break;
    case 5: F<5>::run(a...); break;
    default: F<6>::run(a...); break;
  }
}

template <int KC>
struct FwdLaunch {
  static void run(const uint16_t* z, const uint16_t* r, uint16_t* out, int64_t N, int Z, int K,
                  int routing, const RouteGroups& grp, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(cdiv(N, 32)));
    if (grp.n > 0)
      hipLaunchKernelGGL((router_fwd_kernel<KC, true>), grid, dim3(256), 0, st, z, r, out, N, Z, K,
                         routing, grp);
    else
      hipLaunchKernelGGL((router_fwd_kernel<KC, false>), grid, dim3(256), 0, st, z, r, out, N, Z,
                         K, routing, grp);
  }
};

template <int KC>
struct DzLaunch {
  static void run(const uint16_t* dl, const uint16_t* r, uint16_t* dz, int64_t N, int Z, int K,
                  hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(cdiv(Z / 64, 4)),
                    static_cast<unsigned>(cdiv(N, 16 * kDzBlocks<KC>)));
    hipLaunchKernelGGL(router_dz_kernel<KC>, grid, dim3(256), 0, st, dl, r, dz, N, Z, K);
  }
};

template <int KC>
struct DrLaunch {
  static void run(const uint16_t* dl, const uint16_t* z, float* part, int64_t N, int Z, int K,
                  const BwdPlan& pl, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(Z / 64), static_cast<unsigned>(pl.ranges));
    hipLaunchKernelGGL(router_dr_kernel<KC>, grid, dim3(256), 0, st, dl, z, part, N, Z, K,
                       static_cast<int>(pl.blocks_per_range));
  }
};

void dr_reduce(const float* part, void* dr, int64_t K, int64_t Z, const BwdPlan& pl,
               hipStream_t st) {
  const int64_t KZ = K * Z;
  hipLaunchKernelGGL(router_dr_reduce_kernel, dim3(static_cast<unsigned>(cdiv(KZ, 256))),
                     dim3(256), 0, st, part, static_cast<uint16_t*>(dr), KZ,
                     static_cast<int>(pl.ranges));
}

}  // namespace router

void router_forward(const void* z, const void* r, void* logits, int64_t N, int64_t Z, int64_t K,
                    int routing, hipStream_t st) {
  // the fused activation (routing 1 / 2) is built for K <= 32 only
  const RouteGroups none{};
  router::with_kc<router::FwdLaunch>(K, static_cast<const uint16_t*>(z),
                                     static_cast<const uint16_t*>(r),
                                     static_cast<uint16_t*>(logits), N, static_cast<int>(Z),
                                     static_cast<int>(K), K <= 32 ? routing : ROUTE_ALPHA, none,
                                     st);
}

void router_forward_grouped(const void* z, const void* r, const RouteGroups& groups, int64_t N,
                            int64_t Z, hipStream_t st) {
  int K = 0;
  for (int g = 0; g < groups.n; ++g) K += groups.kn[g];
  router::with_kc<router::FwdLaunch>(K, static_cast<const uint16_t*>(z),
                                     static_cast<const uint16_t*>(r), static_cast<uint16_t*>(nullptr),
                                     N, static_cast<int>(Z), K, ROUTE_ALPHA, groups, st);
}

void router_backward(const void* z, const void* r, const void* dl, void* dz, void* dr,
                     int64_t N, int64_t Z, int64_t K, void* workspace, hipStream_t st) {
  const auto* zp = static_cast<const uint16_t*>(z);
  const auto* rp = static_cast<const uint16_t*>(r);
  const auto* dp = static_cast<const uint16_t*>(dl);
  const int Zi = static_cast<int>(Z), Ki = static_cast<int>(K);
  const router::BwdPlan pl = router::bwd_plan(N, Z);
  float* part = static_cast<float*>(workspace);
  // both outputs, K <= 32: one pass over z and dz
  if (dz != nullptr && dr != nullptr && K <= 32) {
    const dim3 grid(static_cast<unsigned>(Z / 64), static_cast<unsigned>(pl.ranges));
    auto* op = static_cast<uint16_t*>(dz);
    if (K <= 16)
      hipLaunchKernelGGL(router::router_bwd_kernel<1>, grid, dim3(256), 0, st, dp, zp, rp, op,
                         part, N, Zi, Ki, static_cast<int>(pl.blocks_per_range));
    else
      hipLaunchKernelGGL(router::router_bwd_kernel<2>, grid, dim3(256), 0, st, dp, zp, rp, op,
                         part, N, Zi, Ki, static_cast<int>(pl.blocks_per_range));
    router::dr_reduce(part, dr, K, Z, pl, st);
    return;
  }
  if (dz != nullptr)
    router::with_kc<router::DzLaunch>(K, dp, rp, static_cast<uint16_t*>(dz), N, Zi, Ki, st);
  if (dr != nullptr) {
    router::with_kc<router::DrLaunch>(K, dp, zp, part, N, Zi, Ki, pl, st);
    router::dr_reduce(part, dr, K, Z, pl, st);
  }
}

}  // namespace moc
