// Decode step on the matrix cores (bf16 x, cache, logits and basis; contiguous
// [B, D, S] cache):
// the reference's _moc_update_kernel (moc/kernels.py:442-550 of the reference).
//
//   y[b, d]  = act(sum_{s < S-1} cache[b, d, s+1] W[b, s, d] + x[b, d] W[b, S-1, d])
//   W[b,s,d] = sum_k alpha[b, k] basis[k, s, d]     (alpha = softmax / exp of the logits)
//   cache[b, d, :] <- (cache[b, d, 1:], x[b, d])    (pure copies: bit-exact)
//
// Layout as in the forward kernel: a wave covers 16 tokens (MFMA rows) and
// CW = 16 NC channels (NC contiguous per lane).  The routing weights are formed
// in the A-operand layout itself (lane (i, qq): token i, routes 16 kc + 4 qq +
// {0..3}; softmax over the 4 lanes i, i + 16, i + 32, i + 48) and rounded as the
// forward path rounds them; W comes from one MFMA per (tap, channel column).
// Each lane reads and writes one cache row of NC channels x S slots per token
// (4 S bytes, contiguous) and touches nothing else of the cache.
#pragma once

#include "moc_kernels.h"
#include "moc_mfma.h"

namespace moc {
namespace decode {

using mfma::Buf;
using mfma::CT;
using mfma::f32x4;
using mfma::kOffNone;
using mfma::s16x4;

constexpr int kNC = 2;  // channels per lane

// Row of NC channels x S slots (bf16) as 32-bit words.
template <int S>
struct CacheRow {
  static constexpr int kWords = kNC * S / 2;
  uint32_t w[kWords];
  __device__ __forceinline__ uint16_t get(int c, int s) const {
    const int e = c * S + s;
    return static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
  }
  __device__ __forceinline__ void set(int c, int s, uint16_t v) {
    const int e = c * S + s;
    const uint32_t sh = 16 * (e & 1);
    w[e >> 1] = (w[e >> 1] & ~(0xffffu << sh)) | (static_cast<uint32_t>(v) << sh);
  }
  // whole rows per access (16 or 8 bytes; 4-byte words for 3 slots): a 16-lane
  // group then moves one contiguous span of rows per instruction
  static constexpr int kVec = kWords % 4 == 0 ? 4 : (kWords % 2 == 0 ? 2 : 1);
  static __device__ __forceinline__ int at(uint32_t off, int i) {
    return static_cast<int>(off == kOffNone ? off : off + 4 * kVec * i);
  }
  __device__ __forceinline__ void load(const Buf& b, uint32_t off) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < kWords / kVec; ++i) {
      if constexpr (kVec == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(b.r, at(off, i), 0, 0);
        __builtin_memcpy(&w[4 * i], &v, 16);
      } else if constexpr (kVec == 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(b.r, at(off, i), 0, 0);
        __builtin_memcpy(&w[2 * i], &v, 8);
      } else {
        w[i] = __builtin_amdgcn_raw_buffer_load_b32(b.r, at(off, i), 0, 0);
      }
    }
  }
  __device__ __forceinline__ void store(const Buf& b, uint32_t off) const {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < kWords / kVec; ++i) {
      if constexpr (kVec == 4) {
        u32x4 v;
        __builtin_memcpy(&v, &w[4 * i], 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, b.r, at(off, i), 0, 0);
      } else if constexpr (kVec == 2) {
        u32x2 v;
        __builtin_memcpy(&v, &w[2 * i], 8);
        __builtin_amdgcn_raw_buffer_store_b64(v, b.r, at(off, i), 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(w[i], b.r, at(off, i), 0, 0);
      }
    }
  }
};

// FUSED: the logits come from the router GEMM in the same kernel (z [B, Z],
// router [K, Z]); otherwise `alpha` holds them (or the weights, ROUTE_ALPHA).
template <int S, int KC, bool ACT, bool FUSED>
__global__ void __launch_bounds__(256) decode_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ alpha, int routing,
    const uint16_t* __restrict__ basis, uint16_t* __restrict__ cache, uint16_t* __restrict__ y,
    int64_t B, int64_t D, int K, const uint16_t* __restrict__ z,
    const uint16_t* __restrict__ router, int Z) {
  using C = CT<true>;
  constexpr int CW = 16 * kNC;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, qq = lane >> 4;
  const int64_t tb = static_cast<int64_t>(blockIdx.y) * 16;
  const int64_t d0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * CW;
  const bool wave_on = d0 < D;
  // without the router stage the kernel has no barrier and idle waves leave
  if (!FUSED && !wave_on) return;
  const int64_t ta = tb + i;              // token of this lane's A-operand row
  const bool tok_ok = ta < B;
  const int64_t dl = d0 + kNC * i;        // first channel of this lane
  const bool ch_ok = wave_on && dl < D;   // D is even: both channels are in or out

  // FUSED: the router GEMV's loads go first, all of a wave's z chunks in one
  // round (UBW chunks; more rounds only past 256 UBW z columns), so that the
  // GEMV waits for them alone: the memory counter retires loads in issue
  // order, and loads issued before them would hold it up.  Wave w takes the
  // 64-wide z chunks c = w, w + 4, ...; lane (i, qq) loads columns 64 c + 8 qq
  // + [0, 8) and 64 c + 32 + 8 qq + [0, 8) of token tb + i and route 16 kc + i.
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int UBW = KC == 1 ? 8 : 4;
  u32x4 za[UBW][2], ra[UBW][KC][2];
  const int nchunk = Z / 64;
  const uint32_t zrow = static_cast<uint32_t>(i * Z * 2);
  const int64_t zrows = (B - tb < 16) ? B - tb : 16;
  const Buf zb(z + tb * Z, FUSED ? zrows * Z * 2 : 0);
  const Buf rbuf(router, FUSED ? static_cast<int64_t>(K) * Z * 2 : 0);
  auto gemv_load = [&](int c0) {
#pragma unroll
    for (int u = 0; u < UBW; ++u) {
      const int c = c0 + 4 * u;
      const bool on = c < nchunk;
      const uint32_t col0 = static_cast<uint32_t>((64 * c + 8 * qq) * 2), col1 = col0 + 64;
      za[u][0] = __builtin_amdgcn_raw_buffer_load_b128(zb.r, static_cast<int>(on ? zrow + col0 : kOffNone), 0, 0);
      za[u][1] = __builtin_amdgcn_raw_buffer_load_b128(zb.r, static_cast<int>(on ? zrow + col1 : kOffNone), 0, 0);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const uint32_t rrow = static_cast<uint32_t>((16 * kc + i) * Z * 2);
        ra[u][kc][0] = __builtin_amdgcn_raw_buffer_load_b128(rbuf.r, static_cast<int>(on ? rrow + col0 : kOffNone), 0, 0);
        ra[u][kc][1] = __builtin_amdgcn_raw_buffer_load_b128(rbuf.r, static_cast<int>(on ? rrow + col1 : kOffNone), 0, 0);
      }
    }
  };
  if constexpr (FUSED) gemv_load(wave);
  __builtin_amdgcn_sched_barrier(0);

  // The other loads of the step, without branches (out-of-range offsets load
  // zeros): logits (not FUSED), basis rows, x and cache rows.
  // logits of token ta, routes 16 kc + 4 qq + {0..3} (K % 4 == 0: whole words)
  uint32_t lw[KC][2];
  if constexpr (!FUSED) {
    const Buf ab(alpha, B * K * 2);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = 16 * kc + 4 * qq;
      const uint32_t off = (tok_ok && k < K) ? static_cast<uint32_t>((ta * K + k) * 2) : kOffNone;
      lw[kc][0] = __builtin_amdgcn_raw_buffer_load_b32(ab.r, static_cast<int>(off), 0, 0);
      lw[kc][1] = __builtin_amdgcn_raw_buffer_load_b32(ab.r, static_cast<int>(off == kOffNone ? off : off + 4), 0, 0);
    }
  }
  // basis row (k, s) at this lane's two channels: bw[s][kc][v], k = 16 kc + 4 qq + v
  const Buf bbuf(basis, static_cast<int64_t>(K) * S * D * 2);
  uint32_t bw[S][KC][4];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        const uint32_t off = (ch_ok && k < K)
            ? static_cast<uint32_t>(((static_cast<int64_t>(k) * S + s) * D + dl) * 2) : kOffNone;
        bw[s][kc][v] = __builtin_amdgcn_raw_buffer_load_b32(bbuf.r, static_cast<int>(off), 0, 0);
      }
  // result lane (j, q): channels dl, dl + 1 of tokens tb + 4 q + v
  const int64_t rows = (B - tb < 16) ? B - tb : 16;
  const Buf xb(x + tb * D, rows * D * 2);
  const Buf yb(y + tb * D, rows * D * 2);
  const Buf cb(cache + tb * D * S, rows * D * S * 2);
  CacheRow<S> cr[4];
  uint32_t xv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * qq + v;
    const uint32_t xo = ch_ok ? static_cast<uint32_t>((r * D + dl) * 2) : kOffNone;
    xv[v] = __builtin_amdgcn_raw_buffer_load_b32(xb.r, static_cast<int>(xo), 0, 0);
    cr[v].load(cb, ch_ok ? static_cast<uint32_t>((r * D + dl) * S * 2) : kOffNone);
  }

  // every load above is issued before the GEMV's products consume its loads
  __builtin_amdgcn_sched_barrier(0);

  // the cache update needs no routing weights: the history shifted one slot and
  // x appended go out as soon as the rows have landed, so that these 4 S bytes
  // per channel and token are written while the GEMV, the softmax and the
  // mixture run, not after them
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * qq + v;
    CacheRow<S> nr;
#pragma unroll
    for (int c = 0; c < kNC; ++c) {
#pragma unroll
      for (int s = 0; s + 1 < S; ++s) nr.set(c, s, cr[v].get(c, s + 1));
      nr.set(c, S - 1, static_cast<uint16_t>(xv[v] >> (16 * c)));
    }
    nr.store(cb, ch_ok ? static_cast<uint32_t>((r * D + dl) * S * 2) : kOffNone);
  }
  __builtin_amdgcn_sched_barrier(0);

  // routing weights in the A-operand layout, rounded as the forward path rounds
  // them (softmax / exp in fp32, then to bf16)
  float l[KC][4];
  if constexpr (FUSED) {
    // logits of tokens tb..tb+15 = z . router^T (bf16-rounded, as the router
    // GEMM's output): wave w sums the 64-wide z chunks c = w, w + 4, ... of all
    // 16 tokens (lane (i, qq): columns 64 c + 8 qq + [0, 8) and 64 c + 32 + 8 qq
    // + [0, 8) of token tb + i and route 16 kc + i); the 4 partial tiles are
    // summed in LDS in wave order
    __shared__ float red[4][16 * KC][17];
    f32x4 acc[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) acc[kc] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto gemv_mma = [&]() {
#pragma unroll
      for (int u = 0; u < UBW; ++u)
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            acc[kc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, za[u][h]),
                                                              __builtin_bit_cast(bf16x8, ra[u][kc][h]),
                                                              acc[kc], 0, 0, 0);
    };
    // the first round in straight-line code, so that each product waits for
    // its own loads only (not for the step's later-issued loads); further
    // rounds (z_dim above 256 UBW) in a loop
    gemv_mma();
    for (int c0 = wave + 4 * UBW; c0 < nchunk; c0 += 4 * UBW) {
      gemv_load(c0);
      gemv_mma();
    }
    // result lane (j, q): route 16 kc + j, tokens 4 q + v
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][16 * kc + i][4 * qq + v] = acc[kc][v];
    __syncthreads();
    if (!wave_on) return;  // no barrier follows
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        const float sv = ((red[0][k][i] + red[1][k][i]) + red[2][k][i]) + red[3][k][i];
        l[kc][v] = (tok_ok && k < K) ? round_to(sv, DT_BF16) : -INFINITY;
      }
  } else {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        l[kc][v] = (tok_ok && k < K) ? bf16_to_f32(static_cast<uint16_t>(lw[kc][v >> 1] >> (16 * (v & 1))))
                                     : -INFINITY;
      }
  }
  float a[KC][4];
  if (routing == ROUTE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) m = fmaxf(m, l[kc][v]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        a[kc][v] = (k < K && tok_ok) ? __expf(l[kc][v] - m) : 0.f;
        sum += a[kc][v];
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = tok_ok ? 1.0f / sum : 0.f;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) a[kc][v] = round_to(a[kc][v] * inv, DT_BF16);
  } else {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * kc + 4 * qq + v;
        const bool on = tok_ok && k < K;
        a[kc][v] = !on ? 0.f : (routing == ROUTE_EXP ? round_to(__expf(l[kc][v]), DT_BF16) : l[kc][v]);
      }
  }
  s16x4 aop[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
    aop[kc] = C::make(C::from_f(a[kc][0]), C::from_f(a[kc][1]), C::from_f(a[kc][2]),
                      C::from_f(a[kc][3]));
  // B operands: bw[s][kc][v] holds channels (dl, dl + 1) of route 16 kc + 4 qq + v
  s16x4 bop[S][kNC][KC];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int c = 0; c < kNC; ++c) {
        const uint32_t sel = c == 0 ? 0x05040100u : 0x07060302u;  // low / high halves
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 wv = {__builtin_amdgcn_perm(bw[s][kc][1], bw[s][kc][0], sel),
                          __builtin_amdgcn_perm(bw[s][kc][3], bw[s][kc][2], sel)};
        bop[s][c][kc] = __builtin_bit_cast(s16x4, wv);
      }

  f32x4 w[S][kNC];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int c = 0; c < kNC; ++c) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KC == 2) {
        acc = C::mma2(aop[0], aop[1], bop[s][c][0], bop[s][c][1], acc);
      } else {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) acc = C::mma(aop[kc], bop[s][c][kc], acc);
      }
      w[s][c] = acc;
    }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * qq + v;
    uint16_t xo[kNC];
    float yo[kNC];
#pragma unroll
    for (int c = 0; c < kNC; ++c) {
      xo[c] = static_cast<uint16_t>(xv[v] >> (16 * c));
      // taps in ascending order: history slots 1..S-1, then the new input
      float p = 0.f;
#pragma unroll
      for (int s = 0; s < S - 1; ++s) p = fmaf(bf16_to_f32(cr[v].get(c, s + 1)), w[s][c][v], p);
      p = fmaf(bf16_to_f32(xo[c]), w[S - 1][c][v], p);
      yo[c] = ACT ? p * sigmoid_f(p) : p;
    }
    const uint32_t yw = static_cast<uint32_t>(f32_to_bf16(yo[0])) |
                        (static_cast<uint32_t>(f32_to_bf16(yo[1])) << 16);
    __builtin_amdgcn_raw_buffer_store_b32(
        yw, yb.r, static_cast<int>(ch_ok ? static_cast<uint32_t>((r * D + dl) * 2) : kOffNone), 0, 0);
  }
}

template <int S, int KC, bool ACT, bool FUSED>
void launch_one(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                void* y, int64_t B, int64_t D, int64_t K, const void* z, const void* router,
                int64_t Z, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((D + 4 * 16 * kNC - 1) / (4 * 16 * kNC)),
                  static_cast<unsigned>((B + 15) / 16));
  hipLaunchKernelGGL((decode_kernel<S, KC, ACT, FUSED>), grid, dim3(256), 0, st,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(alpha), routing,
                     static_cast<const uint16_t*>(basis), static_cast<uint16_t*>(cache),
                     static_cast<uint16_t*>(y), B, D, static_cast<int>(K),
                     static_cast<const uint16_t*>(z), static_cast<const uint16_t*>(router),
                     static_cast<int>(Z));
}

template <int S, bool FUSED>
bool launch_s(const void* x, const void* alpha, int routing, const void* basis, void* cache,
              void* y, int64_t B, int64_t D, int64_t K, int act, const void* z, const void* router,
              int64_t Z, hipStream_t st) {
  if (K <= 16) {
    if (act) launch_one<S, 1, true, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
    else launch_one<S, 1, false, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
  } else if (K <= 32) {
    if (act) launch_one<S, 2, true, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
    else launch_one<S, 2, false, FUSED>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
  } else if constexpr (!FUSED) {
    // 33-64 routes: given logits / weights only (the fused router GEMV stops at 32)
    if (act) launch_one<S, 4, true, false>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
    else launch_one<S, 4, false, false>(x, alpha, routing, basis, cache, y, B, D, K, z, router, Z, st);
  } else {
    return false;  // the fused step is built for up to 32 routes
  }
  return true;
}

// 9 to 16 taps (moc_decode_long.hip): launch_s for those kernel sizes.
template <bool FUSED>
bool launch_long(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                 void* y, int64_t B, int64_t D, int64_t K, int64_t S, int act, const void* z,
                 const void* router, int64_t Z, hipStream_t st);

}  // namespace decode
}  // namespace moc
