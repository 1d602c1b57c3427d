// Generic MoC kernels: any K, any kernel size S, any storage dtypes.
//
// One lane per (token, channel) element; the mixture W[n,s,d] = sum_k a[n,k] b[k,s,d]
// is formed on VALU.  These kernels serve shapes outside the MFMA kernels'
// instantiations (moc_mfma.hip) and the decode step.  They keep the reference's
// semantics (moc/kernels.py:36-142 forward, 156-268 dx, 282-426 dalpha/dbasis,
// 442-550 decode) but reduce dalpha / dbasis in a fixed order instead of atomics.
#include <type_traits>

#include "moc_common.h"
#include "moc_kernels.h"
#include "moc_mfma.h"

namespace moc {

// ---------------------------------------------------------------------------
// Routing weights: a_r[n,k] = act(alpha_in[n,:])[k] rounded to the dtype the
// router activation would have produced (the logits' dtype), as fp32.  The
// mixture then uses round_to(a_r, compute dtype) (moc/kernels.py:92-95).
// One lane per token.
__global__ void prep_alpha_kernel(const void* __restrict__ alpha_in, int a_dt, int routing,
                                  int64_t n_tokens, int64_t K, float* __restrict__ a_r) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_tokens) return;
  const int64_t base = t * K;
  if (routing == ROUTE_SOFTMAX) {
    float m = -INFINITY;
    for (int64_t k = 0; k < K; ++k) m = fmaxf(m, load_any(alpha_in, a_dt, base + k));
    float sum = 0.f;
    for (int64_t k = 0; k < K; ++k) sum += __expf(load_any(alpha_in, a_dt, base + k) - m);
    const float inv = 1.0f / sum;
    for (int64_t k = 0; k < K; ++k)
      a_r[base + k] = round_to(__expf(load_any(alpha_in, a_dt, base + k) - m) * inv, a_dt);
  } else if (routing == ROUTE_EXP) {
    for (int64_t k = 0; k < K; ++k)
      a_r[base + k] = round_to(__expf(load_any(alpha_in, a_dt, base + k)), a_dt);
  } else {
    for (int64_t k = 0; k < K; ++k) a_r[base + k] = load_any(alpha_in, a_dt, base + k);
  }
}

// basis_c = basis rounded to the compute dtype, fp32.
__global__ void prep_basis_kernel(const void* __restrict__ basis, int b_dt, int64_t count,
                                  int c_dt, float* __restrict__ basis_c) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  basis_c[i] = round_to(load_any(basis, b_dt, i), c_dt);
}

// W[t,s,d] from the prepared operands.
__device__ __forceinline__ float mix_w(const float* __restrict__ a_r, const float* __restrict__ basis_c,
                                       int64_t t, int64_t s, int64_t d, int64_t K, int64_t S,
                                       int64_t D, int c_dt) {
  float w = 0.f;
  for (int64_t k = 0; k < K; ++k)
    w = fmaf(round_to(a_r[t * K + k], c_dt), basis_c[(k * S + s) * D + d], w);
  return w;
}

// Pre-activation P[t,d] (moc/kernels.py:97-130).
__device__ __forceinline__ float preact_at(const void* __restrict__ x, int x_dt,
                                           const float* __restrict__ a_r,
                                           const float* __restrict__ basis_c,
                                           int64_t t, int64_t d, int64_t pos, int64_t K,
                                           int64_t S, int64_t D, int c_dt) {
  float acc = 0.f;
  for (int64_t s = 0; s < S; ++s) {
    const int64_t off = S - 1 - s;
    if (off > pos) continue;
    const float w = mix_w(a_r, basis_c, t, s, d, K, S, D, c_dt);
    acc = fmaf(load_any(x, x_dt, (t - off) * D + d), w, acc);
  }
  return acc;
}

__global__ void fwd_generic_kernel(const void* __restrict__ x, int x_dt,
                                   const float* __restrict__ a_r,
                                   const float* __restrict__ basis_c, void* __restrict__ y,
                                   SeqLayout seq, int64_t D, int64_t K, int64_t S,
                                   int activation) {
  const int64_t total = seq.n_tokens * D;
  const int c_dt = x_dt;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / D, d = i - t * D;
    int64_t lo, hi;
    seq.bounds(t, lo, hi);
    float p = preact_at(x, x_dt, a_r, basis_c, t, d, t - lo, K, S, D, c_dt);
    if (activation) p = p * sigmoid_f(p);
    store_any(y, x_dt, i, p);
  }
}

// ---------------------------------------------------------------------------
// Backward.  g = dy * silu'(P) (or dy), kept in fp32 scratch; dy rows are
// dys elements apart (0: one row for every token; -1: one element for all).
__global__ void bwd_g_kernel(const void* __restrict__ x, const void* __restrict__ dy, int64_t dys,
                             int x_dt, const float* __restrict__ a_r,
                             const float* __restrict__ basis_c, float* __restrict__ g,
                             SeqLayout seq, int64_t D, int64_t K, int64_t S, int activation) {
  const int64_t total = seq.n_tokens * D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / D, d = i - t * D;
    float gv = load_any(dy, x_dt, dys < 0 ? 0 : t * dys + d);
    if (activation) {
      int64_t lo, hi;
      seq.bounds(t, lo, hi);
      const float p = preact_at(x, x_dt, a_r, basis_c, t, d, t - lo, K, S, D, x_dt);
      const float sg = sigmoid_f(p);
      gv = gv * (sg * (1.0f + p * (1.0f - sg)));  // moc/kernels.py:231-232
    }
    g[i] = gv;
  }
}

// dx[u,d] = sum_s g[u+S-1-s,d] * W[u+S-1-s,s,d] for u+S-1-s inside u's sequence
// (moc/kernels.py:207-259).
__global__ void bwd_dx_kernel(const float* __restrict__ g, const float* __restrict__ a_r,
                              const float* __restrict__ basis_c, void* __restrict__ dx,
                              int x_dt, SeqLayout seq, int64_t D, int64_t K, int64_t S) {
  const int64_t total = seq.n_tokens * D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t u = i / D, d = i - u * D;
    int64_t lo, hi;
    seq.bounds(u, lo, hi);
    float acc = 0.f;
    for (int64_t s = 0; s < S; ++s) {
      const int64_t t = u + (S - 1 - s);
      if (t >= hi) continue;
      acc = fmaf(g[t * D + d], mix_w(a_r, basis_c, t, s, d, K, S, D, x_dt), acc);
    }
    store_any(dx, x_dt, i, acc);
  }
}

constexpr int kRedThreads = 256;
constexpr int kKChunk = 16;

// Sum v over the 256 lanes of the block; every lane gets the result.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// dalpha[t,k] = sum_d sum_s g[t,d] x[t-(S-1-s),d] basis[k,s,d] (moc/kernels.py:344-406),
// then the router activation gradient.  One 256-lane block per token; dynamic LDS
// holds K floats of dalpha.
__global__ void __launch_bounds__(kRedThreads)
bwd_dalpha_kernel(const void* __restrict__ x, int x_dt, const float* __restrict__ g,
                  const float* __restrict__ a_r, const float* __restrict__ basis_c,
                  void* __restrict__ dalpha, int a_dt, int routing, SeqLayout seq,
                  int64_t D, int64_t K, int64_t S) {
  extern __shared__ float da[];  // [K]
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  int64_t lo, hi;
  seq.bounds(t, lo, hi);
  const int64_t pos = t - lo;
  for (int64_t k0 = 0; k0 < K; k0 += kKChunk) {
    float acc[kKChunk];
#pragma unroll
    for (int j = 0; j < kKChunk; ++j) acc[j] = 0.f;
    for (int64_t d = threadIdx.x; d < D; d += kRedThreads) {
      const float gv = g[t * D + d];
      for (int64_t s = 0; s < S; ++s) {
        const int64_t off = S - 1 - s;
        if (off > pos) continue;
        const float m = gv * load_any(x, x_dt, (t - off) * D + d);
#pragma unroll
        for (int j = 0; j < kKChunk; ++j) {
          if (k0 + j < K) acc[j] = fmaf(m, basis_c[((k0 + j) * S + s) * D + d], acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kKChunk; ++j) {
      const float v = block_sum256(acc[j], red);
      if (threadIdx.x == 0 && k0 + j < K) da[k0 + j] = v;
    }
  }
  __syncthreads();
  float dot = 0.f;
  if (routing == ROUTE_SOFTMAX) {
    for (int64_t k = 0; k < K; ++k) dot = fmaf(a_r[t * K + k], da[k], dot);
  }
  for (int64_t k = threadIdx.x; k < K; k += kRedThreads) {
    float v = da[k];
    if (routing == ROUTE_SOFTMAX) v = a_r[t * K + k] * (v - dot);
    else if (routing == ROUTE_EXP) v = a_r[t * K + k] * v;
    store_any(dalpha, a_dt, t * K + k, v);
  }
}

// dbasis partial over a chunk of kTokChunk tokens: part[c,k,s,d] =
// sum_{t in chunk c} a[t,k] g[t,d] x[t-(S-1-s),d].  One lane per channel.
constexpr int64_t kTokChunk = 256;

__global__ void bwd_dbasis_partial_kernel(const void* __restrict__ x, int x_dt,
                                          const float* __restrict__ g,
                                          const float* __restrict__ a_r,
                                          float* __restrict__ part, SeqLayout seq, int64_t D,
                                          int64_t K, int64_t S) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t c = blockIdx.y;
  if (d >= D) return;
  const int64_t t0 = c * kTokChunk;
  const int64_t t1 = (t0 + kTokChunk < seq.n_tokens) ? t0 + kTokChunk : seq.n_tokens;
  const int64_t KS = K * S;
  for (int64_t p0 = 0; p0 < KS; p0 += kKChunk) {
    float acc[kKChunk];
#pragma unroll
    for (int j = 0; j < kKChunk; ++j) acc[j] = 0.f;
    for (int64_t t = t0; t < t1; ++t) {
      int64_t lo, hi;
      seq.bounds(t, lo, hi);
      const int64_t pos = t - lo;
      const float gv = g[t * D + d];
#pragma unroll
      for (int j = 0; j < kKChunk; ++j) {
        const int64_t p = p0 + j;
        if (p >= KS) continue;
        const int64_t k = p / S, s = p - k * S, off = S - 1 - s;
        if (off > pos) continue;
        const float m = gv * load_any(x, x_dt, (t - off) * D + d);
        acc[j] = fmaf(round_to(a_r[t * K + k], x_dt), m, acc[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < kKChunk; ++j) {
      if (p0 + j < KS) part[(c * KS + p0 + j) * D + d] = acc[j];
    }
  }
}

// dbasis[i] = sum_c part[c, i] in chunk order, stored in the basis dtype.
__global__ void reduce_partials_kernel(const float* __restrict__ part, int64_t n_parts,
                                       int64_t count, void* __restrict__ out, int out_dt) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float acc = 0.f;
  for (int64_t c = 0; c < n_parts; ++c) acc += part[c * count + i];
  store_any(out, out_dt, i, acc);
}

// ---------------------------------------------------------------------------
// Decode step (moc/kernels.py:442-550).  Block = (batch row, 256 channels); the
// routing weights of the row are formed once per block in LDS.
__global__ void __launch_bounds__(256)
update_kernel(const void* __restrict__ x, const void* __restrict__ alpha, int a_dt,
              int routing, const void* __restrict__ basis, int b_dt, void* __restrict__ cache,
              int64_t cs_b, int64_t cs_d, int64_t cs_s, void* __restrict__ y, int x_dt,
              int64_t D, int64_t K, int64_t S, int activation) {
  extern __shared__ float a_s[];  // [K]
  const int64_t b = blockIdx.y;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (threadIdx.x == 0) {
    // K is small; one lane forms the row's weights in a fixed order.
    float m = -INFINITY, sum = 0.f;
    if (routing == ROUTE_SOFTMAX) {
      for (int64_t k = 0; k < K; ++k) m = fmaxf(m, load_any(alpha, a_dt, b * K + k));
      for (int64_t k = 0; k < K; ++k) sum += __expf(load_any(alpha, a_dt, b * K + k) - m);
    }
    for (int64_t k = 0; k < K; ++k) {
      const float l = load_any(alpha, a_dt, b * K + k);
      float a = l;
      if (routing == ROUTE_SOFTMAX) a = round_to(__expf(l - m) * (1.0f / sum), a_dt);
      else if (routing == ROUTE_EXP) a = round_to(__expf(l), a_dt);
      a_s[k] = round_to(a, x_dt);
    }
  }
  __syncthreads();
  if (d >= D) return;
  char* cb = static_cast<char*>(cache);
  const int esz = (x_dt == DT_F32) ? 4 : 2;
  const int64_t cbase = b * cs_b + d * cs_d;
  const float xv = load_any(x, x_dt, b * D + d);
  float acc = 0.f;
  for (int64_t s = 0; s < S; ++s) {
    float w = 0.f;
    for (int64_t k = 0; k < K; ++k)
      w = fmaf(a_s[k], round_to(load_any(basis, b_dt, (k * S + s) * D + d), x_dt), w);
    const float h = (s == S - 1) ? xv : load_any(cb, x_dt, 0 + (cbase + (s + 1) * cs_s));
    acc = fmaf(h, w, acc);
  }
  if (activation) acc = acc * sigmoid_f(acc);
  store_any(y, x_dt, b * D + d, acc);
  // Shift the history one slot left (pure copies: bit-exact), append x.
  if (esz == 4) {
    float* c = reinterpret_cast<float*>(cb);
    for (int64_t s = 0; s + 1 < S; ++s) c[cbase + s * cs_s] = c[cbase + (s + 1) * cs_s];
    c[cbase + (S - 1) * cs_s] = static_cast<const float*>(x)[b * D + d];
  } else {
    uint16_t* c = reinterpret_cast<uint16_t*>(cb);
    for (int64_t s = 0; s + 1 < S; ++s) c[cbase + s * cs_s] = c[cbase + (s + 1) * cs_s];
    c[cbase + (S - 1) * cs_s] = static_cast<const uint16_t*>(x)[b * D + d];
  }
}

// ---------------------------------------------------------------------------
// Decode step for the shapes the matrix-core decode kernel does not take (fp32
// data, mixed storage dtypes, strided caches, any D, 9 to 16 taps), 2 to 16
// taps and up to 64 routes.  A workgroup covers 64 channels (one per lane) and
// 4 T tokens (T per wave):
//   * every load goes out first: the wave's logits, x, the cache slots and its
//     quarter of the basis tile (KT routes x S taps x 64 channels), with
//     clamped indices and selected values (a load under a per-lane condition
//     compiles to a branch that waits for it);
//   * the routing weights are formed in the wave as soon as the logits have
//     landed (lane: token lane / LPT, routes lane % LPT + LPT i; max and sum
//     over the token's LPT lanes by shuffles) into the wave's LDS rows;
//   * the shifted cache goes out (it needs no routing weights), and the basis
//     quarter goes to LDS, rounded to x's dtype once;
//   * after the barrier, W[t][s] = sum_k alpha[t][k] basis[k][s][d] with k
//     ascending, then y = act(sum_s h_s W_s) with s ascending, as update_kernel
//     orders them.
// ROW: the cache rows are contiguous (cache_stride_s == 1) and aligned to the
// row's vector width, so each lane moves a token's S slots as whole words.
constexpr int kDecMaxK = 64;

// Typed element loads: the storage dtype is chosen once per loop (a uniform
// branch around it), so a loop's loads issue back to back.
struct BF16Tag {};
__device__ __forceinline__ float ld(const void* p, int64_t i, float) { return static_cast<const float*>(p)[i]; }
__device__ __forceinline__ float ld(const void* p, int64_t i, BF16Tag) {
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ float ld(const void* p, int64_t i, _Float16) {
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}
template <typename F>
__device__ __forceinline__ void with_dtype(int dt, F&& f) {
  if (dt == DT_F32) f(float{});
  else if (dt == DT_BF16) f(BF16Tag{});
  else f(_Float16{});
}

// Bytes per access of a whole cache row of S slots of `esize` bytes: the
// largest power of two dividing the row (at most 16); 0 when the row is not a
// whole number of 4-byte words.
__host__ __device__ constexpr int dec_row_vec_bytes(int S, int esize) {
  return (S * esize) % 4 != 0 ? 0 : (S * esize) % 16 == 0 ? 16 : (S * esize) % 8 == 0 ? 8 : 4;
}
__host__ __device__ constexpr int dec_tokens_per_wave(int) { return 4; }

template <int S, bool F32, bool ROW>
__global__ void __launch_bounds__(256)
update_tile_kernel(const void* __restrict__ x, const void* __restrict__ alpha, int a_dt, int routing,
                   const void* __restrict__ basis, int b_dt, void* __restrict__ cache, int64_t cs_b,
                   int64_t cs_d, int64_t cs_s, void* __restrict__ y, int64_t B, int64_t D, int K,
                   int activation) {
  constexpr int T = dec_tokens_per_wave(S);
  constexpr int LPT = 64 / T;             // lanes per token in the softmax
  constexpr int NV = kDecMaxK / LPT;      // routing entries per lane
  constexpr int KT = S <= 2 ? 32 : S <= 4 ? 16 : S <= 8 ? 8 : 4;  // routes per basis chunk
  constexpr int R = KT * S;               // basis rows (route, tap) per chunk: 36 to 64
  constexpr int RP = R + 4;               // padded LDS row of one channel (16-byte reads
                                          // of 8 lanes fall in distinct banks)
  constexpr int ES = F32 ? 4 : 2;         // element bytes of x, y and the cache
  constexpr int x_dt = F32 ? DT_F32 : DT_BF16;
  using E = std::conditional_t<F32, uint32_t, uint16_t>;
  static_assert(R % 4 == 0 && R <= 64, "basis chunk: whole 16-byte groups, at most 64 rows");
  __shared__ float a_s[4][T][kDecMaxK];   // each wave's routing weights
  __shared__ __align__(16) float b_s[64][RP];  // basis chunk, [channel][k * S + s]

  // (the wave index made scalar: addresses built on it stay in SGPRs)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t d = d0 + lane;
  const bool d_ok = d < D;
  const int64_t dc = d_ok ? d : d0;
  const int64_t tb = (static_cast<int64_t>(blockIdx.y) * 4 + wave) * T;
  const int nt = static_cast<int>(B - tb < 0 ? 0 : (B - tb < T ? B - tb : T));  // tokens of this wave
  auto tok = [&](int t) { return tb + t < B ? tb + t : B - 1; };  // a valid token for every t

  // 1. loads: logits, x, cache slots, this wave's rows of the first basis chunk
  float lg[NV];
  const int tl = lane / LPT, kl = lane % LPT;
  with_dtype(a_dt, [&](auto tag) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (LPT * i >= K) {  // wave-uniform: no loads past the last route
        lg[i] = 0.f;
        continue;
      }
      const int k = kl + LPT * i;
      const bool in = tl < nt && k < K;
      lg[i] = ld(alpha, in ? (tb + tl) * K + k : 0, tag);
    }
  });
  const E* xe = static_cast<const E*>(x);
  E xr[T];
#pragma unroll
  for (int t = 0; t < T; ++t) xr[t] = xe[tok(t) * D + dc];
  char* cb = static_cast<char*>(cache);
  constexpr int VB = dec_row_vec_bytes(S, ES);
  constexpr int RW = ROW ? S * ES / 4 : 1;  // 32-bit words per row
  uint32_t rw[T][RW];                        // ROW: whole rows
  E he[T][S];                                // otherwise: slots 1 .. S-1
  if constexpr (ROW) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const char* row = cb + (tok(t) * cs_b + dc * cs_d) * ES;
#pragma unroll
      for (int v = 0; v < RW * 4 / VB; ++v) {
        if constexpr (VB == 16) {
          const u32x4 q = *reinterpret_cast<const u32x4*>(row + 16 * v);
          __builtin_memcpy(&rw[t][4 * v], &q, 16);
        } else if constexpr (VB == 8) {
          const u32x2 q = *reinterpret_cast<const u32x2*>(row + 8 * v);
          __builtin_memcpy(&rw[t][2 * v], &q, 8);
        } else {
          rw[t][v] = *reinterpret_cast<const uint32_t*>(row + 4 * v);
        }
      }
    }
  } else {
    const E* ce = reinterpret_cast<const E*>(cb);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t base = tok(t) * cs_b + dc * cs_d;
#pragma unroll
      for (int s = 1; s < S; ++s) he[t][s] = ce[base + s * cs_s];
    }
  }
  // basis rows r = wave + 4 j of a chunk (route k0 + r / S, tap r % S), through
  // a buffer resource based at the block's first channel: the row offset is
  // block-uniform (a scalar offset), the lane's offset fixed; rounded to x's
  // dtype, zero past route K
  float bq[R / 4];
  auto load_basis = [&](int k0) {
    with_dtype(b_dt, [&](auto tag) {
      constexpr int BS = std::is_same_v<decltype(tag), float> ? 4 : 2;
      const mfma::Buf bb(static_cast<const char*>(basis) + d0 * BS, (static_cast<int64_t>(K) * S * D - d0) * BS);
      const int vo = static_cast<int>((dc - d0) * BS);
#pragma unroll
      for (int j = 0; j < R / 4; ++j) {
        const int r = wave + 4 * j, k = k0 + r / S;
        const bool in = k < K;
        const int so = static_cast<int>((static_cast<int64_t>(in ? k : 0) * S + r % S) * D * BS);
        float v;
        if constexpr (BS == 4) {
          v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(bb.r, vo, so, 0));
        } else {
          const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(bb.r, vo, so, 0);
          if constexpr (std::is_same_v<decltype(tag), BF16Tag>) v = bf16_to_f32(h);
          else v = static_cast<float>(__builtin_bit_cast(_Float16, h));
        }
        bq[j] = in ? v : 0.f;
      }
    });
  };
  auto stage_basis = [&]() {
#pragma unroll
    for (int j = 0; j < R / 4; ++j) b_s[lane][wave + 4 * j] = round_to(bq[j], x_dt);
  };
  load_basis(0);

  // 2. routing weights of token tl, routes kl + LPT i, rounded as update_kernel
  //    rounds them (softmax / exp in fp32, to the logits dtype, to x's dtype);
  //    first, as the logits were loaded first: it waits for them alone
  {
    float m = -INFINITY, sum = 0.f;
    if (routing == ROUTE_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (kl + LPT * i < K) m = fmaxf(m, lg[i]);
#pragma unroll
      for (int o = 1; o < LPT; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        lg[i] = kl + LPT * i < K ? __expf(lg[i] - m) : 0.f;
        sum += lg[i];
      }
#pragma unroll
      for (int o = 1; o < LPT; o <<= 1) sum += __shfl_xor(sum, o, 64);
    }
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = kl + LPT * i;
      float a = lg[i];
      if (routing == ROUTE_SOFTMAX) a = round_to(a * inv, a_dt);
      else if (routing == ROUTE_EXP) a = round_to(__expf(a), a_dt);
      a_s[wave][tl][k] = k < K ? round_to(a, x_dt) : 0.f;
    }
  }
  // 3. the shifted cache (pure copies: bit-exact) with x appended
  auto slot = [&](int t, int s) -> E {  // slot s >= 1 of token t's history
    if constexpr (ROW) {
      if constexpr (F32) return rw[t][s];
      else return static_cast<E>(rw[t][s >> 1] >> (16 * (s & 1)));
    } else {
      return he[t][s];
    }
  };
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t >= nt || !d_ok) continue;
    if constexpr (ROW) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      uint32_t nw[RW];
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        if constexpr (F32) {
          nw[i] = i + 1 < RW ? rw[t][i + 1] : xr[t];
        } else {
          const uint32_t hi = i + 1 < RW ? rw[t][i + 1] : static_cast<uint32_t>(xr[t]);
          nw[i] = (rw[t][i] >> 16) | (hi << 16);
        }
      }
      char* row = cb + ((tb + t) * cs_b + d * cs_d) * ES;
#pragma unroll
      for (int v = 0; v < RW * 4 / VB; ++v) {
        if constexpr (VB == 16) {
          u32x4 q;
          __builtin_memcpy(&q, &nw[4 * v], 16);
          *reinterpret_cast<u32x4*>(row + 16 * v) = q;
        } else if constexpr (VB == 8) {
          u32x2 q;
          __builtin_memcpy(&q, &nw[2 * v], 8);
          *reinterpret_cast<u32x2*>(row + 8 * v) = q;
        } else {
          *reinterpret_cast<uint32_t*>(row + 4 * v) = nw[v];
        }
      }
    } else {
      E* ce = reinterpret_cast<E*>(cb);
      const int64_t base = (tb + t) * cs_b + d * cs_d;
#pragma unroll
      for (int s = 0; s + 1 < S; ++s) ce[base + s * cs_s] = he[t][s + 1];
      ce[base + (S - 1) * cs_s] = xr[t];
    }
  }
  stage_basis();

  __syncthreads();

  // 4. W, k ascending (routes past K have zero weight and zero basis values)
  float w[T][S];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int s = 0; s < S; ++s) w[t][s] = 0.f;
  for (int k0 = 0; k0 < K; k0 += KT) {
    if (k0 > 0) {  // the next chunk, once every wave has read this one
      load_basis(k0);
      __syncthreads();
      stage_basis();
      __syncthreads();
    }
    float bv[R];
#pragma unroll
    for (int q = 0; q < R / 4; ++q) {
      const float4 v = *reinterpret_cast<const float4*>(&b_s[lane][4 * q]);
      bv[4 * q] = v.x;
      bv[4 * q + 1] = v.y;
      bv[4 * q + 2] = v.z;
      bv[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float a[KT];
#pragma unroll
      for (int q = 0; q < KT / 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(&a_s[wave][t][k0 + 4 * q]);
        a[4 * q] = v.x;
        a[4 * q + 1] = v.y;
        a[4 * q + 2] = v.z;
        a[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int kk = 0; kk < KT; ++kk)
#pragma unroll
        for (int s = 0; s < S; ++s) w[t][s] = fmaf(a[kk], bv[kk * S + s], w[t][s]);
    }
  }

  // 5. y = act(sum_{s < S-1} slot[s+1] W_s + x W_{S-1})
  auto to_f = [](E r) {
    if constexpr (F32) return __uint_as_float(r);
    else return bf16_to_f32(r);
  };
  E* ye = static_cast<E*>(y);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t >= nt || !d_ok) continue;
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) v = fmaf(to_f(s == S - 1 ? xr[t] : slot(t, s + 1)), w[t][s], v);
    if (activation) v = v * sigmoid_f(v);
    if constexpr (F32) ye[(tb + t) * D + d] = __float_as_uint(v);
    else ye[(tb + t) * D + d] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// Host launchers.

static inline unsigned grid_for(int64_t total, int threads, int64_t cap = 65536) {
  int64_t g = (total + threads - 1) / threads;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

void launch_prep(const Problem& p, const void* alpha, const void* basis, float* a_r,
                 float* basis_c, hipStream_t st) {
  hipLaunchKernelGGL(prep_alpha_kernel, dim3(grid_for(p.n_tokens, 256, 1LL << 30)), dim3(256),
                     0, st, alpha, p.a_dt, route_form(p.routing), p.n_tokens, p.K, a_r);
  const int64_t nb = p.K * p.S * p.D;
  hipLaunchKernelGGL(prep_basis_kernel, dim3(grid_for(nb, 256, 1LL << 30)), dim3(256), 0, st,
                     basis, p.b_dt, nb, p.x_dt, basis_c);
}

void launch_prep_alpha(const Problem& p, const void* alpha, float* a_r, hipStream_t st) {
  hipLaunchKernelGGL(prep_alpha_kernel, dim3(grid_for(p.n_tokens, 256, 1LL << 30)), dim3(256),
                     0, st, alpha, p.a_dt, route_form(p.routing), p.n_tokens, p.K, a_r);
}

void launch_forward_generic(const Problem& p, const void* x, const float* a_r,
                            const float* basis_c, void* y, hipStream_t st) {
  hipLaunchKernelGGL(fwd_generic_kernel, dim3(grid_for(p.n_tokens * p.D, 256)), dim3(256), 0,
                     st, x, p.x_dt, a_r, basis_c, y, p.seq, p.D, p.K, p.S, p.activation);
}

size_t generic_bwd_scratch_floats(const Problem& p) {
  const int64_t n_chunks = (p.n_tokens + kTokChunk - 1) / kTokChunk;
  return static_cast<size_t>(p.n_tokens * p.D + n_chunks * p.K * p.S * p.D);
}

void launch_backward_generic(const Problem& p, const void* x, const void* dy, void* dx,
                             void* dalpha, void* dbasis, const float* a_r,
                             const float* basis_c, float* scratch, hipStream_t st) {
  float* g = scratch;
  float* part = scratch + p.n_tokens * p.D;
  const int64_t n_chunks = (p.n_tokens + kTokChunk - 1) / kTokChunk;
  const unsigned ge = grid_for(p.n_tokens * p.D, 256);
  hipLaunchKernelGGL(bwd_g_kernel, dim3(ge), dim3(256), 0, st, x, dy, p.dy_stride, p.x_dt, a_r,
                     basis_c, g, p.seq, p.D, p.K, p.S, p.activation);
  if (dx != nullptr) {
    hipLaunchKernelGGL(bwd_dx_kernel, dim3(ge), dim3(256), 0, st, g, a_r, basis_c, dx, p.x_dt,
                       p.seq, p.D, p.K, p.S);
  }
  hipLaunchKernelGGL(bwd_dalpha_kernel, dim3(static_cast<unsigned>(p.n_tokens)),
                     dim3(kRedThreads), static_cast<size_t>(p.K) * sizeof(float), st, x, p.x_dt,
                     g, a_r, basis_c, dalpha, p.a_dt, route_grad(p.routing), p.seq, p.D, p.K,
                     p.S);
  hipLaunchKernelGGL(bwd_dbasis_partial_kernel,
                     dim3(static_cast<unsigned>((p.D + 255) / 256), static_cast<unsigned>(n_chunks)),
                     dim3(256), 0, st, x, p.x_dt, g, a_r, part, p.seq, p.D, p.K, p.S);
  const int64_t nb = p.K * p.S * p.D;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(grid_for(nb, 256, 1LL << 30)), dim3(256), 0, st,
                     part, n_chunks, nb, dbasis, p.b_dt);
}

void launch_update_generic(const void* x, const void* alpha, const void* basis, void* cache,
                           int64_t cs_b, int64_t cs_d, int64_t cs_s, void* y, int64_t B,
                           int64_t D, int64_t K, int64_t S, int x_dt, int a_dt, int b_dt,
                           int activation, int routing, hipStream_t st) {
  // (the wave kernel addresses the basis with 32-bit byte offsets)
  if (S >= 2 && S <= 16 && K <= kDecMaxK && K * S * D * 4 < (int64_t(1) << 31)) {
    const int es = x_dt == DT_F32 ? 4 : 2;
    const int vb = dec_row_vec_bytes(static_cast<int>(S), es);
    const bool row = cs_s == 1 && vb > 0 && reinterpret_cast<uintptr_t>(cache) % vb == 0 &&
                     (cs_d * es) % vb == 0 && (cs_b * es) % vb == 0;
    const int tpw = 4 * dec_tokens_per_wave(static_cast<int>(S));
    const dim3 wgrid(static_cast<unsigned>((D + 63) / 64), static_cast<unsigned>((B + tpw - 1) / tpw));
    const int k = static_cast<int>(K), rf = route_form(routing);
#define MOC_WAVE(S_, F32_, ROW_)                                                                   \
  hipLaunchKernelGGL((update_tile_kernel<S_, F32_, ROW_>), wgrid, dim3(256), 0, st, x, alpha, a_dt, rf, \
                     basis, b_dt, cache, cs_b, cs_d, cs_s, y, B, D, k, activation)
#define MOC_WAVE_S(S_)                                                                             \
  case S_:                                                                                         \
    if (x_dt == DT_F32) {                                                                          \
      if (row) MOC_WAVE(S_, true, true);                                                           \
      else MOC_WAVE(S_, true, false);                                                              \
    } else {                                                                                       \
      if (row) MOC_WAVE(S_, false, (dec_row_vec_bytes(S_, 2) > 0));                                \
      else MOC_WAVE(S_, false, false);                                                             \
    }                                                                                              \
    return;
    switch (S) {
      MOC_WAVE_S(2)
      MOC_WAVE_S(3)
      MOC_WAVE_S(4)
      MOC_WAVE_S(5)
      MOC_WAVE_S(6)
      MOC_WAVE_S(7)
      MOC_WAVE_S(8)
      MOC_WAVE_S(9)
      MOC_WAVE_S(10)
      MOC_WAVE_S(11)
      MOC_WAVE_S(12)
      MOC_WAVE_S(13)
      MOC_WAVE_S(14)
      MOC_WAVE_S(15)
      MOC_WAVE_S(16)
      default: break;
    }
#undef MOC_WAVE_S
#undef MOC_WAVE
  }
  dim3 grid(static_cast<unsigned>((D + 255) / 256), static_cast<unsigned>(B));
  hipLaunchKernelGGL(update_kernel, grid, dim3(256), static_cast<size_t>(K) * sizeof(float), st,
                     x, alpha, a_dt, route_form(routing), basis, b_dt, cache, cs_b, cs_d, cs_s, y, x_dt, D, K,
                     S, activation);
}

}  // namespace moc
