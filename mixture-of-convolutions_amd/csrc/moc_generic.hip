// Generic MoC kernels: any K, any kernel size S, any storage dtypes.
//
// One lane per (token, channel) element; the mixture W[n,s,d] = sum_k a[n,k] b[k,s,d]
// is formed on VALU.  These kernels serve shapes outside the MFMA kernels'
// instantiations (moc_mfma.hip) and the decode step.  They keep the reference's
// semantics (moc/kernels.py:36-142 forward, 156-268 dx, 282-426 dalpha/dbasis,
// 442-550 decode) but reduce dalpha / dbasis in a fixed order instead of atomics.
#include "moc_common.h"
#include "moc_kernels.h"

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
// or fp16 data, mixed storage dtypes, strided caches, any D), 2 to 8 taps and
// up to 64 routes; same arithmetic and order as update_kernel, so the two give
// the same bits.  A block covers 16 tokens x 64 channels: the 16 tokens'
// routing weights are formed once per block in LDS (thread t < 16: token t),
// and each thread takes one channel of 4 tokens, loading each basis value once
// for the 4 and issuing a tap's loads together (update_kernel waits for one
// load per routing weight and tap).
constexpr int kTileMaxK = 64;

// Typed element loads for the tile kernel: the storage dtype is chosen once per
// loop (a uniform branch around it), so a loop's loads issue back to back.
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

template <int S>
__global__ void __launch_bounds__(256)
update_tile_kernel(const void* __restrict__ x, const void* __restrict__ alpha, int a_dt, int routing,
                   const void* __restrict__ basis, int b_dt, void* __restrict__ cache, int64_t cs_b,
                   int64_t cs_d, int64_t cs_s, void* __restrict__ y, int x_dt, int64_t B, int64_t D,
                   int K, int activation) {
  // basis values of the first KT routes x S taps are loaded with everything
  // else before the routing weights are formed (one memory round trip for all
  // of them); further routes in chunks of KT
  constexpr int KT = S <= 4 ? 16 : 8;
  __shared__ float l_s[16][kTileMaxK + 1];
  __shared__ float a_s[16][kTileMaxK];
  const int tid = threadIdx.x;
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * 16;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + (tid & 63);
  const bool d_ok = d < D;
  // loads are issued by every lane at a valid index (element 0 where the lane
  // has nothing to load) and their values selected: a load under a per-lane
  // condition compiles to a divergent branch that waits for it
  const int64_t dc = d_ok ? d : 0;
  const int tg = tid >> 6;  // this thread's tokens b0 + 4 tg + u, u < 4
  int64_t bt[4];
  bool on[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    bt[u] = b0 + 4 * tg + u;
    on[u] = d_ok && bt[u] < B;
  }
  char* cb = static_cast<char*>(cache);

  // 1. every load that does not depend on the routing weights
  // the 16 tokens' logits (or weights): token tid / 16, entries tid % 16 + 16 i
  float lr[kTileMaxK / 16];
  {
    const int tk = tid >> 4, k0 = tid & 15;
    const bool tok = b0 + tk < B;
    with_dtype(a_dt, [&](auto t) {
#pragma unroll
      for (int i = 0; i < kTileMaxK / 16; ++i) {
        const int k = k0 + 16 * i;
        const bool in = tok && k < K;
        const float v = ld(alpha, in ? (b0 + tk) * K + k : 0, t);
        lr[i] = in ? v : 0.f;
      }
    });
  }
  // x and the cache slots the output reads (slots 1 .. S-1 of each token's row),
  // as raw bits (the shift below moves them unchanged)
  uint32_t xr[4], hr[4][S];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t xi = on[u] ? bt[u] * D + d : 0, ci = on[u] ? bt[u] * cs_b + d * cs_d : 0;
    const int64_t cs = on[u] ? cs_s : 0;
    if (x_dt == DT_F32) {
      xr[u] = static_cast<const uint32_t*>(x)[xi];
#pragma unroll
      for (int s = 1; s < S; ++s) hr[u][s] = reinterpret_cast<const uint32_t*>(cb)[ci + s * cs];
    } else {
      xr[u] = static_cast<const uint16_t*>(x)[xi];
#pragma unroll
      for (int s = 1; s < S; ++s) hr[u][s] = reinterpret_cast<const uint16_t*>(cb)[ci + s * cs];
    }
  }
  // basis[k][s][d] of the first KT routes
  float bv[KT][S];
  auto load_basis = [&](int k0) {
    with_dtype(b_dt, [&](auto t) {
#pragma unroll
      for (int kk = 0; kk < KT; ++kk)
#pragma unroll
        for (int s = 0; s < S; ++s)
        {
          const bool in = k0 + kk < K;
          const float v = ld(basis, (static_cast<int64_t>(in ? k0 + kk : 0) * S + s) * D + dc, t);
          bv[kk][s] = in ? v : 0.f;
        }
    });
  };
  load_basis(0);

  // 2. routing weights in update_kernel's order and rounding (thread t < 16: token t)
  {
    const int tk = tid >> 4, k0 = tid & 15;
#pragma unroll
    for (int i = 0; i < kTileMaxK / 16; ++i) l_s[tk][k0 + 16 * i] = lr[i];
  }
  __syncthreads();
  if (tid < 16 && b0 + tid < B) {
    float m = -INFINITY, sum = 0.f;
    if (routing == ROUTE_SOFTMAX) {
      for (int k = 0; k < K; ++k) m = fmaxf(m, l_s[tid][k]);
      for (int k = 0; k < K; ++k) sum += __expf(l_s[tid][k] - m);
    }
    for (int k = 0; k < K; ++k) {
      const float l = l_s[tid][k];
      float a = l;
      if (routing == ROUTE_SOFTMAX) a = round_to(__expf(l - m) * (1.0f / sum), a_dt);
      else if (routing == ROUTE_EXP) a = round_to(__expf(l), a_dt);
      a_s[tid][k] = round_to(a, x_dt);
    }
  }
  __syncthreads();
  if (!d_ok) return;  // (after the block's barriers)

  // 3. W[u][s] = sum_k alpha[u][k] basis[k][s][d], k ascending
  float w[4][S];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int s = 0; s < S; ++s) w[u][s] = 0.f;
  for (int k0 = 0; k0 < K; k0 += KT) {
    if (k0 > 0) load_basis(k0);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      if (k0 + kk < K) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const float b = round_to(bv[kk][s], x_dt);
#pragma unroll
          for (int u = 0; u < 4; ++u) w[u][s] = fmaf(a_s[4 * tg + u][k0 + kk], b, w[u][s]);
        }
      }
    }
  }
  const bool f32 = x_dt == DT_F32;
  auto to_f = [&](uint32_t r) { return f32 ? __uint_as_float(r) : bf16_to_f32(static_cast<uint16_t>(r)); };
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (!on[u]) continue;
    float v = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) v = fmaf(to_f(s == S - 1 ? xr[u] : hr[u][s + 1]), w[u][s], v);
    if (activation) v = v * sigmoid_f(v);
    store_any(y, x_dt, bt[u] * D + d, v);
    // shift the history one slot left (pure copies: bit-exact), append x
    const int64_t cbase = bt[u] * cs_b + d * cs_d;
    if (f32) {
      uint32_t* c = reinterpret_cast<uint32_t*>(cb);
#pragma unroll
      for (int s = 0; s + 1 < S; ++s) c[cbase + s * cs_s] = hr[u][s + 1];
      c[cbase + (S - 1) * cs_s] = xr[u];
    } else {
      uint16_t* c = reinterpret_cast<uint16_t*>(cb);
#pragma unroll
      for (int s = 0; s + 1 < S; ++s) c[cbase + s * cs_s] = static_cast<uint16_t>(hr[u][s + 1]);
      c[cbase + (S - 1) * cs_s] = static_cast<uint16_t>(xr[u]);
    }
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
  if (S >= 2 && S <= 8 && K <= kTileMaxK) {
    const dim3 tgrid(static_cast<unsigned>((D + 63) / 64), static_cast<unsigned>((B + 15) / 16));
    const int k = static_cast<int>(K), rf = route_form(routing);
#define MOC_TILE(S_)                                                                                 \
  case S_:                                                                                           \
    hipLaunchKernelGGL(update_tile_kernel<S_>, tgrid, dim3(256), 0, st, x, alpha, a_dt, rf, basis, b_dt, \
                       cache, cs_b, cs_d, cs_s, y, x_dt, B, D, k, activation);                       \
    return;
    switch (S) {
      MOC_TILE(2)
      MOC_TILE(3)
      MOC_TILE(4)
      MOC_TILE(5)
      MOC_TILE(6)
      MOC_TILE(7)
      MOC_TILE(8)
      default: break;
    }
#undef MOC_TILE
  }
  dim3 grid(static_cast<unsigned>((D + 255) / 256), static_cast<unsigned>(B));
  hipLaunchKernelGGL(update_kernel, grid, dim3(256), static_cast<size_t>(K) * sizeof(float), st,
                     x, alpha, a_dt, route_form(routing), basis, b_dt, cache, cs_b, cs_d, cs_s, y, x_dt, D, K,
                     S, activation);
}

}  // namespace moc
