// Backward of fp32 layers with 33 to 64 routes on the matrix cores, in two
// halves of at most 32 routes.  The fused fp32 tile does not build for four
// route chunks, but every part of the backward except g is linear in the
// routes once g is known (moc/kernels.py:156-439):
//   g      = dy silu'(P) (or dy), P from the forward kernel over all routes
//            without the activation;
//   dx     = sum over the halves of the backward of (x, weights_h, basis_h) with
//            dy = g and no activation (its dx is sum_s g W_h);
//   dalpha = the router gradient (softmax / exp) over all K routes of the
//            weight gradients the halves return (routing "weights given");
//   dbasis = the halves' rows, each written in place.
// The halves run the 32-route fp32 backward (fused pass, fixed-order partial
// sums), so results are bitwise reproducible.
#include "moc_kernels.h"
#include "moc_mfma_launch.h"

namespace moc {
namespace mfma {

namespace {

constexpr size_t kAl = 256;
inline size_t al(size_t b) { return (b + kAl - 1) / kAl * kAl; }

struct SplitPlan {
  int64_t k0, k1;  // routes of the halves: [0, k0), [k0, k0 + k1)
  size_t a_r, a_h0, a_h1, p, g, dx1, da, ws_f, ws_b, total;
};

Problem half_problem(const Problem& p, int64_t k) {
  Problem q = p;
  q.K = k;
  q.activation = 0;
  q.routing = ROUTE_ALPHA;  // the halves' weights are given (fp32)
  q.a_dt = DT_F32;
  q.dy_stride = p.D;        // dy = g, fp32 rows
  q.prof_start = q.prof_stop = nullptr;
  return q;
}

Problem p_problem(const Problem& p) {
  Problem q = p;
  q.activation = 0;
  q.routing = ROUTE_ALPHA;
  q.a_dt = DT_F32;
  q.prof_start = q.prof_stop = nullptr;
  return q;
}

SplitPlan split_plan(const Problem& p) {
  SplitPlan s{};
  s.k0 = 32;
  s.k1 = p.K - 32;
  const size_t N = static_cast<size_t>(p.n_tokens), D = static_cast<size_t>(p.D);
  size_t off = 0;
  s.a_r = off; off += al(N * p.K * 4);
  s.a_h0 = off; off += al(N * s.k0 * 4);
  s.a_h1 = off; off += al(N * s.k1 * 4);
  s.p = off; off += al(N * D * 4);
  s.g = off; off += al(N * D * 4);
  s.dx1 = off; off += al(N * D * 4);
  s.da = off; off += al(N * p.K * 4);
  s.ws_f = off; off += al(forward_workspace(p_problem(p)));
  size_t wb = backward_workspace(half_problem(p, s.k0));
  const size_t wb1 = backward_workspace(half_problem(p, s.k1));
  if (wb1 > wb) wb = wb1;
  s.ws_b = off; off += al(wb);
  s.total = off;
  return s;
}

// columns [c0, c0 + kh) of a_r [N, K] into a [N, kh]
__global__ void split_cols_kernel(const float* __restrict__ a_r, float* __restrict__ a, int64_t N,
                                  int64_t K, int64_t c0, int64_t kh) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * kh) return;
  const int64_t t = i / kh, k = i - t * kh;
  a[i] = a_r[t * K + c0 + k];
}

// g = dy silu'(P) (activation) or dy, fp32; dy rows dys elements apart (0: one
// row for every token, -1: one element)
__global__ void g_kernel(const float* __restrict__ P, const void* __restrict__ dy, int64_t dys,
                         int x_dt, float* __restrict__ g, int64_t N, int64_t D, int activation) {
  const int64_t total = N * D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / D, d = i - t * D;
    float gv = load_any(dy, x_dt, dys < 0 ? 0 : t * dys + d);
    if (activation) {
      const float p = P[i];
      const float sg = sigmoid_f(p);
      gv = gv * (sg * (1.0f + p * (1.0f - sg)));  // moc/kernels.py:231-232
    }
    g[i] = gv;
  }
}

__global__ void add_kernel(float* __restrict__ dx, const float* __restrict__ dx1, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dx[i] += dx1[i];
}

// dalpha [N, K] from the halves' weight gradients da = [da0 | da1] ([N, k0]
// then [N, k1]) and the router gradient over all K routes on a_r; one 64-lane
// wave per token
__global__ void __launch_bounds__(64)
route_grad_kernel(const float* __restrict__ da0, const float* __restrict__ da1,
                  const float* __restrict__ a_r, void* __restrict__ dalpha, int a_dt, int routing,
                  int64_t K, int64_t k0) {
  const int64_t t = blockIdx.x;
  const int64_t k1 = K - k0;
  const int k = threadIdx.x;  // K <= 64
  const bool on = k < K;
  const float v = !on ? 0.f : (k < k0 ? da0[t * k0 + k] : da1[t * k1 + (k - k0)]);
  const float a = on ? a_r[t * K + k] : 0.f;
  float dot = a * v;
  for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
  float r = v;
  if (routing == ROUTE_SOFTMAX) r = a * (v - dot);
  else if (routing == ROUTE_EXP) r = a * v;
  if (on) store_any(dalpha, a_dt, t * K + k, r);
}

inline unsigned grid_of(int64_t total, int threads, int64_t cap = 65536) {
  int64_t g = (total + threads - 1) / threads;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<unsigned>(g);
}

}  // namespace

bool routesplit_supported(const Problem& p) {
  return p.x_dt == DT_F32 && p.K > 32 && p.K <= 64 && p.S <= 8 && supported(p) &&
         bwd_supported(half_problem(p, 32));
}

size_t routesplit_workspace(const Problem& p) { return split_plan(p).total; }

void backward_routesplit(const Problem& p, const void* x, const void* alpha, const void* basis,
                         const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                         hipStream_t st) {
  const SplitPlan s = split_plan(p);
  char* ws = static_cast<char*>(workspace);
  float* a_r = reinterpret_cast<float*>(ws + s.a_r);
  float* a_h0 = reinterpret_cast<float*>(ws + s.a_h0);
  float* a_h1 = reinterpret_cast<float*>(ws + s.a_h1);
  float* P = reinterpret_cast<float*>(ws + s.p);
  float* g = reinterpret_cast<float*>(ws + s.g);
  float* dx1 = reinterpret_cast<float*>(ws + s.dx1);
  float* da0 = reinterpret_cast<float*>(ws + s.da);
  float* da1 = da0 + p.n_tokens * s.k0;
  const int64_t N = p.n_tokens, D = p.D;
  // the routing weights as the router activation forms them (fp32), and the halves
  launch_prep_alpha(p, alpha, a_r, st);
  hipLaunchKernelGGL(split_cols_kernel, dim3(grid_of(N * s.k0, 256, 1LL << 30)), dim3(256), 0, st,
                     a_r, a_h0, N, p.K, int64_t(0), s.k0);
  hipLaunchKernelGGL(split_cols_kernel, dim3(grid_of(N * s.k1, 256, 1LL << 30)), dim3(256), 0, st,
                     a_r, a_h1, N, p.K, s.k0, s.k1);
  prof_begin(p, st);
  // P over all routes (the forward kernel without the activation), then g
  forward(p_problem(p), x, a_r, basis, P, ws + s.ws_f, st);
  hipLaunchKernelGGL(g_kernel, dim3(grid_of(N * D, 256)), dim3(256), 0, st, P, dy, p.dy_stride,
                     p.x_dt, g, N, D, p.activation);
  // the halves: dy = g, no activation, weights given
  const size_t esz_b = p.b_dt == DT_F32 ? 4 : 2;
  const char* b1 = static_cast<const char*>(basis) + static_cast<size_t>(s.k0 * p.S * D) * esz_b;
  char* db1 = static_cast<char*>(dbasis) + static_cast<size_t>(s.k0 * p.S * D) * esz_b;
  backward(half_problem(p, s.k0), x, a_h0, basis, g, dx, da0, dbasis, ws + s.ws_b, st);
  backward(half_problem(p, s.k1), x, a_h1, b1, g, dx != nullptr ? dx1 : nullptr, da1, db1,
           ws + s.ws_b, st);
  prof_end(p, st);
  if (dx != nullptr)
    hipLaunchKernelGGL(add_kernel, dim3(grid_of(N * D, 256, 1LL << 30)), dim3(256), 0, st,
                       static_cast<float*>(dx), dx1, N * D);
  hipLaunchKernelGGL(route_grad_kernel, dim3(static_cast<unsigned>(N)), dim3(64), 0, st, da0, da1,
                     a_r, dalpha, p.a_dt, route_grad(p.routing), p.K, s.k0);
}

}  // namespace mfma
}  // namespace moc
