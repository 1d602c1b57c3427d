// fp32 layers whose route count the fp32 matrix-core tiles do not take in one
// piece, in route parts: the backward with 33-64 routes up to 8 taps (parts of
// 32) and with 17-64 routes at 9-16 taps (parts of 16), and the forward with
// 33-64 routes at 9-16 taps (halves of 32).  The fused fp32 tile does not
// build for four route chunks, and past 8 taps the fp32 forward spills at four
// chunks and the backward at two, but every part of the layer except the
// activation is linear in the routes (moc/kernels.py:36-439):
//   P      = sum over the parts of the forward without the activation;
//   y      = act(P);
//   g      = dy silu'(P) (without the activation dy itself, P not formed);
//   dx     = sum over the parts of the backward of (x, weights_i, basis_i) with
//            dy = g and no activation (its dx is sum_s g W_i);
//   dalpha = the router gradient (softmax / exp) over all K routes of the
//            weight gradients the parts return (routing "weights given");
//   dbasis = the parts' rows, each written in place.
// Each part runs the matrix-core kernels of its route count with fixed-order
// partial sums, and the parts are summed in order, so results are bitwise
// reproducible.
#include "moc_kernels.h"
#include "moc_mfma_launch.h"

namespace moc {
namespace mfma {

namespace {

constexpr size_t kAl = 256;
inline size_t al(size_t b) { return (b + kAl - 1) / kAl * kAl; }

// Routes per backward part: 32 up to 8 taps, 16 past (the fp32 two passes).
inline int64_t bwd_part(const Problem& p) { return p.S <= 8 ? 32 : 16; }
inline int64_t n_parts(int64_t K, int64_t h) { return (K + h - 1) / h; }
inline int64_t part_k(int64_t K, int64_t h, int64_t i) { return K - h * i < h ? K - h * i : h; }

// A part of k routes: no activation, its fp32 weights given, dy = g (fp32 rows).
Problem part_problem(const Problem& p, int64_t k) {
  Problem q = p;
  q.K = k;
  q.activation = 0;
  q.routing = ROUTE_ALPHA;
  q.a_dt = DT_F32;
  q.dy_stride = p.D;
  q.prof_start = q.prof_stop = nullptr;
  return q;
}

// The forward over all routes in one launch (no activation), where the tiles take it.
Problem p_problem(const Problem& p) {
  Problem q = p;
  q.activation = 0;
  q.routing = ROUTE_ALPHA;
  q.a_dt = DT_F32;
  q.prof_start = q.prof_stop = nullptr;
  return q;
}

// The forward in halves of 32 routes (33-64 routes past 8 taps), or in one piece.
bool fwd_in_halves(const Problem& p) { return !supported(p_problem(p)); }

struct SplitPlan {
  int64_t h, n;  // routes per backward part, parts
  size_t a_r, a_p, p, p1, g, dx1, da, ws_f, ws_b, total;
};

// Forward workspace of P: one launch, or each half's.
size_t fwd_ws(const Problem& p) {
  if (!fwd_in_halves(p)) return forward_workspace(p_problem(p));
  size_t w = forward_workspace(part_problem(p, 32));
  const size_t w1 = forward_workspace(part_problem(p, p.K - 32));
  return w1 > w ? w1 : w;
}

SplitPlan split_plan(const Problem& p, bool backward) {
  SplitPlan s{};
  s.h = bwd_part(p);
  s.n = n_parts(p.K, s.h);
  const size_t N = static_cast<size_t>(p.n_tokens), D = static_cast<size_t>(p.D);
  size_t off = 0;
  s.a_r = off; off += al(N * p.K * 4);
  s.a_p = off; off += al(N * p.K * 4);  // the parts' weights, part i from N h i
  s.p = off; off += al(N * D * 4);
  s.p1 = off; off += fwd_in_halves(p) ? al(N * D * 4) : 0;
  s.ws_f = off; off += al(fwd_ws(p));
  if (backward) {
    s.g = off; off += al(N * D * 4);
    s.dx1 = off; off += al(N * D * 4);
    s.da = off; off += al(N * p.K * 4);  // the parts' weight gradients, laid out as a_p
    size_t wb = 0;
    for (int64_t i = 0; i < s.n; ++i) {
      const size_t w = backward_workspace(part_problem(p, part_k(p.K, s.h, i)));
      if (w > wb) wb = w;
    }
    s.ws_b = off; off += al(wb);
  }
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

// y = act(y + t): the forward halves' sum with the activation
__global__ void sum_act_kernel(float* __restrict__ y, const float* __restrict__ t, int64_t n,
                               int activation) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = y[i] + t[i];
  y[i] = activation ? v * sigmoid_f(v) : v;
}

// dalpha [N, K] from the parts' weight gradients (part i of k_i routes at
// da + N h i, [N, k_i]) and the router gradient over all K routes on a_r; one
// 64-lane wave per token
__global__ void __launch_bounds__(64)
route_grad_kernel(const float* __restrict__ da, const float* __restrict__ a_r,
                  void* __restrict__ dalpha, int a_dt, int routing, int64_t N, int64_t K,
                  int64_t h) {
  const int64_t t = blockIdx.x;
  const int k = threadIdx.x;  // K <= 64
  const bool on = k < K;
  const int64_t i = k / h, kk = k - h * i;
  const int64_t ki = K - h * i < h ? K - h * i : h;
  const float v = on ? da[N * h * i + t * ki + kk] : 0.f;
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

// The columns of the routing weights a_r [N, K] in parts of h routes (part i
// from a_p + N h i).
void split_weights(const Problem& p, const float* a_r, float* a_p, int64_t h, hipStream_t st) {
  const int64_t N = p.n_tokens;
  for (int64_t i = 0; i < n_parts(p.K, h); ++i) {
    const int64_t k = part_k(p.K, h, i);
    hipLaunchKernelGGL(split_cols_kernel, dim3(grid_of(N * k, 256, 1LL << 30)), dim3(256), 0, st,
                       a_r, a_p + N * h * i, N, p.K, h * i, k);
  }
}

// P without the activation into P: one launch over a_r, or (fwd_in_halves)
// the halves of 32 routes, their weights split into a_p and the second half's
// P into P1, summed into P, with the activation applied when act_out.
void forward_p(const Problem& p, const void* x, const float* a_r, float* a_p, const void* basis,
               float* P, float* P1, void* ws, bool act_out, hipStream_t st) {
  const int64_t N = p.n_tokens, D = p.D;
  if (!fwd_in_halves(p)) {  // (the backward only: act_out is false)
    forward(p_problem(p), x, a_r, basis, P, ws, st);
    return;
  }
  split_weights(p, a_r, a_p, 32, st);
  const size_t esz_b = p.b_dt == DT_F32 ? 4 : 2;
  const char* b1 = static_cast<const char*>(basis) + static_cast<size_t>(32 * p.S * D) * esz_b;
  forward(part_problem(p, 32), x, a_p, basis, P, ws, st);
  forward(part_problem(p, p.K - 32), x, a_p + N * 32, b1, P1, ws, st);
  hipLaunchKernelGGL(sum_act_kernel, dim3(grid_of(N * D, 256, 1LL << 30)), dim3(256), 0, st, P, P1,
                     N * D, act_out && p.activation ? 1 : 0);
}

}  // namespace

bool routesplit_supported(const Problem& p) {
  if (p.x_dt != DT_F32 || p.K > 64 || p.S < 2 || p.S > 16) return false;
  if (p.S <= 8 ? p.K <= 32 : p.K <= 16) return false;  // one piece
  const int64_t h = bwd_part(p);
  // every part's backward, and P's forward, on the matrix cores
  if (!bwd_supported(part_problem(p, h)) || !bwd_supported(part_problem(p, part_k(p.K, h, n_parts(p.K, h) - 1))))
    return false;
  return routesplit_fwd_supported(p) || supported(p_problem(p));
}

bool routesplit_fwd_supported(const Problem& p) {
  return p.x_dt == DT_F32 && p.K > 32 && p.K <= 64 && p.S > 8 && p.S <= 16 &&
         supported(part_problem(p, 32)) && supported(part_problem(p, p.K - 32));
}

size_t routesplit_workspace(const Problem& p) { return split_plan(p, true).total; }

size_t routesplit_fwd_workspace(const Problem& p) { return split_plan(p, false).total; }

void forward_routesplit(const Problem& p, const void* x, const void* alpha, const void* basis,
                        void* y, void* workspace, hipStream_t st) {
  const SplitPlan s = split_plan(p, false);
  char* ws = static_cast<char*>(workspace);
  float* a_r = reinterpret_cast<float*>(ws + s.a_r);
  launch_prep_alpha(p, alpha, a_r, st);
  prof_begin(p, st);
  // (y is fp32: the first half's P lands there, the sum and activation in place)
  forward_p(p, x, a_r, reinterpret_cast<float*>(ws + s.a_p), basis, static_cast<float*>(y),
            reinterpret_cast<float*>(ws + s.p1), ws + s.ws_f, true, st);
  prof_end(p, st);
}

void backward_routesplit(const Problem& p, const void* x, const void* alpha, const void* basis,
                         const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                         hipStream_t st) {
  const SplitPlan s = split_plan(p, true);
  char* ws = static_cast<char*>(workspace);
  float* a_r = reinterpret_cast<float*>(ws + s.a_r);
  float* a_p = reinterpret_cast<float*>(ws + s.a_p);
  float* P = reinterpret_cast<float*>(ws + s.p);
  float* g = reinterpret_cast<float*>(ws + s.g);
  float* dx1 = reinterpret_cast<float*>(ws + s.dx1);
  float* da = reinterpret_cast<float*>(ws + s.da);
  const int64_t N = p.n_tokens, D = p.D;
  launch_prep_alpha(p, alpha, a_r, st);
  prof_begin(p, st);
  // with the activation: P over all routes (no activation), then g; without
  // it g is dy, which the parts read as it is (rows, one row or one element)
  const void* gsrc = dy;
  int64_t gstride = p.dy_stride;
  if (p.activation != 0) {
    forward_p(p, x, a_r, a_p, basis, P, reinterpret_cast<float*>(ws + s.p1), ws + s.ws_f, false, st);
    hipLaunchKernelGGL(g_kernel, dim3(grid_of(N * D, 256)), dim3(256), 0, st, P, dy, p.dy_stride,
                       p.x_dt, g, N, D, p.activation);
    gsrc = g;
    gstride = D;
  }
  // the parts' weights (the halves' split in forward_p shares a_p: the same
  // stream runs this after those forwards), then each part with dy = g
  split_weights(p, a_r, a_p, s.h, st);
  const size_t esz_b = p.b_dt == DT_F32 ? 4 : 2;
  for (int64_t i = 0; i < s.n; ++i) {
    const int64_t k = part_k(p.K, s.h, i);
    const size_t boff = static_cast<size_t>(s.h * i * p.S * D) * esz_b;
    Problem q = part_problem(p, k);
    q.dy_stride = gstride;
    backward(q, x, a_p + N * s.h * i, static_cast<const char*>(basis) + boff, gsrc,
             dx == nullptr ? nullptr : (i == 0 ? dx : dx1), da + N * s.h * i,
             static_cast<char*>(dbasis) + boff, ws + s.ws_b, st);
    if (i > 0 && dx != nullptr)
      hipLaunchKernelGGL(add_kernel, dim3(grid_of(N * D, 256, 1LL << 30)), dim3(256), 0, st,
                         static_cast<float*>(dx), dx1, N * D);
  }
  prof_end(p, st);
  hipLaunchKernelGGL(route_grad_kernel, dim3(static_cast<unsigned>(N)), dim3(64), 0, st, da, a_r,
                     dalpha, p.a_dt, route_grad(p.routing), N, p.K, s.h);
}

}  // namespace mfma
}  // namespace moc
