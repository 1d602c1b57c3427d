// Odd channel counts on the matrix-core kernels through a padded copy.  The
// tiles give each lane a pair of channels, so they take D even only.  With D
// odd the layer runs at D + 1 channels on copies of x, dy and basis with a zero
// last channel (in whichever form the padded shape takes: one launch family,
// route chunks or route parts), and y, dx and dbasis are copied back without
// it.  The extra
// channel changes nothing the caller sees: its x, dy and basis are zero, so its
// y is act(0) and dropped, its m products x dy are zero (dalpha sums over
// channels add exact zeros) and its dbasis is dropped.  Costs two passes over
// the rows on either side of the kernels, against the generic kernels' tens of
// times the matrix-core time.
#include "moc_kernels.h"

namespace moc {
namespace mfma {

namespace {

constexpr size_t kAl = 256;
inline size_t al(size_t b) { return (b + kAl - 1) / kAl * kAl; }

Problem padded(const Problem& p) {
  Problem q = p;
  q.D = p.D + 1;
  // dy rows: D elements apart becomes D + 1 (the padded copy); one row for
  // every token (0) is copied to one padded row; one element (-1) stays
  if (p.dy_stride == p.D) q.dy_stride = q.D;
  return q;
}

inline size_t esz(int dt) { return dt == DT_F32 ? 4 : 2; }

// dst [rows, D + 1] from src rows of D elements, src_stride elements apart,
// with a zero last column; one workgroup per row, so the column index is a
// 32-bit lane offset (no division per element).  Pairs of 16-bit elements go
// out as one 32-bit store (the padded rows have an even length).
template <typename T>
__global__ void __launch_bounds__(256)
pad_rows_kernel(const T* __restrict__ src, int64_t src_stride, T* __restrict__ dst, int64_t D) {
  const int64_t r = blockIdx.x;
  const T* s = src + r * src_stride;
  const int W = static_cast<int>(D) + 1;
  if constexpr (sizeof(T) == 2) {
    uint32_t* d = reinterpret_cast<uint32_t*>(dst + r * W);
    for (int c = 2 * static_cast<int>(threadIdx.x); c < W; c += 2 * 256) {
      const uint32_t lo = s[c];
      const uint32_t hi = c + 1 < D ? s[c + 1] : 0u;
      d[c / 2] = lo | (hi << 16);
    }
  } else {
    T* d = dst + r * W;
    for (int c = threadIdx.x; c < W; c += 256) d[c] = c < D ? s[c] : T(0);
  }
}

// dst [rows, D] from src [rows, D + 1] (the last column dropped); one
// workgroup per row
template <typename T>
__global__ void __launch_bounds__(256)
unpad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t D) {
  const int64_t r = blockIdx.x;
  const T* s = src + r * (D + 1);
  T* d = dst + r * D;
  for (int c = threadIdx.x; c < D; c += 256) d[c] = s[c];
}

void pad(const void* src, int64_t stride, void* dst, int64_t rows, int64_t D, int dt,
         hipStream_t st) {
  const dim3 g(static_cast<unsigned>(rows));
  if (esz(dt) == 4)
    hipLaunchKernelGGL(pad_rows_kernel<uint32_t>, g, dim3(256), 0, st,
                       static_cast<const uint32_t*>(src), stride, static_cast<uint32_t*>(dst), D);
  else
    hipLaunchKernelGGL(pad_rows_kernel<uint16_t>, g, dim3(256), 0, st,
                       static_cast<const uint16_t*>(src), stride, static_cast<uint16_t*>(dst), D);
}

void unpad(const void* src, void* dst, int64_t rows, int64_t D, int dt, hipStream_t st) {
  const dim3 g(static_cast<unsigned>(rows));
  if (esz(dt) == 4)
    hipLaunchKernelGGL(unpad_rows_kernel<uint32_t>, g, dim3(256), 0, st,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), D);
  else
    hipLaunchKernelGGL(unpad_rows_kernel<uint16_t>, g, dim3(256), 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), D);
}

// The padded problem's own forms: one launch family, or route chunks / parts.
size_t inner_ws(const Problem& q, bool backward) {
  if (!backward) return supported(q) ? forward_workspace(q) : routesplit_fwd_workspace(q);
  if (bwd_supported(q)) return backward_workspace(q);
  return chunks_supported(q) ? chunks_workspace(q) : routesplit_workspace(q);
}

struct PadPlan {
  size_t x, b, io, dy, db, inner, total;  // io: y (forward) or dx (backward)
};

PadPlan pad_plan(const Problem& p, bool backward) {
  const Problem q = padded(p);
  const size_t N = static_cast<size_t>(p.n_tokens), W = static_cast<size_t>(q.D);
  const size_t KS = static_cast<size_t>(p.K * p.S);
  PadPlan s{};
  size_t off = 0;
  s.x = off; off += al(N * W * esz(p.x_dt));
  s.b = off; off += al(KS * W * esz(p.b_dt));
  s.io = off; off += al(N * W * esz(p.x_dt));
  if (backward) {
    s.dy = off; off += p.dy_stride < 0 ? 0 : al((p.dy_stride == 0 ? 1 : N) * W * esz(p.x_dt));
    s.db = off; off += al(KS * W * esz(p.b_dt));
  }
  s.inner = off; off += al(inner_ws(q, backward));
  s.total = off;
  return s;
}

}  // namespace

bool pad_supported(const Problem& p, bool backward) {
  if (p.D % 2 == 0 || p.D + 1 > (int64_t(1) << 20)) return false;
  const Problem q = padded(p);
  return backward ? bwd_supported(q) || chunks_supported(q) || routesplit_supported(q)
                  : supported(q) || routesplit_fwd_supported(q);
}

size_t pad_workspace(const Problem& p, bool backward) { return pad_plan(p, backward).total; }

void forward_padded(const Problem& p, const void* x, const void* alpha, const void* basis, void* y,
                    void* workspace, hipStream_t st) {
  const Problem q = padded(p);
  const PadPlan s = pad_plan(p, false);
  char* ws = static_cast<char*>(workspace);
  pad(x, p.D, ws + s.x, p.n_tokens, p.D, p.x_dt, st);
  pad(basis, p.D, ws + s.b, p.K * p.S, p.D, p.b_dt, st);
  if (supported(q)) forward(q, ws + s.x, alpha, ws + s.b, ws + s.io, ws + s.inner, st);
  else forward_routesplit(q, ws + s.x, alpha, ws + s.b, ws + s.io, ws + s.inner, st);
  unpad(ws + s.io, y, p.n_tokens, p.D, p.x_dt, st);
}

void backward_padded(const Problem& p, const void* x, const void* alpha, const void* basis,
                     const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                     hipStream_t st) {
  const Problem q = padded(p);
  const PadPlan s = pad_plan(p, true);
  char* ws = static_cast<char*>(workspace);
  pad(x, p.D, ws + s.x, p.n_tokens, p.D, p.x_dt, st);
  pad(basis, p.D, ws + s.b, p.K * p.S, p.D, p.b_dt, st);
  const void* dyq = dy;
  if (p.dy_stride >= 0) {
    pad(dy, p.dy_stride, ws + s.dy, p.dy_stride == 0 ? 1 : p.n_tokens, p.D, p.x_dt, st);
    dyq = ws + s.dy;
  }
  void* dxq = dx != nullptr ? ws + s.io : nullptr;
  if (bwd_supported(q))
    backward(q, ws + s.x, alpha, ws + s.b, dyq, dxq, dalpha, ws + s.db, ws + s.inner, st);
  else if (chunks_supported(q))
    backward_chunks(q, ws + s.x, alpha, ws + s.b, dyq, dxq, dalpha, ws + s.db, ws + s.inner, st);
  else
    backward_routesplit(q, ws + s.x, alpha, ws + s.b, dyq, dxq, dalpha, ws + s.db, ws + s.inner, st);
  if (dx != nullptr) unpad(ws + s.io, dx, p.n_tokens, p.D, p.x_dt, st);
  unpad(ws + s.db, dbasis, p.K * p.S, p.D, p.b_dt, st);
}

}  // namespace mfma
}  // namespace moc
