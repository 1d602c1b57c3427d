// C ABI of libmoc_hip.so (declared in include/moc_hip.h): argument checks,
// workspace carving and dispatch to the kernels.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/moc_hip.h"
#include "moc_kernels.h"

namespace {

thread_local char g_err[512] = "";
thread_local hipEvent_t g_prof_start = nullptr;
thread_local hipEvent_t g_prof_stop = nullptr;
// kernel family override of moc_set_kernel_path (process-wide)
std::atomic<int> g_path{MOC_PATH_AUTO};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool dt_ok(int dt) { return dt == MOC_DT_F32 || dt == MOC_DT_BF16 || dt == MOC_DT_F16; }

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Largest extents the launch grids are sized for.
constexpr int64_t kMaxTokens = int64_t(1) << 31;
constexpr int64_t kMaxBatch = 65535;
constexpr int64_t kMaxK = 4096;   // dynamic LDS of the reduction kernels holds K floats
constexpr int64_t kMaxS = 1024;

int check_dims(int64_t n_tokens, int64_t dim, int64_t k, int64_t ks) {
  if (n_tokens <= 0 || dim <= 0 || k <= 0 || ks <= 0)
    return fail(MOC_ERR_ARG, "n_tokens, dim, k and kernel_size must be positive "
                             "(got %lld, %lld, %lld, %lld)",
                (long long)n_tokens, (long long)dim, (long long)k, (long long)ks);
  if (n_tokens >= kMaxTokens) return fail(MOC_ERR_ARG, "n_tokens too large: %lld", (long long)n_tokens);
  if (k > kMaxK) return fail(MOC_ERR_ARG, "k too large: %lld (max %lld)", (long long)k, (long long)kMaxK);
  if (ks > kMaxS)
    return fail(MOC_ERR_ARG, "kernel_size too large: %lld (max %lld)", (long long)ks, (long long)kMaxS);
  return MOC_OK;
}

int check_common(int x_dt, int a_dt, int b_dt, int activation, int routing) {
  if (x_dt != MOC_DT_F32 && x_dt != MOC_DT_BF16)
    return fail(MOC_ERR_DTYPE, "unsupported x dtype code %d (bf16 or f32 only)", x_dt);
  if (!dt_ok(a_dt)) return fail(MOC_ERR_DTYPE, "unsupported alpha dtype code %d", a_dt);
  if (!dt_ok(b_dt)) return fail(MOC_ERR_DTYPE, "unsupported basis dtype code %d", b_dt);
  if (activation != 0 && activation != 1)
    return fail(MOC_ERR_ARG, "activation must be 0 or 1, got %d", activation);
  if (routing < MOC_ROUTE_ALPHA || routing > MOC_ROUTE_EXP_WEIGHTS)
    return fail(MOC_ERR_ARG, "routing must be 0, 1, 2, 3 or 4, got %d", routing);
  return MOC_OK;
}

struct Carve {
  char* base;
  size_t used;
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base + used);
    used += align_up(count * sizeof(T));
    return p;
  }
};

size_t fwd_bytes(int64_t n, int64_t d, int64_t k, int64_t s) {
  return align_up(size_t(n * k) * 4) + align_up(size_t(k * s * d) * 4);
}

size_t bwd_bytes(const moc::Problem& p) {
  return fwd_bytes(p.n_tokens, p.D, p.K, p.S) +
         align_up(moc::generic_bwd_scratch_floats(p) * 4);
}

moc::Problem make_problem(const void* cu, int cu64, int64_t n_seqs, int64_t n_tokens,
                          int64_t seq_len, int64_t dim, int64_t k, int64_t ks, int x_dt,
                          int a_dt, int b_dt, int activation, int routing) {
  moc::Problem p;
  p.seq.cu = cu;
  p.seq.cu64 = cu64 ? 1 : 0;
  p.seq.n_seqs = n_seqs;
  p.seq.seq_len = seq_len;
  p.seq.n_tokens = n_tokens;
  p.n_tokens = n_tokens;
  p.D = dim;
  p.K = k;
  p.S = ks;
  p.x_dt = x_dt;
  p.a_dt = a_dt;
  p.b_dt = b_dt;
  p.activation = activation;
  p.routing = routing;
  p.dy_stride = dim;
  p.path = g_path.load(std::memory_order_relaxed);
  p.prof_start = g_prof_start;
  p.prof_stop = g_prof_stop;
  return p;
}

int check_seq(const void* cu, int64_t n_seqs, int64_t seq_len) {
  if (cu == nullptr && seq_len <= 0)
    return fail(MOC_ERR_ARG, "seq_len must be positive for fixed-length inputs");
  if (cu != nullptr && n_seqs <= 0)
    return fail(MOC_ERR_ARG, "n_seqs must be positive when cu_seqlens is given");
  return MOC_OK;
}

// Kernel family for a problem: the MFMA kernels where they are instantiated,
// the generic kernels otherwise, or the generic kernels for every problem while
// moc_set_kernel_path(MOC_PATH_GENERIC) holds (used to cross-check the two).
bool use_mfma(const moc::Problem& p) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return moc::mfma::supported(p);
}
// the backward's family (the matrix-core backward covers fewer shapes)
bool use_mfma_bwd(const moc::Problem& p) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return moc::mfma::bwd_supported(p);
}
// fp32 forward with 33-64 routes at 9-16 taps: route halves on the matrix cores
bool use_routesplit_fwd(const moc::Problem& p) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return !moc::mfma::supported(p) && moc::mfma::routesplit_fwd_supported(p);
}
// fp32 backward with 33-64 routes up to 8 taps or 17-64 at 9-16: route parts on
// the matrix cores
bool use_routesplit(const moc::Problem& p) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return !moc::mfma::bwd_supported(p) && moc::mfma::routesplit_supported(p);
}
// bf16 with 9-16 taps and 17-64 routes: the dx pass, then the taps pass per
// 16-route chunk
bool use_chunks(const moc::Problem& p) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return !moc::mfma::bwd_supported(p) && moc::mfma::chunks_supported(p);
}

// odd channel counts: the matrix-core kernels on a zero-padded copy
bool use_pad(const moc::Problem& p, bool backward) {
  if (p.path == MOC_PATH_GENERIC) return false;
  return moc::mfma::pad_supported(p, backward);
}

size_t forward_bytes(const moc::Problem& p) {
  if (use_mfma(p)) return moc::mfma::forward_workspace(p);
  if (use_pad(p, false)) return moc::mfma::pad_workspace(p, false);
  if (use_routesplit_fwd(p)) return moc::mfma::routesplit_fwd_workspace(p);
  return fwd_bytes(p.n_tokens, p.D, p.K, p.S);
}

size_t backward_bytes(const moc::Problem& p) {
  if (use_mfma_bwd(p)) return moc::mfma::backward_workspace(p);
  if (use_pad(p, true)) return moc::mfma::pad_workspace(p, true);
  if (use_chunks(p)) return moc::mfma::chunks_workspace(p);
  return use_routesplit(p) ? moc::mfma::routesplit_workspace(p) : bwd_bytes(p);
}

int hip_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MOC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MOC_OK;
}

}  // namespace

extern "C" {

int moc_abi_version(void) { return 5; }

const char* moc_last_error(void) { return g_err; }

int moc_set_kernel_path(int path) {
  if (path != MOC_PATH_AUTO && path != MOC_PATH_GENERIC && path != MOC_PATH_MFMA_PREP)
    return fail(MOC_ERR_ARG, "kernel path must be 0, 1 or 2, got %d", path);
  return g_path.exchange(path, std::memory_order_relaxed);
}

int moc_profile_events(void* start_event, void* stop_event) {
  g_prof_start = static_cast<hipEvent_t>(start_event);
  g_prof_stop = static_cast<hipEvent_t>(stop_event);
  return MOC_OK;
}

size_t moc_forward_workspace_bytes(int64_t n_tokens, int64_t dim, int64_t k,
                                   int64_t kernel_size, int x_dtype, int routing) {
  if (n_tokens <= 0 || dim <= 0 || k <= 0 || kernel_size <= 0) return 0;
  moc::Problem p = make_problem(nullptr, 0, 0, n_tokens, n_tokens, dim, k, kernel_size, x_dtype,
                                MOC_DT_F32, MOC_DT_F32, 0, routing);
  return forward_bytes(p);
}

int moc_forward(const void* x, const void* alpha, const void* basis, void* y,
                const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                int64_t n_tokens, int64_t seq_len, int64_t dim, int64_t k, int64_t kernel_size,
                int x_dtype, int alpha_dtype, int basis_dtype, int activation, int routing,
                void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  int rc;
  if ((rc = check_dims(n_tokens, dim, k, kernel_size)) != MOC_OK) return rc;
  if ((rc = check_common(x_dtype, alpha_dtype, basis_dtype, activation, routing)) != MOC_OK) return rc;
  if ((rc = check_seq(cu_seqlens, n_seqs, seq_len)) != MOC_OK) return rc;
  if (!x || !alpha || !basis || !y) return fail(MOC_ERR_ARG, "null tensor pointer");
  moc::Problem p = make_problem(cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens, seq_len, dim, k,
                                kernel_size, x_dtype, alpha_dtype, basis_dtype, activation,
                                routing);
  const size_t need = forward_bytes(p);
  if (workspace_bytes < need || (need && !workspace))
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_mfma(p)) {
    moc::mfma::forward(p, x, alpha, basis, y, workspace, st);
    return hip_status("moc_forward launch");
  }
  if (use_routesplit_fwd(p)) {
    moc::mfma::forward_routesplit(p, x, alpha, basis, y, workspace, st);
    return hip_status("moc_forward launch");
  }
  if (use_pad(p, false)) {
    moc::mfma::forward_padded(p, x, alpha, basis, y, workspace, st);
    return hip_status("moc_forward launch");
  }
  Carve cv{static_cast<char*>(workspace), 0};
  float* a_r = cv.take<float>(size_t(n_tokens * k));
  float* basis_c = cv.take<float>(size_t(k * kernel_size * dim));
  moc::launch_prep(p, alpha, basis, a_r, basis_c, st);
  moc::prof_begin(p, st);
  moc::launch_forward_generic(p, x, a_r, basis_c, y, st);
  moc::prof_end(p, st);
  return hip_status("moc_forward launch");
}

size_t moc_backward_workspace_bytes(int64_t n_tokens, int64_t dim, int64_t k,
                                    int64_t kernel_size, int x_dtype, int routing) {
  if (n_tokens <= 0 || dim <= 0 || k <= 0 || kernel_size <= 0) return 0;
  // the activation is not an argument, and the kernel plan depends on it (bf16
  // two-pass shapes: the taps pass's partials, and with SiLU the g buffer);
  // the same query serves moc_backward_prefill, whose plan keeps the fused
  // pass at some shapes where the plain backward runs two (another grid, so
  // other partial sizes): the larger of every plan
  size_t need = 0;
  for (int act = 0; act <= 1; ++act)
    for (int pre = 0; pre <= 1; ++pre) {
      moc::Problem p = make_problem(nullptr, 0, 0, n_tokens, n_tokens, dim, k, kernel_size,
                                    x_dtype, MOC_DT_F32, MOC_DT_F32, act, routing);
      p.pre = pre != 0;
      const size_t b = backward_bytes(p);
      if (b > need) need = b;
    }
  return need;
}

}  // extern "C"

namespace {

// Checks of moc_backward / moc_backward_noalloc; fills p.
int backward_problem(const void* x, const void* alpha, const void* basis, const void* dy,
                     int64_t dy_row_stride, void* dalpha, void* dbasis, const void* cu_seqlens,
                     int cu_seqlens_i64, int64_t n_seqs, int64_t n_tokens, int64_t seq_len,
                     int64_t dim, int64_t k, int64_t kernel_size, int x_dtype, int alpha_dtype,
                     int basis_dtype, int activation, int routing, moc::Problem& p) {
  int rc;
  if ((rc = check_dims(n_tokens, dim, k, kernel_size)) != MOC_OK) return rc;
  if ((rc = check_common(x_dtype, alpha_dtype, basis_dtype, activation, routing)) != MOC_OK) return rc;
  if ((rc = check_seq(cu_seqlens, n_seqs, seq_len)) != MOC_OK) return rc;
  if (!x || !alpha || !basis || !dy || !dalpha || !dbasis)
    return fail(MOC_ERR_ARG, "null tensor pointer");
  if (dy_row_stride != 0 && dy_row_stride != dim && dy_row_stride != -1)
    return fail(MOC_ERR_ARG, "dy_row_stride must be dim (%lld), 0 or -1, got %lld",
                (long long)dim, (long long)dy_row_stride);
  if ((n_tokens + 255) / 256 > 65535)
    return fail(MOC_ERR_ARG, "n_tokens too large for the backward grid: %lld", (long long)n_tokens);
  p = make_problem(cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens, seq_len, dim, k, kernel_size,
                   x_dtype, alpha_dtype, basis_dtype, activation, routing);
  p.dy_stride = dy_row_stride;
  return MOC_OK;
}

// Launches of a checked backward problem on a workspace of backward_bytes(p).
int backward_launch(const moc::Problem& p, const void* x, const void* alpha, const void* basis,
                    const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                    hipStream_t st) {
  if (use_mfma_bwd(p)) {
    moc::mfma::backward(p, x, alpha, basis, dy, dx, dalpha, dbasis, workspace, st);
    return hip_status("moc_backward launch");
  }
  if (use_routesplit(p)) {
    moc::mfma::backward_routesplit(p, x, alpha, basis, dy, dx, dalpha, dbasis, workspace, st);
    return hip_status("moc_backward launch");
  }
  if (use_pad(p, true)) {
    moc::mfma::backward_padded(p, x, alpha, basis, dy, dx, dalpha, dbasis, workspace, st);
    return hip_status("moc_backward launch");
  }
  if (use_chunks(p)) {
    moc::mfma::backward_chunks(p, x, alpha, basis, dy, dx, dalpha, dbasis, workspace, st);
    return hip_status("moc_backward launch");
  }
  Carve cv{static_cast<char*>(workspace), 0};
  float* a_r = cv.take<float>(size_t(p.n_tokens * p.K));
  float* basis_c = cv.take<float>(size_t(p.K * p.S * p.D));
  float* scratch_g = cv.take<float>(moc::generic_bwd_scratch_floats(p));
  moc::launch_prep(p, alpha, basis, a_r, basis_c, st);
  moc::prof_begin(p, st);
  moc::launch_backward_generic(p, x, dy, dx, dalpha, dbasis, a_r, basis_c, scratch_g, st);
  moc::prof_end(p, st);
  return hip_status("moc_backward launch");
}

// Device scratch of moc_backward_noalloc: part of this library's code object,
// so each GPU the library runs on holds one copy from its first use until the
// process ends.  Host code reaches it only through the per-device address that
// hipGetSymbolAddress returns (the name itself is a host-side stand-in).
static __device__ __align__(256) unsigned char scratch[MOC_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch` (looked up once per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MOC_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MOC_ERR_ARG, "device index %d out of range", dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr)
        return fail(MOC_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return MOC_OK;
}

}  // namespace

extern "C" {

int moc_backward(const void* x, const void* alpha, const void* basis, const void* dy,
                 int64_t dy_row_stride, void* dx, void* dalpha, void* dbasis,
                 const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs, int64_t n_tokens,
                 int64_t seq_len, int64_t dim, int64_t k, int64_t kernel_size, int x_dtype,
                 int alpha_dtype, int basis_dtype, int activation, int routing, void* workspace,
                 size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  moc::Problem p;
  int rc = backward_problem(x, alpha, basis, dy, dy_row_stride, dalpha, dbasis, cu_seqlens,
                            cu_seqlens_i64, n_seqs, n_tokens, seq_len, dim, k, kernel_size,
                            x_dtype, alpha_dtype, basis_dtype, activation, routing, p);
  if (rc != MOC_OK) return rc;
  const size_t need = backward_bytes(p);
  if (workspace_bytes < need || !workspace)
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  return backward_launch(p, x, alpha, basis, dy, dx, dalpha, dbasis, workspace,
                         static_cast<hipStream_t>(stream));
}

int moc_backward_noalloc(const void* x, const void* alpha, const void* basis, const void* dy,
                         int64_t dy_row_stride, void* dx, void* dalpha, void* dbasis,
                         const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                         int64_t n_tokens, int64_t seq_len, int64_t dim, int64_t k,
                         int64_t kernel_size, int x_dtype, int alpha_dtype, int basis_dtype,
                         int activation, int routing, void* stream) {
  g_err[0] = '\0';
  moc::Problem p;
  int rc = backward_problem(x, alpha, basis, dy, dy_row_stride, dalpha, dbasis, cu_seqlens,
                            cu_seqlens_i64, n_seqs, n_tokens, seq_len, dim, k, kernel_size,
                            x_dtype, alpha_dtype, basis_dtype, activation, routing, p);
  if (rc != MOC_OK) return rc;
  const size_t need = backward_bytes(p);
  if (need > MOC_NOALLOC_SCRATCH_BYTES)
    return fail(MOC_ERR_WORKSPACE,
                "problem needs %zu bytes of scratch; moc_backward_noalloc holds %zu "
                "(call moc_backward with a workspace instead)",
                need, static_cast<size_t>(MOC_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  if ((rc = scratch_address(&ws)) != MOC_OK) return rc;
  return backward_launch(p, x, alpha, basis, dy, dx, dalpha, dbasis, ws,
                         static_cast<hipStream_t>(stream));
}


// ---------------------------------------------------------------------------
// Prefill from a cache (fixed-length sequences, MFMA kernels).

int moc_matrix_core_supported(int64_t n_tokens, int64_t dim, int64_t k, int64_t kernel_size,
                              int x_dtype, int backward) {
  if (n_tokens <= 0 || dim <= 0 || k <= 0 || kernel_size <= 0) return 0;
  if (x_dtype != MOC_DT_BF16 && x_dtype != MOC_DT_F32) return 0;
  moc::Problem p = make_problem(nullptr, 0, 0, n_tokens, n_tokens, dim, k, kernel_size, x_dtype,
                                MOC_DT_F32, MOC_DT_F32, 0, MOC_ROUTE_ALPHA);
  return (backward ? use_mfma_bwd(p) || use_routesplit(p) || use_chunks(p) || use_pad(p, true)
                   : use_mfma(p) || use_routesplit_fwd(p) || use_pad(p, false))
             ? 1
             : 0;
}

int moc_prefill_supported(int64_t n_seqs, int64_t seq_len, int64_t dim, int64_t k,
                          int64_t kernel_size, int x_dtype, int with_cache) {
  if (n_seqs <= 0 || seq_len <= 0 || dim <= 0 || k <= 0 || kernel_size <= 0) return 0;
  if (n_seqs > kMaxTokens / seq_len) return 0;
  moc::Problem p = make_problem(nullptr, 0, n_seqs, n_seqs * seq_len, seq_len, dim, k,
                                kernel_size, x_dtype, MOC_DT_F32, MOC_DT_F32, 0, MOC_ROUTE_ALPHA);
  return use_mfma_bwd(p) && moc::mfma::prefill_supported(p, with_cache != 0) ? 1 : 0;
}

}  // extern "C"

namespace {

// Checks shared by the prefill entries; fills p (fixed-length, n_seqs x seq_len tokens).
int prefill_problem(int64_t n_seqs, int64_t seq_len, int64_t dim, int64_t k, int64_t kernel_size,
                    int x_dtype, int alpha_dtype, int basis_dtype, int activation, int routing,
                    bool has_cache, moc::Problem& p) {
  int rc;
  if (n_seqs <= 0 || seq_len <= 0)
    return fail(MOC_ERR_ARG, "n_seqs and seq_len must be positive (got %lld, %lld)",
                (long long)n_seqs, (long long)seq_len);
  if (n_seqs > kMaxTokens / seq_len)
    return fail(MOC_ERR_ARG, "n_seqs * seq_len too large: %lld x %lld", (long long)n_seqs,
                (long long)seq_len);
  const int64_t n_tokens = n_seqs * seq_len;
  if ((rc = check_dims(n_tokens, dim, k, kernel_size)) != MOC_OK) return rc;
  if ((rc = check_common(x_dtype, alpha_dtype, basis_dtype, activation, routing)) != MOC_OK) return rc;
  p = make_problem(nullptr, 0, n_seqs, n_tokens, seq_len, dim, k, kernel_size, x_dtype,
                   alpha_dtype, basis_dtype, activation, routing);
  p.pre = true;
  if (!use_mfma_bwd(p) || !moc::mfma::prefill_supported(p, has_cache))
    return fail(MOC_ERR_ARG,
                "prefill not supported for this problem (seq_len %lld, dim %lld, k %lld, "
                "kernel_size %lld%s); see moc_prefill_supported",
                (long long)seq_len, (long long)dim, (long long)k, (long long)kernel_size,
                has_cache && seq_len < kernel_size - 1 ? ", seq_len < kernel_size - 1 with a cache" : "");
  return MOC_OK;
}

}  // namespace

extern "C" {

int moc_forward_prefill(const void* x, const void* alpha, const void* basis, void* y,
                        const void* cache, void* final_state, int64_t n_seqs, int64_t seq_len,
                        int64_t dim, int64_t k, int64_t kernel_size, int x_dtype,
                        int alpha_dtype, int basis_dtype, int activation, int routing,
                        void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  moc::Problem p;
  int rc = prefill_problem(n_seqs, seq_len, dim, k, kernel_size, x_dtype, alpha_dtype, basis_dtype,
                           activation, routing, cache != nullptr, p);
  if (rc != MOC_OK) return rc;
  if (!x || !alpha || !basis || !y) return fail(MOC_ERR_ARG, "null tensor pointer");
  const size_t need = forward_bytes(p);
  if (workspace_bytes < need || (need && !workspace))
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  moc::mfma::forward_prefill(p, x, alpha, basis, y, cache, final_state, workspace,
                             static_cast<hipStream_t>(stream));
  return hip_status("moc_forward_prefill launch");
}

int moc_backward_prefill(const void* x, const void* alpha, const void* basis, const void* dy,
                         int64_t dy_row_stride, const void* cache, void* dx, void* dalpha,
                         void* dbasis, void* dcache, int64_t n_seqs, int64_t seq_len, int64_t dim,
                         int64_t k, int64_t kernel_size, int x_dtype, int alpha_dtype,
                         int basis_dtype, int activation, int routing, void* workspace,
                         size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  moc::Problem p;
  int rc = prefill_problem(n_seqs, seq_len, dim, k, kernel_size, x_dtype, alpha_dtype, basis_dtype,
                           activation, routing, true, p);
  if (rc != MOC_OK) return rc;
  if (!x || !alpha || !basis || !dy || !cache || !dalpha || !dbasis)
    return fail(MOC_ERR_ARG, "null tensor pointer");
  if (dy_row_stride != 0 && dy_row_stride != dim)
    return fail(MOC_ERR_ARG, "dy_row_stride must be dim (%lld) or 0, got %lld", (long long)dim,
                (long long)dy_row_stride);
  if ((p.n_tokens + 255) / 256 > 65535)
    return fail(MOC_ERR_ARG, "n_tokens too large for the backward grid: %lld",
                (long long)p.n_tokens);
  p.dy_stride = dy_row_stride;
  const size_t need = backward_bytes(p);
  if (workspace_bytes < need || !workspace)
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  moc::mfma::backward_prefill(p, x, alpha, basis, dy, cache, dx, dalpha, dbasis, dcache, workspace,
                              static_cast<hipStream_t>(stream));
  return hip_status("moc_backward_prefill launch");
}

}  // extern "C"

namespace {

// Problems of a layer set (checked); n_layers in [1, MOC_MAX_LAYERS].
int layer_problems(const MocLayer* layers, int n_layers, const void* cu, int cu64,
                   int64_t n_seqs, int64_t n_tokens, int64_t seq_len, int64_t ks, int x_dt,
                   bool backward, moc::Problem* ps) {
  if (n_layers < 1 || n_layers > MOC_MAX_LAYERS)
    return fail(MOC_ERR_ARG, "n_layers must be in [1, %d], got %d", MOC_MAX_LAYERS, n_layers);
  if (!layers) return fail(MOC_ERR_ARG, "null layer array");
  int rc;
  if ((rc = check_seq(cu, n_seqs, seq_len)) != MOC_OK) return rc;
  for (int i = 0; i < n_layers; ++i) {
    const MocLayer& l = layers[i];
    if ((rc = check_dims(n_tokens, l.dim, l.k, ks)) != MOC_OK) return rc;
    if ((rc = check_common(x_dt, l.alpha_dtype, l.basis_dtype, l.activation, l.routing)) != MOC_OK)
      return rc;
    ps[i] = make_problem(cu, cu64, n_seqs, n_tokens, seq_len, l.dim, l.k, ks, x_dt, l.alpha_dtype,
                         l.basis_dtype, l.activation, l.routing);
    if (backward) {
      if (l.dy_row_stride != 0 && l.dy_row_stride != l.dim && l.dy_row_stride != -1)
        return fail(MOC_ERR_ARG, "layer %d: dy_row_stride must be dim (%lld), 0 or -1, got %lld",
                    i, (long long)l.dim, (long long)l.dy_row_stride);
      ps[i].dy_stride = l.dy_row_stride;
    }
  }
  if (backward && (n_tokens + 255) / 256 > 65535)
    return fail(MOC_ERR_ARG, "n_tokens too large for the backward grid: %lld", (long long)n_tokens);
  return MOC_OK;
}

bool grouped(const moc::Problem* ps, int n, bool backward) {
  for (int i = 0; i < n; ++i)
    if (!(backward ? use_mfma_bwd(ps[i]) : use_mfma(ps[i]))) return false;
  return moc::mfma::layers_grouped(ps, n, backward);
}

size_t layers_bytes(const moc::Problem* ps, int n, bool backward) {
  if (grouped(ps, n, backward))
    return backward ? moc::mfma::backward_layers_workspace(ps, n)
                    : moc::mfma::forward_layers_workspace(ps, n);
  size_t total = 0;
  for (int i = 0; i < n; ++i) total += align_up(backward ? backward_bytes(ps[i]) : forward_bytes(ps[i]));
  return total;
}

}  // namespace

extern "C" {

size_t moc_forward_layers_workspace_bytes(const MocLayer* layers, int n_layers, int64_t n_tokens,
                                          int64_t kernel_size, int x_dtype) {
  moc::Problem ps[MOC_MAX_LAYERS];
  const char saved = g_err[0];
  if (layer_problems(layers, n_layers, nullptr, 0, 0, n_tokens, n_tokens, kernel_size, x_dtype,
                     false, ps) != MOC_OK) {
    g_err[0] = saved;
    return 0;
  }
  return layers_bytes(ps, n_layers, false);
}

size_t moc_backward_layers_workspace_bytes(const MocLayer* layers, int n_layers, int64_t n_tokens,
                                           int64_t kernel_size, int x_dtype) {
  moc::Problem ps[MOC_MAX_LAYERS];
  const char saved = g_err[0];
  if (layer_problems(layers, n_layers, nullptr, 0, 0, n_tokens, n_tokens, kernel_size, x_dtype,
                     false, ps) != MOC_OK) {
    g_err[0] = saved;
    return 0;
  }
  return layers_bytes(ps, n_layers, true);
}

int moc_forward_layers(const MocLayer* layers, int n_layers, const void* cu_seqlens,
                       int cu_seqlens_i64, int64_t n_seqs, int64_t n_tokens, int64_t seq_len,
                       int64_t kernel_size, int x_dtype, void* workspace, size_t workspace_bytes,
                       void* stream) {
  g_err[0] = '\0';
  moc::Problem ps[MOC_MAX_LAYERS];
  int rc = layer_problems(layers, n_layers, cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens, seq_len,
                          kernel_size, x_dtype, false, ps);
  if (rc != MOC_OK) return rc;
  for (int i = 0; i < n_layers; ++i)
    if (!layers[i].x || !layers[i].alpha || !layers[i].basis || !layers[i].y)
      return fail(MOC_ERR_ARG, "layer %d: null tensor pointer", i);
  const size_t need = layers_bytes(ps, n_layers, false);
  if (workspace_bytes < need || (need && !workspace))
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (grouped(ps, n_layers, false)) {
    moc::mfma::LayerIO io[MOC_MAX_LAYERS] = {};
    for (int i = 0; i < n_layers; ++i)
      io[i] = moc::mfma::LayerIO{layers[i].x, layers[i].alpha, layers[i].basis, layers[i].y,
                                 nullptr, nullptr, nullptr, nullptr};
    moc::mfma::forward_layers(ps, io, n_layers, ws, st);
    return hip_status("moc_forward_layers launch");
  }
  for (int i = 0; i < n_layers; ++i) {
    const MocLayer& l = layers[i];
    const size_t nb = align_up(forward_bytes(ps[i]));
    rc = moc_forward(l.x, l.alpha, l.basis, l.y, cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens,
                     seq_len, l.dim, l.k, kernel_size, x_dtype, l.alpha_dtype, l.basis_dtype,
                     l.activation, l.routing, nb ? ws : nullptr, nb, stream);
    if (rc != MOC_OK) return rc;
    ws += nb;
  }
  return MOC_OK;
}

int moc_backward_layers(const MocLayer* layers, int n_layers, const void* cu_seqlens,
                        int cu_seqlens_i64, int64_t n_seqs, int64_t n_tokens, int64_t seq_len,
                        int64_t kernel_size, int x_dtype, void* workspace, size_t workspace_bytes,
                        void* stream) {
  g_err[0] = '\0';
  moc::Problem ps[MOC_MAX_LAYERS];
  int rc = layer_problems(layers, n_layers, cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens, seq_len,
                          kernel_size, x_dtype, true, ps);
  if (rc != MOC_OK) return rc;
  for (int i = 0; i < n_layers; ++i) {
    const MocLayer& l = layers[i];
    if (!l.x || !l.alpha || !l.basis || !l.dy || !l.dalpha || !l.dbasis)
      return fail(MOC_ERR_ARG, "layer %d: null tensor pointer", i);
  }
  const size_t need = layers_bytes(ps, n_layers, true);
  if (workspace_bytes < need || !workspace)
    return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (grouped(ps, n_layers, true)) {
    moc::mfma::LayerIO io[MOC_MAX_LAYERS] = {};
    for (int i = 0; i < n_layers; ++i)
      io[i] = moc::mfma::LayerIO{layers[i].x, layers[i].alpha, layers[i].basis, nullptr,
                                 layers[i].dy, layers[i].dx, layers[i].dalpha, layers[i].dbasis};
    moc::mfma::backward_layers(ps, io, n_layers, ws, st);
    return hip_status("moc_backward_layers launch");
  }
  for (int i = 0; i < n_layers; ++i) {
    const size_t nb = align_up(backward_bytes(ps[i]));
    rc = backward_launch(ps[i], layers[i].x, layers[i].alpha, layers[i].basis, layers[i].dy,
                         layers[i].dx, layers[i].dalpha, layers[i].dbasis, ws, st);
    if (rc != MOC_OK) return rc;
    ws += nb;
  }
  return MOC_OK;
}

int moc_update(const void* x, const void* alpha, const void* basis, void* cache,
               int64_t cache_stride_b, int64_t cache_stride_d, int64_t cache_stride_s, void* y,
               int64_t batch, int64_t dim, int64_t k, int64_t kernel_size, int x_dtype,
               int alpha_dtype, int basis_dtype, int activation, int routing, void* stream) {
  g_err[0] = '\0';
  int rc;
  if ((rc = check_dims(batch, dim, k, kernel_size)) != MOC_OK) return rc;
  if ((rc = check_common(x_dtype, alpha_dtype, basis_dtype, activation, routing)) != MOC_OK) return rc;
  if (batch > kMaxBatch) return fail(MOC_ERR_ARG, "batch too large: %lld", (long long)batch);
  if (!x || !alpha || !basis || !cache || !y) return fail(MOC_ERR_ARG, "null tensor pointer");
  const bool force_generic = g_path.load(std::memory_order_relaxed) == MOC_PATH_GENERIC;
  if (!force_generic && moc::decode_supported(batch, dim, k, kernel_size, x_dtype, alpha_dtype,
                                              basis_dtype, cache_stride_b, cache_stride_d,
                                              cache_stride_s)) {
    if (!moc::launch_decode(x, alpha, moc::route_form(routing), basis, cache, y, batch, dim, k,
                            kernel_size, activation, static_cast<hipStream_t>(stream)))
      return fail(MOC_ERR_ARG, "decode kernel not built for k %lld, kernel_size %lld", (long long)k,
                  (long long)kernel_size);
    return hip_status("moc_update launch");
  }
  moc::launch_update_generic(x, alpha, basis, cache, cache_stride_b, cache_stride_d,
                             cache_stride_s, y, batch, dim, k, kernel_size, x_dtype, alpha_dtype,
                             basis_dtype, activation, routing, static_cast<hipStream_t>(stream));
  return hip_status("moc_update launch");
}

int moc_decode_step_supported(int64_t batch, int64_t z_dim, int64_t dim, int64_t k,
                              int64_t kernel_size) {
  return moc::decode_step_supported(batch, dim, z_dim, k, kernel_size) ? 1 : 0;
}

int moc_decode_step(const void* z, const void* router, const void* x, const void* basis,
                    void* cache, void* y, int64_t batch, int64_t z_dim, int64_t dim, int64_t k,
                    int64_t kernel_size, int activation, int routing, void* stream) {
  g_err[0] = '\0';
  int rc;
  if ((rc = check_dims(batch, dim, k, kernel_size)) != MOC_OK) return rc;
  if (batch > kMaxBatch) return fail(MOC_ERR_ARG, "batch too large: %lld", (long long)batch);
  if (activation != 0 && activation != 1)
    return fail(MOC_ERR_ARG, "activation must be 0 or 1, got %d", activation);
  if (routing != MOC_ROUTE_SOFTMAX && routing != MOC_ROUTE_EXP)
    return fail(MOC_ERR_ARG, "routing must be softmax (1) or exp (2), got %d", routing);
  if (!moc::decode_step_supported(batch, dim, z_dim, k, kernel_size))
    return fail(MOC_ERR_ARG, "decode step shape not supported (batch %lld, z_dim %lld, dim %lld, "
                             "k %lld, kernel_size %lld)",
                (long long)batch, (long long)z_dim, (long long)dim, (long long)k,
                (long long)kernel_size);
  if (!z || !router || !x || !basis || !cache || !y) return fail(MOC_ERR_ARG, "null tensor pointer");
  if (!moc::launch_decode_step(z, router, x, basis, cache, y, batch, z_dim, dim, k, kernel_size,
                               activation, routing, static_cast<hipStream_t>(stream)))
    return fail(MOC_ERR_ARG, "decode step kernel not built for k %lld, kernel_size %lld",
                (long long)k, (long long)kernel_size);
  return hip_status("moc_decode_step launch");
}

int moc_router_supported(int64_t n_tokens, int64_t z_dim, int64_t k, int dtype) {
  return moc::router_supported(n_tokens, z_dim, k, dtype) ? 1 : 0;
}

int moc_router_forward(const void* z, const void* router, void* logits, int64_t n_tokens,
                       int64_t z_dim, int64_t k, int dtype, void* stream) {
  g_err[0] = '\0';
  if (!moc::router_supported(n_tokens, z_dim, k, dtype))
    return fail(MOC_ERR_ARG, "router shape not supported (n_tokens %lld, z_dim %lld, k %lld, "
                             "dtype %d): bf16, k %% 4 == 0, k <= 96, z_dim %% 64 == 0",
                (long long)n_tokens, (long long)z_dim, (long long)k, dtype);
  if (!z || !router || !logits) return fail(MOC_ERR_ARG, "null tensor pointer");
  if ((n_tokens + 15) / 16 > 0x7fffffff) return fail(MOC_ERR_ARG, "n_tokens too large");
  moc::router_forward(z, router, logits, n_tokens, z_dim, k, moc::ROUTE_ALPHA,
                      static_cast<hipStream_t>(stream));
  return hip_status("moc_router_forward launch");
}

int moc_router_forward_routed(const void* z, const void* router, void* weights, int64_t n_tokens,
                              int64_t z_dim, int64_t k, int dtype, int routing, void* stream) {
  g_err[0] = '\0';
  if (!moc::router_supported(n_tokens, z_dim, k, dtype))
    return fail(MOC_ERR_ARG, "router shape not supported (n_tokens %lld, z_dim %lld, k %lld, "
                             "dtype %d): bf16, k %% 4 == 0, k <= 96, z_dim %% 64 == 0",
                (long long)n_tokens, (long long)z_dim, (long long)k, dtype);
  if (routing != MOC_ROUTE_SOFTMAX && routing != MOC_ROUTE_EXP)
    return fail(MOC_ERR_ARG, "routing must be softmax (1) or exp (2), got %d", routing);
  if (k > moc::kRouterMaxRoutedK)
    return fail(MOC_ERR_ARG, "the fused router activation needs k <= %d, got %lld",
                moc::kRouterMaxRoutedK, (long long)k);
  if (!z || !router || !weights) return fail(MOC_ERR_ARG, "null tensor pointer");
  if ((n_tokens + 15) / 16 > 0x7fffffff) return fail(MOC_ERR_ARG, "n_tokens too large");
  moc::router_forward(z, router, weights, n_tokens, z_dim, k, routing,
                      static_cast<hipStream_t>(stream));
  return hip_status("moc_router_forward_routed launch");
}

int moc_router_forward_grouped(const void* z, const void* router, void* const* weights,
                               const int64_t* k, const int* routing, int n_groups,
                               int64_t n_tokens, int64_t z_dim, int dtype, void* stream) {
  g_err[0] = '\0';
  if (n_groups < 1 || n_groups > moc::kMaxRouteGroups)
    return fail(MOC_ERR_ARG, "n_groups must be in [1, %d], got %d", moc::kMaxRouteGroups, n_groups);
  if (!k || !routing || !weights) return fail(MOC_ERR_ARG, "null group array");
  moc::RouteGroups grp{};
  grp.n = n_groups;
  int64_t total = 0;
  for (int g = 0; g < n_groups; ++g) {
    if (k[g] <= 0 || k[g] > moc::kRouterMaxRoutedK || k[g] % 4 != 0)
      return fail(MOC_ERR_ARG, "group %d: k must be a multiple of 4 in [4, %d], got %lld", g,
                  moc::kRouterMaxRoutedK, (long long)k[g]);
    if (routing[g] < MOC_ROUTE_ALPHA || routing[g] > MOC_ROUTE_EXP)
      return fail(MOC_ERR_ARG, "group %d: routing must be 0, 1 or 2, got %d", g, routing[g]);
    if (!weights[g] || (reinterpret_cast<uintptr_t>(weights[g]) & 7) != 0)
      return fail(MOC_ERR_ARG, "group %d: output pointer null or not 8-byte aligned", g);
    grp.k0[g] = static_cast<int>(total);
    grp.kn[g] = static_cast<int>(k[g]);
    grp.routing[g] = routing[g];
    grp.out[g] = static_cast<uint16_t*>(weights[g]);
    total += k[g];
  }
  if (!moc::router_supported(n_tokens, z_dim, total, dtype))
    return fail(MOC_ERR_ARG, "router shape not supported (n_tokens %lld, z_dim %lld, total k %lld, "
                             "dtype %d): bf16, total k <= %d, z_dim %% 64 == 0",
                (long long)n_tokens, (long long)z_dim, (long long)total, dtype, moc::kRouterMaxK);
  if (!z || !router) return fail(MOC_ERR_ARG, "null tensor pointer");
  if ((n_tokens + 15) / 16 > 0x7fffffff) return fail(MOC_ERR_ARG, "n_tokens too large");
  moc::router_forward_grouped(z, router, grp, n_tokens, z_dim, static_cast<hipStream_t>(stream));
  return hip_status("moc_router_forward_grouped launch");
}

size_t moc_router_backward_workspace_bytes(int64_t n_tokens, int64_t z_dim, int64_t k,
                                           int dtype) {
  if (!moc::router_supported(n_tokens, z_dim, k, dtype)) return 0;
  return moc::router_backward_workspace(n_tokens, z_dim, k);
}

int moc_router_backward(const void* z, const void* router, const void* dlogits, void* dz,
                        void* drouter, int64_t n_tokens, int64_t z_dim, int64_t k, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = '\0';
  if (!moc::router_supported(n_tokens, z_dim, k, dtype))
    return fail(MOC_ERR_ARG, "router shape not supported (n_tokens %lld, z_dim %lld, k %lld, "
                             "dtype %d): bf16, k %% 4 == 0, k <= 96, z_dim %% 64 == 0",
                (long long)n_tokens, (long long)z_dim, (long long)k, dtype);
  if (!router || !dlogits || (drouter && !z)) return fail(MOC_ERR_ARG, "null tensor pointer");
  if (drouter) {
    const size_t need = moc::router_backward_workspace(n_tokens, z_dim, k);
    if (workspace_bytes < need || !workspace)
      return fail(MOC_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need,
                  workspace_bytes);
  }
  moc::router_backward(z, router, dlogits, dz, drouter, n_tokens, z_dim, k, workspace,
                       static_cast<hipStream_t>(stream));
  return hip_status("moc_router_backward launch");
}

}  // extern "C"
