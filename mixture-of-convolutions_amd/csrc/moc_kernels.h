// Internal host-side interface between the C ABI (moc_capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "moc_common.h"

namespace moc {

// Kernel family a call runs on (moc_set_kernel_path).
enum KernelPath : int { PATH_AUTO = 0, PATH_GENERIC = 1, PATH_MFMA_PREP = 2 };

struct Problem {
  SeqLayout seq;     // token axis layout (n_tokens lives here)
  int64_t n_tokens;
  int64_t D, K, S;
  int x_dt, a_dt, b_dt;
  int activation;    // 0 = none, 1 = SiLU
  int routing;       // Route
  int64_t dy_stride = 0;  // backward: elements between token rows of dy (D; 0: one row for all
                          // tokens; -1: one element for every token and channel)
  int path = PATH_AUTO;   // PATH_MFMA_PREP: MFMA kernels, operands always through prep
  bool pre = false;       // prefill from a cache: with the activation, the two passes only at
                          // 32 routes and 6-8 taps (pre_two_pass_g)
  bool grouped = false;   // a layer of a grouped launch: with the activation, the fused pass
  hipEvent_t prof_start = nullptr;  // recorded around the main kernel when set
  hipEvent_t prof_stop = nullptr;
};

// Record p.prof_start / p.prof_stop around the main kernel of a call.
inline void prof_begin(const Problem& p, hipStream_t st) {
  if (p.prof_start) (void)hipEventRecord(p.prof_start, st);
}
inline void prof_end(const Problem& p, hipStream_t st) {
  if (p.prof_stop) (void)hipEventRecord(p.prof_stop, st);
}

// generic path (moc_generic.hip)
void launch_prep(const Problem& p, const void* alpha, const void* basis, float* a_r,
                 float* basis_c, hipStream_t st);
// a_r alone (the routing weights as the router activation forms them, fp32)
void launch_prep_alpha(const Problem& p, const void* alpha, float* a_r, hipStream_t st);
void launch_forward_generic(const Problem& p, const void* x, const float* a_r,
                            const float* basis_c, void* y, hipStream_t st);
size_t generic_bwd_scratch_floats(const Problem& p);
// dy rows are p.dy_stride elements apart
void launch_backward_generic(const Problem& p, const void* x, const void* dy, void* dx,
                             void* dalpha, void* dbasis, const float* a_r,
                             const float* basis_c, float* scratch, hipStream_t st);
void launch_update_generic(const void* x, const void* alpha, const void* basis, void* cache,
                           int64_t cs_b, int64_t cs_d, int64_t cs_s, void* y, int64_t B,
                           int64_t D, int64_t K, int64_t S, int x_dt, int a_dt, int b_dt,
                           int activation, int routing, hipStream_t st);

// MFMA path (moc_mfma_common.hip): supported() for the forward (2 <= S <= 16,
// K <= 32, or <= 64 with bf16 x or S <= 8; D even), bwd_supported() for the
// backward in one pass family (the same with S <= 8 and K <= 32 for fp32 x, or
// bf16 and fp32 with K <= 16 up to S = 16), routesplit_supported() for the
// fp32 backward in route parts (33-64 routes up to S = 8, 17-64 routes at S 9
// to 16), routesplit_fwd_supported() for the fp32 forward in route halves (33-64
// routes at S 9 to 16)
namespace mfma {
bool supported(const Problem& p);
bool bwd_supported(const Problem& p);
// fp32 layers in route parts (moc_routesplit.hip): the backward with 33-64
// routes up to 8 taps (parts of 32) and 17-64 routes at 9-16 taps (parts of
// 16); the forward with 33-64 routes at 9-16 taps (halves of 32)
bool routesplit_supported(const Problem& p);
size_t routesplit_workspace(const Problem& p);
bool routesplit_fwd_supported(const Problem& p);
size_t routesplit_fwd_workspace(const Problem& p);
void forward_routesplit(const Problem& p, const void* x, const void* alpha, const void* basis,
                        void* y, void* workspace, hipStream_t st);
// the backward of bf16 layers with 9-16 taps and 17-64 routes: the dx pass over
// every route, then the taps pass per 16-route chunk (moc_mfma_common.hip)
bool chunks_supported(const Problem& p);
size_t chunks_workspace(const Problem& p);
void backward_chunks(const Problem& p, const void* x, const void* alpha, const void* basis,
                     const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                     hipStream_t st);
void backward_routesplit(const Problem& p, const void* x, const void* alpha, const void* basis,
                         const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                         hipStream_t st);
// odd channel counts through a zero-padded copy at D + 1 channels (moc_pad.hip)
bool pad_supported(const Problem& p, bool backward);
size_t pad_workspace(const Problem& p, bool backward);
void forward_padded(const Problem& p, const void* x, const void* alpha, const void* basis, void* y,
                    void* workspace, hipStream_t st);
void backward_padded(const Problem& p, const void* x, const void* alpha, const void* basis,
                     const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                     hipStream_t st);
size_t forward_workspace(const Problem& p);
size_t backward_workspace(const Problem& p);
void forward(const Problem& p, const void* x, const void* alpha, const void* basis, void* y,
             void* workspace, hipStream_t st);
void backward(const Problem& p, const void* x, const void* alpha, const void* basis,
              const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
              hipStream_t st);

// Prefill from a cache (moc/api.py:299-309): fixed-length sequences
// (p.seq.seq_len tokens each; at least S-1 with a cache).  cache [n_seqs, D, S]
// in the x dtype (or null: zero history); fin (or null) receives the final
// state [n_seqs, D, S]; dcache (or null) the cache gradient.  The workspaces
// are those of forward / backward.
bool prefill_supported(const Problem& p, bool has_cache);
void forward_prefill(const Problem& p, const void* x, const void* alpha, const void* basis,
                     void* y, const void* cache, void* fin, void* workspace, hipStream_t st);
void backward_prefill(const Problem& p, const void* x, const void* alpha, const void* basis,
                      const void* dy, const void* cache, void* dx, void* dalpha, void* dbasis,
                      void* dcache, void* workspace, hipStream_t st);

// Grouped layers: layer i is problem ps[i] (one token axis; K, S, activation
// shared) on tensors io[i]; layers_grouped tells whether they can run as one
// launch per pass (bf16, at most 4 layers; for the backward, not the shapes
// whose single launch runs a form the grouped launch lacks).
struct LayerIO {
  const void* x;
  const void* alpha;
  const void* basis;
  void* y;        // forward
  const void* dy; // backward (rows ps[i].dy_stride apart)
  void* dx;
  void* dalpha;
  void* dbasis;
};
bool layers_grouped(const Problem* ps, int n, bool backward);
size_t forward_layers_workspace(const Problem* ps, int n);
size_t backward_layers_workspace(const Problem* ps, int n);
void forward_layers(const Problem* ps, const LayerIO* io, int n, void* workspace, hipStream_t st);
void backward_layers(const Problem* ps, const LayerIO* io, int n, void* workspace,
                     hipStream_t st);
}  // namespace mfma

// decode step on the matrix cores (moc_decode.hip): bf16 x, logits / weights
// and basis, contiguous [B, D, S] cache, 2 <= S <= 8, K % 4 == 0, K <= 64,
// D % 4 == 0
bool decode_supported(int64_t B, int64_t D, int64_t K, int64_t S, int x_dt, int a_dt, int b_dt,
                      int64_t cs_b, int64_t cs_d, int64_t cs_s);
// (false: nothing launched, a shape decode_supported does not admit)
bool launch_decode(const void* x, const void* alpha, int routing, const void* basis, void* cache,
                   void* y, int64_t B, int64_t D, int64_t K, int64_t S, int activation,
                   hipStream_t st);

// decode step with the router GEMM in the same kernel (moc_decode.hip)
bool decode_step_supported(int64_t B, int64_t D, int64_t Z, int64_t K, int64_t S);
// (false: nothing launched, a shape decode_step_supported does not admit)
bool launch_decode_step(const void* z, const void* router, const void* x, const void* basis,
                        void* cache, void* y, int64_t B, int64_t Z, int64_t D, int64_t K,
                        int64_t S, int activation, int routing, hipStream_t st);

// router GEMMs (moc_router.hip): bf16, K % 4 == 0, K <= 96, Z % 64 == 0; the
// fused router activation needs K <= 32
constexpr int kRouterMaxK = 96;
constexpr int kRouterMaxRoutedK = 32;
bool router_supported(int64_t N, int64_t Z, int64_t K, int dt);

// Routes [k0, k0 + kn) of a concatenated router form group g: its weights are
// routing[g] (softmax / exp) of those logits, written to out[g] as [N, kn].
constexpr int kMaxRouteGroups = 4;
struct RouteGroups {
  int n;
  int k0[kMaxRouteGroups];
  int kn[kMaxRouteGroups];
  int routing[kMaxRouteGroups];
  uint16_t* out[kMaxRouteGroups];
};
void router_forward_grouped(const void* z, const void* r, const RouteGroups& groups, int64_t N,
                            int64_t Z, hipStream_t st);
size_t router_backward_workspace(int64_t N, int64_t Z, int64_t K);
// routing ROUTE_ALPHA: out = the bf16 logits; ROUTE_SOFTMAX / ROUTE_EXP: out =
// that activation of the bf16 logits, rounded to bf16
void router_forward(const void* z, const void* r, void* out, int64_t N, int64_t Z, int64_t K,
                    int routing, hipStream_t st);
void router_backward(const void* z, const void* r, const void* dl, void* dz, void* dr,
                     int64_t N, int64_t Z, int64_t K, void* workspace, hipStream_t st);

}  // namespace moc
