/*
 * moc_hip.h - C ABI of libmoc_hip.so, the MI355X (gfx950) Mixture-of-Convolutions
 * hot path: fused forward, backward (dx / dalpha / dbasis) and the decode-step
 * cache update, for fixed-length [B,T,D] and packed (cu_seqlens) inputs.
 *
 * Every entry point replaces one launch function of the reference's launch layer
 * (andrewmouldon/mixture-of-convolutions, moc/ops.py); the Python package in this
 * repository binds them with ctypes (moc/_lib.py) the way that layer launched
 * its kernels.  Conventions:
 *   - plain device pointers, element counts and dtype codes; no framework types;
 *   - all tensors contiguous row-major, except the decode cache (strided);
 *   - the caller owns every buffer, including the workspace, whose size comes
 *     from the matching *_workspace_bytes query; the library never allocates;
 *   - all work is enqueued on `stream` (a hipStream_t, NULL = default stream);
 *     no call synchronises the host;
 *   - return 0 on success, a negative MOC_ERR_* code otherwise;
 *     moc_last_error() then returns a message (thread-local).
 *
 * Math (tap s = S-1 multiplies the current token, moc/reference.py:29-32):
 *   alpha[n,k] = alpha_in[n,k]            (MOC_ROUTE_ALPHA, *_WEIGHTS)
 *              = softmax_k(logits[n,:])    (MOC_ROUTE_SOFTMAX)
 *              = exp(logits[n,k])          (MOC_ROUTE_EXP)
 *   P[n,d] = sum_s x[n-(S-1-s), d] * sum_k alpha[n,k] * basis[k,s,d]
 *            (x taken as 0 before the start of n's sequence)
 *   y = silu(P) if activation else P
 */
#ifndef MOC_HIP_H
#define MOC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* storage dtype codes */
#define MOC_DT_F32  0
#define MOC_DT_BF16 1
#define MOC_DT_F16  2

/* what the `alpha` argument holds: routing weights (ALPHA); router logits whose
 * activation (softmax / exp, moc/api.py:383-388) is fused into the kernels
 * (SOFTMAX, EXP); or weights that already are that activation of the logits,
 * e.g. from moc_router_forward_routed (SOFTMAX_WEIGHTS, EXP_WEIGHTS): the
 * forward uses them as given and the backward's dalpha is d/dlogits, the
 * activation gradient formed from the given weights */
#define MOC_ROUTE_ALPHA           0
#define MOC_ROUTE_SOFTMAX         1
#define MOC_ROUTE_EXP             2
#define MOC_ROUTE_SOFTMAX_WEIGHTS 3
#define MOC_ROUTE_EXP_WEIGHTS     4

/* status codes */
#define MOC_OK             0
#define MOC_ERR_ARG       -1
#define MOC_ERR_DTYPE     -2
#define MOC_ERR_WORKSPACE -3
#define MOC_ERR_HIP       -4

/* ABI version of this header (5: MocLayer carries each layer's k and activation). */
int moc_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* moc_last_error(void);

/*
 * Kernel family override; it has no counterpart in the reference (whose Triton
 * autotuner picks configurations itself).  AUTO runs the matrix-core kernels
 * wherever they are built for the shape and the generic kernels elsewhere;
 * GENERIC runs the generic kernels for every shape (to cross-check the two);
 * MFMA_PREP runs the matrix-core kernels with their operands always converted
 * by the prep launch (an A/B switch).  Process-wide; workspace sizes follow the
 * family, so do not change it between a *_workspace_bytes query and the launch
 * it sizes.  Returns the previous value, or MOC_ERR_ARG.
 */
#define MOC_PATH_AUTO      0
#define MOC_PATH_GENERIC   1
#define MOC_PATH_MFMA_PREP 2
int moc_set_kernel_path(int path);

/*
 * 1 when moc_forward (backward = 0) or moc_backward (backward = 1) runs the
 * matrix-core kernels for a problem of this shape and x dtype (under the
 * current moc_set_kernel_path), 0 when it runs the generic kernels.  No
 * counterpart in the reference, whose Triton kernels take every shape; it lets
 * a caller or a test see which family serves a shape.  Matrix-core forward
 * and backward: 2 <= kernel_size <= 16, k <= 64, x bf16 or f32 (some shapes
 * in route parts: the f32 forward past 32 routes beyond kernel_size 8, the
 * backward past 16 routes beyond kernel_size 8 and the f32 backward past 32
 * routes); an odd dim through a copy padded with a zero channel.
 */
int moc_matrix_core_supported(int64_t n_tokens, int64_t dim, int64_t k, int64_t kernel_size,
                              int x_dtype, int backward);

/*
 * Sequence description shared by forward / backward:
 *   cu_seqlens == NULL: fixed length, n_tokens = B*T tokens, sequences of
 *                       seq_len = T tokens each ([B,T,D] viewed as [B*T,D]);
 *   cu_seqlens != NULL: packed, n_seqs sequences, token n of sequence j lies in
 *                       [cu_seqlens[j], cu_seqlens[j+1]); int32 entries, or
 *                       int64 when cu_seqlens_i64 != 0; seq_len is ignored.
 * Tokens outside every [cu_seqlens[j], cu_seqlens[j+1]) start their own history.
 */

/* Workspace bytes moc_forward needs for this problem (0 is valid). */
size_t moc_forward_workspace_bytes(int64_t n_tokens, int64_t dim, int64_t k,
                                   int64_t kernel_size, int x_dtype, int routing);

/*
 * y[n,d] for all tokens.  Replaces launch_forward (moc/ops.py:129-194), which
 * launched _moc_fwd_kernel (moc/kernels.py:36-153), and launch_preact
 * (moc/ops.py:197-213) when called with activation = 0.
 *   x, y  : [n_tokens, dim], x_dtype (bf16 or f32); y has x's dtype
 *   alpha : [n_tokens, k], alpha_dtype (weights or logits, see routing)
 *   basis : [k, kernel_size, dim], basis_dtype
 * With a bf16 x, alpha and basis are rounded to bf16 before the mixture, as the
 * reference kernels do (moc/kernels.py:92-95, 125-128); accumulation is fp32.
 */
int moc_forward(const void* x, const void* alpha, const void* basis, void* y,
                const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                int64_t n_tokens, int64_t seq_len,
                int64_t dim, int64_t k, int64_t kernel_size,
                int x_dtype, int alpha_dtype, int basis_dtype,
                int activation, int routing,
                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes moc_backward needs for this problem, with or without the
 * activation (it is not an argument here). */
size_t moc_backward_workspace_bytes(int64_t n_tokens, int64_t dim, int64_t k,
                                    int64_t kernel_size, int x_dtype, int routing);

/*
 * Gradients for upstream gradient dy (x_dtype, [n_tokens, dim]).  Replaces
 * launch_backward (moc/ops.py:216-338) and the preact recompute it needed
 * (moc/ops.py:197-213), i.e. _moc_bwd_dx_kernel (moc/kernels.py:156-279) and
 * _moc_bwd_dalpha_dbasis_dot_kernel (moc/kernels.py:282-439).
 *   dy     : token rows dy_row_stride elements apart: dim (contiguous); 0
 *            when one row of dim elements is the gradient of every token; -1
 *            when one element is the gradient of every token and channel (the
 *            broadcast gradient of y.sum(), which the reference copied into a
 *            contiguous tensor with dy.contiguous(), moc/api.py:171)
 *   dx     : [n_tokens, dim] in x_dtype, or NULL to skip it (need_x = False)
 *   dalpha : [n_tokens, k] in alpha_dtype; d/dalpha for MOC_ROUTE_ALPHA, or
 *            d/dlogits with the softmax / exp gradient fused in (routing 1-4;
 *            with *_WEIGHTS: softmax a (g - <a, g>), exp a g, a = alpha)
 *   dbasis : [k, kernel_size, dim] in basis_dtype
 * dbasis and dalpha are reduced in a fixed order: results are bitwise
 * reproducible run to run (the reference used relaxed fp32 atomics).
 */
int moc_backward(const void* x, const void* alpha, const void* basis, const void* dy,
                 int64_t dy_row_stride, void* dx, void* dalpha, void* dbasis,
                 const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                 int64_t n_tokens, int64_t seq_len,
                 int64_t dim, int64_t k, int64_t kernel_size,
                 int x_dtype, int alpha_dtype, int basis_dtype,
                 int activation, int routing,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * moc_backward without a workspace argument; it has no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops and harnesses that forbid hipMalloc): the
 * scratch (dalpha / dbasis partial sums, prepared operands) is a device array
 * of MOC_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held from the
 * first call on that GPU until the process ends.  Same arguments, results and
 * kernels as moc_backward.  A problem whose moc_backward_workspace_bytes exceed
 * MOC_NOALLOC_SCRATCH_BYTES is rejected with MOC_ERR_WORKSPACE.  Every call on
 * a GPU shares that GPU's scratch: calls that overlap on one GPU (different
 * streams, or host threads without ordering) race and must not be made.
 * The call itself performs no allocation.
 */
#define MOC_NOALLOC_SCRATCH_BYTES (64u << 20)
int moc_backward_noalloc(const void* x, const void* alpha, const void* basis, const void* dy,
                         int64_t dy_row_stride, void* dx, void* dalpha, void* dbasis,
                         const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                         int64_t n_tokens, int64_t seq_len,
                         int64_t dim, int64_t k, int64_t kernel_size,
                         int x_dtype, int alpha_dtype, int basis_dtype,
                         int activation, int routing, void* stream);

/*
 * Prefill from a cache: n_seqs fixed-length sequences of seq_len tokens that
 * continue the inputs a cache holds.  Replaces the reference's cache path of
 * moc_triton (moc/api.py:299-309: cat the cache before x with zero routing,
 * run the op, drop the first kernel_size outputs) and its final state
 * (moc/api.py:218-227, _final_state) with one launch per pass:
 *   cache       : [n_seqs, dim, kernel_size] in x_dtype, contiguous, slot
 *                 kernel_size-1 the newest input; NULL for a zero history
 *                 (the plain op); read by the taps that reach before a
 *                 sequence's first token
 *   final_state : [n_seqs, dim, kernel_size] in x_dtype, or NULL: each
 *                 sequence's last kernel_size inputs (with seq_len <
 *                 kernel_size, the cache's newest slots first, or zeros)
 * y equals the reference's prefill output; the other arguments are those of
 * moc_forward with n_tokens = n_seqs * seq_len.  With a cache, seq_len must be
 * at least kernel_size - 1.  Runs on the matrix-core kernels only:
 * moc_prefill_supported tells whether a problem does (with_cache: a cache is
 * given), otherwise the calls fail with MOC_ERR_ARG.  Workspaces are those of
 * moc_forward_workspace_bytes / moc_backward_workspace_bytes for n_tokens.
 */
int moc_prefill_supported(int64_t n_seqs, int64_t seq_len, int64_t dim, int64_t k,
                          int64_t kernel_size, int x_dtype, int with_cache);

int moc_forward_prefill(const void* x, const void* alpha, const void* basis, void* y,
                        const void* cache, void* final_state,
                        int64_t n_seqs, int64_t seq_len,
                        int64_t dim, int64_t k, int64_t kernel_size,
                        int x_dtype, int alpha_dtype, int basis_dtype,
                        int activation, int routing,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gradients of moc_forward_prefill (cache required): moc_backward's dx,
 * dalpha and dbasis (arguments as there; dy_row_stride dim or 0), plus
 *   dcache : [n_seqs, dim, kernel_size] in x_dtype, or NULL to skip it: the
 *            gradient of the cache (slot 0 is read by no output and gets 0).
 * A gradient of the final state is not an input: its dx / dcache part is a
 * copy the caller adds (the state is a slice of x and the cache).
 */
int moc_backward_prefill(const void* x, const void* alpha, const void* basis, const void* dy,
                         int64_t dy_row_stride, const void* cache,
                         void* dx, void* dalpha, void* dbasis, void* dcache,
                         int64_t n_seqs, int64_t seq_len,
                         int64_t dim, int64_t k, int64_t kernel_size,
                         int x_dtype, int alpha_dtype, int basis_dtype,
                         int activation, int routing,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Several MoC layers on one token axis in one launch per pass: the q / k / v
 * pattern of the reference README (README.md:80-129), three MoC.forward calls
 * (moc/api.py:372-400) whose forward / backward launches each cover one layer.
 * A MocLayer names one layer's tensors and shape; the layers share cu_seqlens /
 * n_tokens / seq_len, kernel_size and x_dtype, and each has its own dim, k,
 * activation, routing and alpha / basis dtypes.  Fields are those of
 * moc_forward (x, alpha, basis, y, k, activation) and moc_backward (dy,
 * dy_row_stride, dx or NULL, dalpha, dbasis); each entry uses its own.  When
 * every layer is bf16 and on the matrix-core kernels, the forward is one launch
 * over all layers' channels, and the backward one stage-1 launch per route
 * count present (per route count and activation where the single launches
 * run a two-pass form) plus one stage-2 launch; otherwise the layers run one
 * by one.  Results equal moc_forward / moc_backward per
 * layer bit for bit.  1 <= n_layers <= 4.
 */
typedef struct MocLayer {
  const void* x;
  const void* alpha;
  const void* basis;
  void* y;
  const void* dy;
  int64_t dy_row_stride;
  void* dx;
  void* dalpha;
  void* dbasis;
  int64_t dim;
  int routing;
  int alpha_dtype;
  int basis_dtype;
  int activation;
  int64_t k;
} MocLayer;

#define MOC_MAX_LAYERS 4

size_t moc_forward_layers_workspace_bytes(const MocLayer* layers, int n_layers, int64_t n_tokens,
                                          int64_t kernel_size, int x_dtype);
int moc_forward_layers(const MocLayer* layers, int n_layers,
                       const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                       int64_t n_tokens, int64_t seq_len, int64_t kernel_size, int x_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);
size_t moc_backward_layers_workspace_bytes(const MocLayer* layers, int n_layers, int64_t n_tokens,
                                           int64_t kernel_size, int x_dtype);
int moc_backward_layers(const MocLayer* layers, int n_layers,
                        const void* cu_seqlens, int cu_seqlens_i64, int64_t n_seqs,
                        int64_t n_tokens, int64_t seq_len, int64_t kernel_size, int x_dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step, in place.  Replaces launch_update (moc/ops.py:341-362) and
 * _moc_update_kernel (moc/kernels.py:442-550).
 *   x     : [batch, dim] contiguous, x_dtype
 *   alpha : [batch, k] contiguous (weights or logits, see routing)
 *   cache : [batch, dim, kernel_size] in x_dtype with element strides
 *           (cache_stride_b, cache_stride_d, cache_stride_s); slot S-1 newest
 *   y     : [batch, dim] contiguous, x_dtype
 * y = act(sum_{s<S-1} cache[:,:,s+1] * W_s + x * W_{S-1}); afterwards the cache
 * holds its old slots 1..S-1 in slots 0..S-2 and x in slot S-1.
 */
int moc_update(const void* x, const void* alpha, const void* basis, void* cache,
               int64_t cache_stride_b, int64_t cache_stride_d, int64_t cache_stride_s,
               void* y, int64_t batch, int64_t dim, int64_t k, int64_t kernel_size,
               int x_dtype, int alpha_dtype, int basis_dtype,
               int activation, int routing, void* stream);

/*
 * A whole decode step of the MoC layer in one launch: the router GEMM
 * (logits = z . router^T, rounded to bf16), its softmax / exp (routing 1 / 2)
 * and the step of moc_update, i.e. MoC.step (moc/api.py:403-425, which runs
 * F.linear, the router activation and launch_update, moc/ops.py:341-362).
 * All tensors bf16; cache [batch, dim, kernel_size] contiguous, updated in place.
 *   z : [batch, z_dim], router : [k, z_dim], x, y : [batch, dim],
 *   basis : [k, kernel_size, dim]
 * Shapes: 2 <= kernel_size <= 8, k % 4 == 0, k <= 32, dim even,
 * z_dim % 64 == 0 (moc_decode_step_supported returns 1 for such shapes).
 */
int moc_decode_step_supported(int64_t batch, int64_t z_dim, int64_t dim, int64_t k,
                              int64_t kernel_size);
int moc_decode_step(const void* z, const void* router, const void* x, const void* basis,
                    void* cache, void* y, int64_t batch, int64_t z_dim, int64_t dim, int64_t k,
                    int64_t kernel_size, int activation, int routing, void* stream);

/*
 * Router of the MoC layer: logits = z . router^T, the F.linear(z, router) of
 * MoC.forward (moc/api.py:383-388) that the reference runs as a library GEMM,
 * and its backward.  bf16 only; k % 4 == 0, k <= 96, z_dim % 64 == 0,
 * n_tokens * z_dim * 2 < 2^31 and n_tokens <= 65535 * 64 (moc_router_supported
 * returns 1 for such shapes).
 *   z      : [n_tokens, z_dim] contiguous
 *   router : [k, z_dim] contiguous
 *   logits : [n_tokens, k] (output of the forward)
 * Accumulation is fp32; each result is rounded to bf16 once.
 */
int moc_router_supported(int64_t n_tokens, int64_t z_dim, int64_t k, int dtype);
int moc_router_forward(const void* z, const void* router, void* logits, int64_t n_tokens,
                       int64_t z_dim, int64_t k, int dtype, void* stream);

/*
 * The router forward with the router activation of MoC.forward
 * (moc/api.py:383-388: torch.softmax / torch.exp of the logits) fused in:
 * weights = softmax_k(logits) (routing 1) or exp(logits) (routing 2), formed
 * from the bf16 logits and rounded to bf16, as torch forms them.  The weights
 * feed moc_forward / moc_backward with routing MOC_ROUTE_SOFTMAX_WEIGHTS /
 * MOC_ROUTE_EXP_WEIGHTS, whose dalpha is then the logits gradient for
 * moc_router_backward.  k <= 32.
 *   weights : [n_tokens, k] bf16
 */
int moc_router_forward_routed(const void* z, const void* router, void* weights, int64_t n_tokens,
                              int64_t z_dim, int64_t k, int dtype, int routing, void* stream);

/*
 * Several MoC layers that share their routing input z (the QKV pattern of the
 * reference README, README.md:80-129, where three MoC.forward calls each run
 * F.linear(z, router) and their own activation, moc/api.py:383-388): one pass
 * over z against the concatenated routers [sum k, z_dim] (group g owns rows
 * k[0] + .. + k[g-1] onward), and group g's weights, routing[g] (0 logits,
 * 1 softmax, 2 exp) of its bf16 logits rounded to bf16, written to
 * weights[g] ([n_tokens, k[g]] bf16, 8-byte aligned).  Each group's weights
 * equal moc_router_forward_routed's for that group's router bit for bit.
 * 1 <= n_groups <= 4, k[g] % 4 == 0, k[g] <= 32, sum k <= 96.  The backward
 * is moc_router_backward with the concatenated router and the groups' logits
 * gradients side by side ([n_tokens, sum k]): dz is then their sum.
 * weights, k and routing are host arrays of n_groups entries.
 */
int moc_router_forward_grouped(const void* z, const void* router, void* const* weights,
                               const int64_t* k, const int* routing, int n_groups,
                               int64_t n_tokens, int64_t z_dim, int dtype, void* stream);

/* Workspace bytes moc_router_backward needs when drouter is requested. */
size_t moc_router_backward_workspace_bytes(int64_t n_tokens, int64_t z_dim, int64_t k,
                                           int dtype);

/*
 * dz = dlogits . router ([n_tokens, z_dim]) and drouter = dlogits^T . z
 * ([k, z_dim]); either output may be NULL to skip it.  drouter is reduced in a
 * fixed order (bitwise reproducible).
 */
int moc_router_backward(const void* z, const void* router, const void* dlogits, void* dz,
                        void* drouter, int64_t n_tokens, int64_t z_dim, int64_t k, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Profiling aid; it has no counterpart in the reference.  While set (non-NULL
 * hipEvent_t handles), moc_forward / moc_backward record `start_event` right
 * before and `stop_event` right after their main kernel (the fused forward,
 * resp. the fused backward stage 1) on their stream, so a caller can time that
 * kernel alone with hipEventElapsedTime.  NULL, NULL switches it off.
 * Thread-local; returns 0.
 */
int moc_profile_events(void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif

#endif /* MOC_HIP_H */
