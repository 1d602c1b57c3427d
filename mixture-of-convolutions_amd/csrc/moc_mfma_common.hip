// MFMA path: operand preparation, backward stage 2, workspace plans, dispatch.
#include "moc_mfma_launch.h"

namespace moc {
namespace mfma {

// ---------------------------------------------------------------------------
// Operand preparation (one launch):
//   blocks [0, a_blocks): 16 lanes per token, lane i holding k = i + 16 kc;
//     a_c[t, k] = alpha in the compute dtype, K padded to KP with zeros; with
//     routing, alpha = softmax / exp of the logits rounded to the logits' dtype
//     (what torch's router activation returns), and a_r[t, k] keeps that value
//     in fp32 for the backward's activation gradient;
//   other blocks: b_c[k, s, d] = basis in the compute dtype, rows k >= K zero.
template <bool BF, int KC>
__global__ void __launch_bounds__(256)
prep_kernel(const void* __restrict__ alpha, int a_dt, int routing, const void* __restrict__ basis,
            int b_dt, int64_t N, int K, int S, int64_t D, typename CT<BF>::elem* __restrict__ a_c,
            float* __restrict__ a_r, typename CT<BF>::elem* __restrict__ b_c, int64_t a_blocks) {
  // routing is route_form of the caller's code; a_r (if not null) receives the weights
  using C = CT<BF>;
  using E = typename C::elem;
  constexpr int KP = 16 * KC;
  if (static_cast<int64_t>(blockIdx.x) < a_blocks) {
    const int64_t t = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 4;
    const int i = threadIdx.x & 15;
    const bool live = t < N;
    float l[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = i + 16 * kc;
      l[kc] = (live && k < K) ? load_any(alpha, a_dt, t * K + k) : -INFINITY;
    }
    float v[KC];
    if (routing == ROUTE_SOFTMAX) {
      float m = l[0];
#pragma unroll
      for (int kc = 1; kc < KC; ++kc) m = fmaxf(m, l[kc]);
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
      float e[KC], sum = 0.f;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        e[kc] = (i + 16 * kc < K) ? __expf(l[kc] - m) : 0.f;
        sum += e[kc];
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);
      const float inv = 1.0f / sum;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) v[kc] = round_to(e[kc] * inv, a_dt);
    } else if (routing == ROUTE_EXP) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) v[kc] = (i + 16 * kc < K) ? round_to(__expf(l[kc]), a_dt) : 0.f;
    } else {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) v[kc] = (i + 16 * kc < K) ? l[kc] : 0.f;
    }
    if (!live) return;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = i + 16 * kc;
      a_c[t * KP + k] = C::from_f(v[kc]);
      if (a_r != nullptr && k < K) a_r[t * K + k] = v[kc];
    }
  } else {
    const int64_t idx = (static_cast<int64_t>(blockIdx.x) - a_blocks) * 256 + threadIdx.x;
    const int64_t sd = static_cast<int64_t>(S) * D;
    if (idx >= KP * sd) return;
    const int64_t k = idx / sd;
    b_c[idx] = (k < K) ? C::from_f(load_any(basis, b_dt, idx)) : E(0);
  }
}

// dbasis element idx (of K S D) = sum of the n_db token partials in order.
template <int KP>
__device__ __forceinline__ void stage2_db(const float* __restrict__ part_db, int64_t n_db,
                                          void* __restrict__ dbasis, int b_dt, int K, int S,
                                          int64_t D, int64_t idx) {
  const int64_t sd = static_cast<int64_t>(S) * D;
  if (idx >= static_cast<int64_t>(K) * sd) return;
  const int64_t k = idx / sd, rest = idx - k * sd;
  // eight partials' loads in flight at a time; sums in partial order
  float acc = 0.f;
  int64_t p = 0;
  for (; p + 8 <= n_db; p += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part_db[((p + u) * KP + k) * sd + rest];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  for (; p < n_db; ++p) acc += part_db[(p * KP + k) * sd + rest];
  store_any(dbasis, b_dt, idx, acc);
}

// ---------------------------------------------------------------------------
// Backward stage 2 (one launch):
//   blocks [0, da_blocks): 16 lanes per token, lane i holding k = i + 16 kc;
//     dalpha = sum of the n_da channel partials in order, then the router
//     activation gradient (softmax: a (da - <a, da>), exp: a da), stored in the
//     alpha dtype;
//   other blocks: one lane per basis element; dbasis = sum of the n_db token
//     partials in order, stored in the basis dtype.
// stage2_block is block blk of one layer's stage 2.
template <int KC>
__device__ __forceinline__ void
stage2_block(const float* __restrict__ part_da, int64_t n_da, const float* __restrict__ part_db,
             int64_t n_db, const float* __restrict__ a_r, const uint16_t* __restrict__ a_w,
             void* __restrict__ dalpha, int a_dt, int routing, void* __restrict__ dbasis,
             int b_dt, int64_t N, int K, int S, int64_t D, int64_t da_blocks, int64_t blk) {
  // the weights of the activation gradient: a_r (fp32) or, if a_r is null,
  // a_w (the caller's bf16 weights)
  constexpr int KP = 16 * KC;
  if (blk < da_blocks) {
    const int64_t t = (blk * 256 + threadIdx.x) >> 4;
    const int i = threadIdx.x & 15;
    const bool live = t < N;
    float da[KC], a[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      da[kc] = 0.f;
      a[kc] = 0.f;
    }
    if (live) {
      // eight partials' loads in flight at a time; sums in partial order
      int64_t p = 0;
      for (; p + 8 <= n_da; p += 8) {
        float v[8][KC];
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) v[u][kc] = part_da[((p + u) * N + t) * KP + i + 16 * kc];
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) da[kc] += v[u][kc];
      }
      for (; p < n_da; ++p) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) da[kc] += part_da[(p * N + t) * KP + i + 16 * kc];
      }
      if (routing != ROUTE_ALPHA) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          const int64_t at = t * K + i + 16 * kc;
          if (i + 16 * kc < K) a[kc] = (a_r != nullptr) ? a_r[at] : bf16_to_f32(a_w[at]);
        }
      }
    }
    float dot = 0.f;
    if (routing == ROUTE_SOFTMAX) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) dot = fmaf(a[kc], da[kc], dot);
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 16);
    }
    if (!live) return;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = i + 16 * kc;
      if (k < K) {
        float v = da[kc];
        if (routing == ROUTE_SOFTMAX) v = a[kc] * (v - dot);
        else if (routing == ROUTE_EXP) v = a[kc] * v;
        store_any(dalpha, a_dt, t * K + k, v);
      }
    }
  } else {
    stage2_db<KP>(part_db, n_db, dbasis, b_dt, K, S, D, (blk - da_blocks) * 256 + threadIdx.x);
  }
}

template <int KC>
__global__ void __launch_bounds__(256)
stage2_kernel(const float* __restrict__ part_da, int64_t n_da, const float* __restrict__ part_db,
              int64_t n_db, const float* __restrict__ a_r, const uint16_t* __restrict__ a_w,
              void* __restrict__ dalpha, int a_dt, int routing, void* __restrict__ dbasis,
              int b_dt, int64_t N, int K, int S, int64_t D, int64_t da_blocks) {
  stage2_block<KC>(part_da, n_da, part_db, n_db, a_r, a_w, dalpha, a_dt, routing, dbasis, b_dt, N,
                   K, S, D, da_blocks, static_cast<int64_t>(blockIdx.x));
}

// Stage 2 of several layers in one launch: layer i owns blocks [blk0, blk0 +
// da_blocks + its dbasis blocks) of the grid and has its own K (kc route chunks).
struct Stage2Layer {
  const float* part_da;
  int64_t n_da, n_db;
  const float* a_r;
  const uint16_t* a_w;
  void* dalpha;
  int a_dt, routing;
  void* dbasis;
  int b_dt;
  const float* part_db;
  int64_t D, blk0;
  int K, kc;
};
struct Stage2Layers {
  int n;
  Stage2Layer l[kMaxLayers];
};

__global__ void __launch_bounds__(256)
stage2_layers_kernel(Stage2Layers ly, int64_t N, int S, int64_t da_blocks) {
  const int64_t b = static_cast<int64_t>(blockIdx.x);
  Stage2Layer L = ly.l[0];
#pragma unroll
  for (int i = 1; i < kMaxLayers; ++i)
    if (i < ly.n && b >= ly.l[i].blk0) L = ly.l[i];
  auto run = [&](auto kc) {
    stage2_block<decltype(kc)::value>(L.part_da, L.n_da, L.part_db, L.n_db, L.a_r, L.a_w, L.dalpha,
                                      L.a_dt, L.routing, L.dbasis, L.b_dt, N, L.K, S, L.D, da_blocks,
                                      b - L.blk0);
  };
  if (L.kc == 1) run(std::integral_constant<int, 1>{});
  else if (L.kc == 2) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 4>{});
}

// ---------------------------------------------------------------------------
// Cache gradient of a prefill (one thread per channel d of sequence b): the
// outputs of the sequence's first S-1 tokens read the cache (slot s + 1 + pos
// for tap s < S-1-pos of token pos), so
//   dcache[b, d, j] = sum over pos < S-1, s = j - 1 - pos >= 0 of g[t, d] W[t, s, d]
// (t = b T + pos; slot 0 is read by no kept output and gets zero), with W from the
// kernels' operands and, with SiLU, g = dy silu'(P) recomputed in fp32.  The
// route loop is unrolled (KP = 16 KC), so all of a thread's loads are issued
// before the first product; 64-lane workgroups spread the few sequences' work
// over the CUs.
template <int S, int KC, bool BF>
__global__ void __launch_bounds__(64)
hist_grad_kernel(const typename CT<BF>::elem* __restrict__ x,
                 const typename CT<BF>::elem* __restrict__ a_c,
                 const typename CT<BF>::elem* __restrict__ b_c,
                 const typename CT<BF>::elem* __restrict__ dy, int64_t dys,
                 const typename CT<BF>::elem* __restrict__ hist,
                 typename CT<BF>::elem* __restrict__ dcache, int64_t T, int64_t D, int act) {
  using C = CT<BF>;
  constexpr int KP = 16 * KC;
  constexpr int NP = S - 1;  // tokens of a sequence whose taps reach the cache (T >= S-1)
  const int64_t b = blockIdx.y;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  if (d >= D) return;
  const int64_t t0 = b * T;
  float w[NP][S];
#pragma unroll
  for (int pos = 0; pos < NP; ++pos)
#pragma unroll
    for (int s = 0; s < S; ++s) w[pos][s] = 0.f;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    float bs[S];
#pragma unroll
    for (int s = 0; s < S; ++s) bs[s] = C::to_f(b_c[(static_cast<int64_t>(k) * S + s) * D + d]);
#pragma unroll
    for (int pos = 0; pos < NP; ++pos) {
      const float a = C::to_f(a_c[(t0 + pos) * KP + k]);
#pragma unroll
      for (int s = 0; s < S; ++s) w[pos][s] = fmaf(a, bs[s], w[pos][s]);
    }
  }
  float hv[S];
#pragma unroll
  for (int s = 0; s < S; ++s) hv[s] = C::to_f(hist[(b * D + d) * S + s]);
  float dc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) dc[s] = 0.f;
#pragma unroll
  for (int pos = 0; pos < NP; ++pos) {
    const int64_t t = t0 + pos;
    float g = C::to_f(dy[dys < 0 ? 0 : t * dys + d]);
    if (act) {
      float p = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int src = pos - (S - 1 - s);
        const float xv = src >= 0 ? C::to_f(x[(t0 + src) * D + d]) : hv[src >= 0 ? 0 : s + 1 + pos];
        p = fmaf(xv, w[pos][s], p);
      }
      const float sg = sigmoid_f(p);
      g *= sg * (1.f + p * (1.f - sg));
    }
#pragma unroll
    for (int s = 0; s < S - 1 - pos; ++s) dc[s + 1 + pos] = fmaf(g, w[pos][s], dc[s + 1 + pos]);
  }
#pragma unroll
  for (int s = 0; s < S; ++s) dcache[(b * D + d) * S + s] = C::from_f(dc[s]);
}

// ---------------------------------------------------------------------------
// workspace plans

namespace {

constexpr size_t kAlign = 256;
size_t al(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Plan {
  int KP;
  size_t esz;
  size_t off_ac, off_bc, off_ar, off_pda, off_pdb, off_g, total;
  Grid2 bg;
};

// The kernels read the caller's weights and basis in place when both already
// have the operand layout: weights given (no activation to form), bf16
// everywhere, K = 16 (no padded routes) and 16-byte aligned rows; then no prep
// launch runs.  The workspace is sized for the prep path either way, since its
// size is asked for without the pointers.
bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

bool direct(const Problem& p, const void* alpha, const void* basis, const void* dalpha) {
  // K = 16, 32 or 64: the caller's [N, K] weights and [K, S, D] basis are then the
  // kernels' padded operand layouts (KP = K) as they are; PATH_MFMA_PREP forces
  // the prep launch (an A/B switch)
  return p.path != PATH_MFMA_PREP && route_form(p.routing) == ROUTE_ALPHA && p.x_dt == DT_BF16 &&
         p.a_dt == DT_BF16 && p.b_dt == DT_BF16 && (p.K == 16 || p.K == 32 || p.K == 64) &&
         aligned16(alpha) && aligned16(basis) && aligned16(dalpha);
}

Plan plan(const Problem& p, bool backward) {
  Plan pl{};
  pl.KP = 16 * route_chunks(p.K);
  pl.esz = (p.x_dt == DT_BF16) ? 2 : 4;
  size_t off = 0;
  pl.off_ac = off;
  off += al(static_cast<size_t>(p.n_tokens) * pl.KP * pl.esz);
  pl.off_bc = off;
  off += al(static_cast<size_t>(pl.KP) * p.S * p.D * pl.esz);
  pl.off_ar = off;
  if (route_grad(p.routing) != ROUTE_ALPHA) off += al(static_cast<size_t>(p.n_tokens) * p.K * 4);
  if (backward) {
    pl.bg = bwd_partials_grid(p);
    pl.off_pda = off;
    off += al(static_cast<size_t>(pl.bg.gx) * p.n_tokens * pl.KP * 4);
    pl.off_pdb = off;
    off += al(static_cast<size_t>(pl.bg.gy) * pl.KP * p.S * p.D * 4);
    if (bwd_two_pass_g(p)) {  // g = dy silu'(P) from the dx pass to the taps pass
      pl.off_g = off;
      off += al(static_cast<size_t>(p.n_tokens) * p.D * 4);
    }
  }
  pl.total = off;
  return pl;
}

template <bool BF, int KC>
void prep_one(const Problem& p, const Plan& pl, const void* alpha, const void* basis, char* ws,
              bool keep_ar, hipStream_t st) {
  using E = typename CT<BF>::elem;
  const int64_t a_blocks = cdiv(p.n_tokens * 16, 256);
  const int64_t b_blocks = cdiv(static_cast<int64_t>(pl.KP) * p.S * p.D, 256);
  float* a_r = (keep_ar && route_grad(p.routing) != ROUTE_ALPHA)
                  ? reinterpret_cast<float*>(ws + pl.off_ar) : nullptr;
  hipLaunchKernelGGL((prep_kernel<BF, KC>), dim3(static_cast<unsigned>(a_blocks + b_blocks)),
                     dim3(256), 0, st, alpha, p.a_dt, route_form(p.routing), basis, p.b_dt, p.n_tokens,
                     static_cast<int>(p.K), static_cast<int>(p.S), p.D,
                     reinterpret_cast<E*>(ws + pl.off_ac), a_r, reinterpret_cast<E*>(ws + pl.off_bc),
                     a_blocks);
}

// keep_ar: also store the weights in fp32 for stage 2's activation gradient
void launch_prep(const Problem& p, const Plan& pl, const void* alpha, const void* basis, char* ws,
                 bool keep_ar, hipStream_t st) {
  const bool bf = p.x_dt == DT_BF16;
  if (pl.KP == 16) {
    if (bf) prep_one<true, 1>(p, pl, alpha, basis, ws, keep_ar, st);
    else prep_one<false, 1>(p, pl, alpha, basis, ws, keep_ar, st);
  } else if (pl.KP == 32) {
    if (bf) prep_one<true, 2>(p, pl, alpha, basis, ws, keep_ar, st);
    else prep_one<false, 2>(p, pl, alpha, basis, ws, keep_ar, st);
  } else {
    if (bf) prep_one<true, 4>(p, pl, alpha, basis, ws, keep_ar, st);
    else prep_one<false, 4>(p, pl, alpha, basis, ws, keep_ar, st);
  }
}

// Backward stage 2 of one problem on its plan's partials.
void launch_stage2(const Problem& p, const Plan& pl, bool dir, char* ws, const void* alpha,
                   void* dalpha, void* dbasis, hipStream_t st) {
  float* pda = reinterpret_cast<float*>(ws + pl.off_pda);
  float* pdb = reinterpret_cast<float*>(ws + pl.off_pdb);
  const int64_t db_blocks = cdiv(p.K * p.S * p.D, 256);
  const int64_t da_blocks = cdiv(p.n_tokens * 16, 256);
  const int grad = route_grad(p.routing);
  // weights for the activation gradient: prep's fp32 copy, or the caller's
  // bf16 weights read in place
  const float* a_r = (grad != ROUTE_ALPHA && !dir)
                         ? reinterpret_cast<const float*>(ws + pl.off_ar) : nullptr;
  const auto* a_w = static_cast<const uint16_t*>(alpha);
  const dim3 grid(static_cast<unsigned>(da_blocks + db_blocks));
  const int64_t n_da = pl.bg.gx;
  auto kern = pl.KP == 16 ? stage2_kernel<1> : (pl.KP == 32 ? stage2_kernel<2> : stage2_kernel<4>);
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, pda, n_da, pdb, static_cast<int64_t>(pl.bg.gy),
                     a_r, a_w, dalpha, p.a_dt, grad, dbasis, p.b_dt, p.n_tokens,
                     static_cast<int>(p.K), static_cast<int>(p.S), p.D, da_blocks);
}

}  // namespace

bool supported(const Problem& p) {
  const bool s_ok = p.S >= 2 && p.S <= 16;
  // the grids' y dimensions stay within the 65535 launch limit and one
  // super-block's rows within a buffer's 32-bit range; D even: a lane's two
  // channels are both in or both past the channel axis, and its 2-channel
  // accesses stay aligned (rows of D elements start at even elements)
  return s_ok && p.K >= 1 && (p.K <= 32 || (p.K <= 64 && (p.x_dt == DT_BF16 || p.S <= 8))) && p.D % 2 == 0 &&
         p.D <= (int64_t(1) << 20) &&
         (p.x_dt == DT_BF16 || p.x_dt == DT_F32) &&
         bwd_grid(p.n_tokens, p.D, p.S).gy <= 65535 && fwd_grid(p.n_tokens, p.D, p.S).gy <= 65535;
}

// The backward: fp32 with up to 32 routes (the fused fp32 tile over 64 routes
// crashes LLVM's AGPR-copy rewrite); 9 to 16 taps with up to 16 routes (the
// two-pass form)
bool bwd_supported(const Problem& p) {
  return supported(p) && (p.x_dt == DT_BF16 || p.K <= 32) &&
         (p.S <= 8 || p.K <= 16);
}

size_t forward_workspace(const Problem& p) { return plan(p, false).total; }
size_t backward_workspace(const Problem& p) { return plan(p, true).total; }

void forward(const Problem& p, const void* x, const void* alpha, const void* basis, void* y,
             void* workspace, hipStream_t st) {
  const Plan pl = plan(p, false);
  char* ws = static_cast<char*>(workspace);
  const bool dir = direct(p, alpha, basis, nullptr);
  const void* a_c = alpha;
  const void* b_c = basis;
  if (!dir) {
    launch_prep(p, pl, alpha, basis, ws, false, st);
    a_c = ws + pl.off_ac;
    b_c = ws + pl.off_bc;
  }
  prof_begin(p, st);
  switch (p.S) {
    case 2: launch_fwd<2>(p, x, a_c, b_c, y, st); break;
    case 3: launch_fwd<3>(p, x, a_c, b_c, y, st); break;
    case 4: launch_fwd<4>(p, x, a_c, b_c, y, st); break;
    case 5: launch_fwd<5>(p, x, a_c, b_c, y, st); break;
    case 6: launch_fwd<6>(p, x, a_c, b_c, y, st); break;
    case 7: launch_fwd<7>(p, x, a_c, b_c, y, st); break;
    case 8: launch_fwd<8>(p, x, a_c, b_c, y, st); break;
    case 9: launch_fwd<9>(p, x, a_c, b_c, y, st); break;
    case 10: launch_fwd<10>(p, x, a_c, b_c, y, st); break;
    case 11: launch_fwd<11>(p, x, a_c, b_c, y, st); break;
    case 12: launch_fwd<12>(p, x, a_c, b_c, y, st); break;
    case 13: launch_fwd<13>(p, x, a_c, b_c, y, st); break;
    case 14: launch_fwd<14>(p, x, a_c, b_c, y, st); break;
    case 15: launch_fwd<15>(p, x, a_c, b_c, y, st); break;
    case 16: launch_fwd<16>(p, x, a_c, b_c, y, st); break;
    default: break;
  }
  prof_end(p, st);
}

void backward(const Problem& p, const void* x, const void* alpha, const void* basis,
              const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
              hipStream_t st) {
  const Plan pl = plan(p, true);
  char* ws = static_cast<char*>(workspace);
  const bool dir = direct(p, alpha, basis, dalpha);
  const void* a_c = alpha;
  const void* b_c = basis;
  if (!dir) {
    launch_prep(p, pl, alpha, basis, ws, true, st);
    a_c = ws + pl.off_ac;
    b_c = ws + pl.off_bc;
  }
  float* pda = reinterpret_cast<float*>(ws + pl.off_pda);
  float* pdb = reinterpret_cast<float*>(ws + pl.off_pdb);
  float* gb = bwd_two_pass_g(p) ? reinterpret_cast<float*>(ws + pl.off_g) : nullptr;
  prof_begin(p, st);
  switch (p.S) {
    case 2: launch_bwd<2>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 3: launch_bwd<3>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 4: launch_bwd<4>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 5: launch_bwd<5>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 6: launch_bwd<6>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 7: launch_bwd<7>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 8: launch_bwd<8>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 9: launch_bwd<9>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 10: launch_bwd<10>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 11: launch_bwd<11>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 12: launch_bwd<12>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 13: launch_bwd<13>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 14: launch_bwd<14>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 15: launch_bwd<15>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    case 16: launch_bwd<16>(p, x, dy, a_c, b_c, dx, pda, pdb, gb, st); break;
    default: break;
  }
  prof_end(p, st);
  launch_stage2(p, pl, dir, ws, alpha, dalpha, dbasis, st);
}

// ---------------------------------------------------------------------------
// Backward of bf16 layers with 9 to 16 taps and 17 to 64 routes: the dx pass
// over every route (dx; with the activation also g = dy silu'(P) in fp32),
// then per 16-route chunk the taps pass on that chunk's operands and a stage 2
// with the chunk's weights given (its weight gradient, fp32, and its dbasis
// rows in place), then the router gradient over all routes.  Each part keeps a
// fixed summation order, so results are bitwise reproducible.

namespace {

// columns [c0, c0 + 16) of a [N, KP] (bf16) into a16 [N, 16]
__global__ void cols16_kernel(const uint16_t* __restrict__ a, uint16_t* __restrict__ a16, int64_t N,
                              int KP, int c0) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * 16) return;
  const int64_t t = i >> 4;
  a16[i] = a[t * KP + c0 + (i & 15)];
}

// dalpha [N, K] from the chunks' weight gradients (chunk c: [N, kc] at
// c N 16, kc = min(16, K - 16 c)) and the router gradient over all K routes on
// a_r (nullptr: weights given, no gradient to take); one 64-lane wave per token
__global__ void __launch_bounds__(64)
route_grad_chunks_kernel(const float* __restrict__ da_w, const float* __restrict__ a_r,
                         void* __restrict__ dalpha, int a_dt, int routing, int64_t N, int K) {
  const int64_t t = blockIdx.x;
  const int k = threadIdx.x;
  const bool on = k < K;
  const int c = k >> 4, kc = K - 16 * c < 16 ? K - 16 * c : 16;
  const float v = on ? da_w[static_cast<int64_t>(c) * N * 16 + t * kc + (k & 15)] : 0.f;
  const float a = (on && a_r != nullptr) ? a_r[t * K + k] : 0.f;
  float dot = a * v;
  for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
  float r = v;
  if (routing == ROUTE_SOFTMAX) r = a * (v - dot);
  else if (routing == ROUTE_EXP) r = a * v;
  if (on) store_any(dalpha, a_dt, t * K + k, r);
}

Problem chunk_problem(const Problem& p, int64_t kc) {
  Problem q = p;
  q.K = kc;
  q.routing = ROUTE_ALPHA;  // the chunk's weights are given
  q.a_dt = DT_F32;          // its weight gradient in fp32
  q.prof_start = q.prof_stop = nullptr;
  return q;
}

struct ChunkPlan {
  Plan full;       // prep of the whole problem: a_c, b_c, a_r
  size_t a16, da, wq, total;
  Plan q;          // one chunk's partials and g (offsets from wq)
};

ChunkPlan chunk_plan(const Problem& p) {
  ChunkPlan c{};
  c.full.KP = 16 * route_chunks(p.K);
  c.full.esz = 2;
  size_t off = 0;
  c.full.off_ac = off; off += al(static_cast<size_t>(p.n_tokens) * c.full.KP * 2);
  c.full.off_bc = off; off += al(static_cast<size_t>(c.full.KP) * p.S * p.D * 2);
  c.full.off_ar = off;
  if (route_grad(p.routing) != ROUTE_ALPHA) off += al(static_cast<size_t>(p.n_tokens) * p.K * 4);
  c.a16 = off; off += al(static_cast<size_t>(p.n_tokens) * 16 * 2);
  c.da = off; off += al(static_cast<size_t>(p.n_tokens) * c.full.KP * 4);
  c.wq = off;
  c.q = plan(chunk_problem(p, 16), true);
  off += c.q.total;
  c.total = off;
  return c;
}

}  // namespace

bool chunks_supported(const Problem& p) {
  return p.x_dt == DT_BF16 && p.S > 8 && p.S <= 16 && p.K > 16 && p.K <= 64 && supported(p);
}

size_t chunks_workspace(const Problem& p) { return chunk_plan(p).total; }

void backward_chunks(const Problem& p, const void* x, const void* alpha, const void* basis,
                     const void* dy, void* dx, void* dalpha, void* dbasis, void* workspace,
                     hipStream_t st) {
  const ChunkPlan c = chunk_plan(p);
  char* ws = static_cast<char*>(workspace);
  launch_prep(p, c.full, alpha, basis, ws, true, st);
  const auto* a_c = reinterpret_cast<const uint16_t*>(ws + c.full.off_ac);
  const auto* b_c = reinterpret_cast<const uint16_t*>(ws + c.full.off_bc);
  const float* a_r = route_grad(p.routing) != ROUTE_ALPHA
                         ? reinterpret_cast<const float*>(ws + c.full.off_ar) : nullptr;
  auto* a16 = reinterpret_cast<uint16_t*>(ws + c.a16);
  float* da_w = reinterpret_cast<float*>(ws + c.da);
  char* wq = ws + c.wq;
  float* pda = reinterpret_cast<float*>(wq + c.q.off_pda);
  float* pdb = reinterpret_cast<float*>(wq + c.q.off_pdb);
  float* gb = p.activation != 0 ? reinterpret_cast<float*>(wq + c.q.off_g) : nullptr;
  const int64_t N = p.n_tokens, SD = p.S * p.D;
  const size_t esz_b = p.b_dt == DT_F32 ? 4 : 2;
  prof_begin(p, st);
  switch (p.S) {
#define MOC_CHUNKS_DX(S_) \
    case S_: launch_dx_pass<S_>(p, x, dy, a_c, b_c, dx, gb, st); break;
    MOC_CHUNKS_DX(9) MOC_CHUNKS_DX(10) MOC_CHUNKS_DX(11) MOC_CHUNKS_DX(12)
    MOC_CHUNKS_DX(13) MOC_CHUNKS_DX(14) MOC_CHUNKS_DX(15) MOC_CHUNKS_DX(16)
#undef MOC_CHUNKS_DX
    default: break;
  }
  for (int c0 = 0; c0 < p.K; c0 += 16) {
    const int64_t kc = p.K - c0 < 16 ? p.K - c0 : 16;
    const Problem q = chunk_problem(p, kc);
    hipLaunchKernelGGL(cols16_kernel, dim3(static_cast<unsigned>(cdiv(N * 16, 256))), dim3(256), 0, st,
                       a_c, a16, N, c.full.KP, c0);
    const uint16_t* b16 = b_c + static_cast<int64_t>(c0) * SD;
    switch (p.S) {
#define MOC_CHUNKS_TAPS(S_) \
      case S_: launch_taps_chunk<S_>(q, x, dy, a16, b16, pda, pdb, gb, st); break;
      MOC_CHUNKS_TAPS(9) MOC_CHUNKS_TAPS(10) MOC_CHUNKS_TAPS(11) MOC_CHUNKS_TAPS(12)
      MOC_CHUNKS_TAPS(13) MOC_CHUNKS_TAPS(14) MOC_CHUNKS_TAPS(15) MOC_CHUNKS_TAPS(16)
#undef MOC_CHUNKS_TAPS
      default: break;
    }
    launch_stage2(q, c.q, false, wq, nullptr, da_w + static_cast<int64_t>(c0) * N,
                  static_cast<char*>(dbasis) + static_cast<size_t>(c0 * SD) * esz_b, st);
  }
  prof_end(p, st);
  hipLaunchKernelGGL(route_grad_chunks_kernel, dim3(static_cast<unsigned>(N)), dim3(64), 0, st, da_w,
                     a_r, dalpha, p.a_dt, route_grad(p.routing), N, static_cast<int>(p.K));
}

bool prefill_supported(const Problem& p, bool has_cache) {
  // (prefill kernels are built for 2 to 8 taps)
  if (!bwd_supported(p) || p.S > 8 || p.seq.cu != nullptr || p.seq.seq_len <= 0 ||
      p.n_tokens % p.seq.seq_len != 0)
    return false;
  if (has_cache && p.seq.seq_len < p.S - 1) return false;
  // the cache gradient's grid has one y block per sequence
  if (p.n_tokens / p.seq.seq_len > 65535) return false;
  // the cache / final state are addressed with 32-bit byte offsets
  const int64_t esz = p.x_dt == DT_BF16 ? 2 : 4;
  return p.n_tokens / p.seq.seq_len * p.D * p.S * esz < (int64_t(1) << 31);
}

void forward_prefill(const Problem& p, const void* x, const void* alpha, const void* basis,
                     void* y, const void* cache, void* fin, void* workspace, hipStream_t st) {
  const Plan pl = plan(p, false);
  char* ws = static_cast<char*>(workspace);
  const bool dir = direct(p, alpha, basis, nullptr);
  const void* a_c = alpha;
  const void* b_c = basis;
  if (!dir) {
    launch_prep(p, pl, alpha, basis, ws, false, st);
    a_c = ws + pl.off_ac;
    b_c = ws + pl.off_bc;
  }
  const Pre pre{cache, fin};
  prof_begin(p, st);
  switch (p.S) {
    case 2: launch_fwd_pre<2>(p, x, a_c, b_c, y, pre, st); break;
    case 3: launch_fwd_pre<3>(p, x, a_c, b_c, y, pre, st); break;
    case 4: launch_fwd_pre<4>(p, x, a_c, b_c, y, pre, st); break;
    case 5: launch_fwd_pre<5>(p, x, a_c, b_c, y, pre, st); break;
    case 6: launch_fwd_pre<6>(p, x, a_c, b_c, y, pre, st); break;
    case 7: launch_fwd_pre<7>(p, x, a_c, b_c, y, pre, st); break;
    case 8: launch_fwd_pre<8>(p, x, a_c, b_c, y, pre, st); break;
    default: break;
  }
  prof_end(p, st);
}

template <int S, bool BF>
void hist_grad_one(const Problem& p, const void* x, const void* a_c, const void* b_c,
                   const void* dy, const void* cache, void* dcache, int KP, hipStream_t st) {
  using E = typename CT<BF>::elem;
  const int64_t B = p.n_tokens / p.seq.seq_len;
  auto kern = KP == 16 ? hist_grad_kernel<S, 1, BF>
                       : (KP == 32 ? hist_grad_kernel<S, 2, BF> : hist_grad_kernel<S, 4, BF>);
  hipLaunchKernelGGL(kern,
                     dim3(static_cast<unsigned>(cdiv(p.D, 64)), static_cast<unsigned>(B)),
                     dim3(64), 0, st, static_cast<const E*>(x), static_cast<const E*>(a_c),
                     static_cast<const E*>(b_c), static_cast<const E*>(dy), p.dy_stride,
                     static_cast<const E*>(cache), static_cast<E*>(dcache), p.seq.seq_len, p.D,
                     p.activation);
}

void backward_prefill(const Problem& p, const void* x, const void* alpha, const void* basis,
                      const void* dy, const void* cache, void* dx, void* dalpha, void* dbasis,
                      void* dcache, void* workspace, hipStream_t st) {
  const Plan pl = plan(p, true);
  char* ws = static_cast<char*>(workspace);
  const bool dir = direct(p, alpha, basis, dalpha);
  const void* a_c = alpha;
  const void* b_c = basis;
  if (!dir) {
    launch_prep(p, pl, alpha, basis, ws, true, st);
    a_c = ws + pl.off_ac;
    b_c = ws + pl.off_bc;
  }
  float* pda = reinterpret_cast<float*>(ws + pl.off_pda);
  float* pdb = reinterpret_cast<float*>(ws + pl.off_pdb);
  // g = dy silu'(P) from the dx pass to the taps pass (the two-pass shapes with SiLU)
  float* gb = bwd_two_pass_g(p) ? reinterpret_cast<float*>(ws + pl.off_g) : nullptr;
  const Pre pre{cache, nullptr, gb};
  prof_begin(p, st);
  switch (p.S) {
    case 2: launch_bwd_pre<2>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 3: launch_bwd_pre<3>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 4: launch_bwd_pre<4>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 5: launch_bwd_pre<5>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 6: launch_bwd_pre<6>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 7: launch_bwd_pre<7>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    case 8: launch_bwd_pre<8>(p, x, dy, a_c, b_c, dx, pda, pdb, pre, st); break;
    default: break;
  }
  prof_end(p, st);
  launch_stage2(p, pl, dir, ws, alpha, dalpha, dbasis, st);
  if (dcache != nullptr) {
    const bool bf = p.x_dt == DT_BF16;
#define MOC_HG(S_)                                                              \
  case S_:                                                                      \
    if (bf) hist_grad_one<S_, true>(p, x, a_c, b_c, dy, cache, dcache, pl.KP, st); \
    else hist_grad_one<S_, false>(p, x, a_c, b_c, dy, cache, dcache, pl.KP, st);   \
    break;
    switch (p.S) {
      MOC_HG(2)
      MOC_HG(3)
      MOC_HG(4)
      MOC_HG(5)
      MOC_HG(6)
      MOC_HG(7)
      MOC_HG(8)
      default: break;
    }
#undef MOC_HG
  }
}

// ---------------------------------------------------------------------------
// Grouped layers: bf16 layers on one token axis with the same S, each with its
// own K and activation.  The forward is one launch over all their channel
// groups; the backward one stage-1 launch per class of layers that share the
// route chunks (and, where the single launch's form depends on it, the
// activation), then one stage-2 launch.  Every layer's results are those of its
// single launch, bit for bit.

bool layers_grouped(const Problem* ps, int n, bool backward) {
  if (n < 1 || n > kMaxLayers) return false;
  for (int i = 0; i < n; ++i) {
    const Problem& p = ps[i];
    // (grouped kernels are built for 2 to 8 taps)
    if (!supported(p) || p.x_dt != DT_BF16 || p.S > 8) return false;
    if (p.S != ps[0].S || p.n_tokens != ps[0].n_tokens || p.path != ps[0].path) return false;
  }
  (void)backward;  // every backward form of a single launch has its grouped counterpart
  return true;
}

namespace {
// Stage-1 class of a layer in a grouped backward: its route chunks, and its
// activation where either activation's layers run a two-pass form (the two
// forms, or a two-pass and a fused one, cannot share a launch).
int bwd_class(const Problem& p) {
  const int S = static_cast<int>(p.S), KC = route_chunks(p.K);
  const bool two = bwd_two_pass(S, KC, false, true) || bwd_two_pass_r(S, KC, false, true) ||
                   bwd_two_pass_g(S, KC, true, true);
  const int act = two ? (p.activation != 0 ? 1 : 0) : 2;
  return KC * 4 + act;
}
}  // namespace

size_t forward_layers_workspace(const Problem* ps, int n) {
  size_t total = 0;
  for (int i = 0; i < n; ++i) total += plan(ps[i], false).total;
  return total;
}

// Each layer keeps the partials of its own grid (the grouped backward runs the
// layers' own grids), so the workspace is the layers' workspaces side by side.
size_t backward_layers_workspace(const Problem* ps, int n) {
  size_t total = 0;
  for (int i = 0; i < n; ++i) {
    Problem q = ps[i];
    q.grouped = true;
    total += plan(q, true).total;
  }
  return total;
}

void forward_layers(const Problem* ps, const LayerIO* io, int n, void* workspace,
                    hipStream_t st) {
  LayerOps L[kMaxLayers] = {};
  char* ws = static_cast<char*>(workspace);
  for (int i = 0; i < n; ++i) {
    const Plan pl = plan(ps[i], false);
    L[i].x = io[i].x;
    L[i].a_c = io[i].alpha;
    L[i].b_c = io[i].basis;
    if (!direct(ps[i], io[i].alpha, io[i].basis, nullptr)) {
      launch_prep(ps[i], pl, io[i].alpha, io[i].basis, ws, false, st);
      L[i].a_c = ws + pl.off_ac;
      L[i].b_c = ws + pl.off_bc;
    }
    L[i].y = io[i].y;
    L[i].D = ps[i].D;
    L[i].act = ps[i].activation != 0;
    L[i].kc = route_chunks(ps[i].K);
    ws += pl.total;
  }
  prof_begin(ps[0], st);
  switch (ps[0].S) {
    case 2: launch_fwd_layers<2>(ps[0], L, n, st); break;
    case 3: launch_fwd_layers<3>(ps[0], L, n, st); break;
    case 4: launch_fwd_layers<4>(ps[0], L, n, st); break;
    case 5: launch_fwd_layers<5>(ps[0], L, n, st); break;
    case 6: launch_fwd_layers<6>(ps[0], L, n, st); break;
    case 7: launch_fwd_layers<7>(ps[0], L, n, st); break;
    case 8: launch_fwd_layers<8>(ps[0], L, n, st); break;
    default: break;
  }
  prof_end(ps[0], st);
}

void backward_layers(const Problem* ps, const LayerIO* io, int n, void* workspace,
                     hipStream_t st) {
  LayerOps L[kMaxLayers] = {};
  Stage2Layers s2{};
  s2.n = n;
  char* ws = static_cast<char*>(workspace);
  const int64_t N = ps[0].n_tokens;
  const int64_t da_blocks = cdiv(N * 16, 256);
  int64_t blk = 0;
  for (int i = 0; i < n; ++i) {
    Problem p = ps[i];
    p.grouped = true;
    const Plan pl = plan(p, true);
    const bool dir = direct(p, io[i].alpha, io[i].basis, io[i].dalpha);
    L[i].x = io[i].x;
    L[i].a_c = io[i].alpha;
    L[i].b_c = io[i].basis;
    if (!dir) {
      launch_prep(p, pl, io[i].alpha, io[i].basis, ws, true, st);
      L[i].a_c = ws + pl.off_ac;
      L[i].b_c = ws + pl.off_bc;
    }
    L[i].dy = io[i].dy;
    L[i].dys = p.dy_stride;
    L[i].dx = io[i].dx;
    L[i].part_da = reinterpret_cast<float*>(ws + pl.off_pda);
    L[i].part_db = reinterpret_cast<float*>(ws + pl.off_pdb);
    L[i].D = p.D;
    L[i].act = p.activation != 0;
    L[i].kc = route_chunks(p.K);
    L[i].gbuf = bwd_two_pass_g(p) ? reinterpret_cast<float*>(ws + pl.off_g) : nullptr;
    const int grad = route_grad(p.routing);
    s2.l[i] = Stage2Layer{L[i].part_da,
                          static_cast<int64_t>(pl.bg.gx),
                          static_cast<int64_t>(pl.bg.gy),
                          (grad != ROUTE_ALPHA && !dir) ? reinterpret_cast<const float*>(ws + pl.off_ar)
                                                        : nullptr,
                          static_cast<const uint16_t*>(io[i].alpha),
                          io[i].dalpha,
                          p.a_dt,
                          grad,
                          io[i].dbasis,
                          p.b_dt,
                          L[i].part_db,
                          p.D,
                          blk,
                          static_cast<int>(p.K),
                          L[i].kc};
    blk += da_blocks + cdiv(p.K * p.S * p.D, 256);
    ws += pl.total;
  }
  // stage 1: one launch per class, the classes in the order of their first layer
  prof_begin(ps[0], st);
  bool done[kMaxLayers] = {};
  for (int i = 0; i < n; ++i) {
    if (done[i]) continue;
    LayerOps C[kMaxLayers] = {};
    int nc = 0;
    for (int j = i; j < n; ++j)
      if (!done[j] && bwd_class(ps[j]) == bwd_class(ps[i])) {
        C[nc++] = L[j];
        done[j] = true;
      }
    switch (ps[0].S) {
      case 2: launch_bwd_layers<2>(ps[i], C, nc, st); break;
      case 3: launch_bwd_layers<3>(ps[i], C, nc, st); break;
      case 4: launch_bwd_layers<4>(ps[i], C, nc, st); break;
      case 5: launch_bwd_layers<5>(ps[i], C, nc, st); break;
      case 6: launch_bwd_layers<6>(ps[i], C, nc, st); break;
      case 7: launch_bwd_layers<7>(ps[i], C, nc, st); break;
      case 8: launch_bwd_layers<8>(ps[i], C, nc, st); break;
      default: break;
    }
  }
  prof_end(ps[0], st);
  hipLaunchKernelGGL(stage2_layers_kernel, dim3(static_cast<unsigned>(blk)), dim3(256), 0, st, s2, N,
                     static_cast<int>(ps[0].S), da_blocks);
}

}  // namespace mfma
}  // namespace moc
