// Host-side launch of the MFMA kernels, templated on the kernel size S.  Each
// moc_mfma_s<S>.hip instantiates launch_fwd<S> / launch_bwd<S>; the rest of the
// library sees them through the extern declarations at the bottom.
#pragma once

#include <atomic>

#include "moc_bwd_lean.h"
#include "moc_kernels.h"
#include "moc_mfma.h"

namespace moc {
namespace mfma {

// Tile shapes (see moc_mfma.h): forward NB x NC blocks per wave, 4 waves per
// workgroup; backward NB x NC per wave, kBwdWPG waves per workgroup.
#ifndef MOC_FWD_NC
#define MOC_FWD_NC 2
#endif
// 8 taps with one token block per super-block (11 window rows instead of 15,
// 135 VGPRs, three waves per SIMD) measured slower at configs[4]: 1237 -> 1251 us
#ifndef MOC_FWD_NB8
#define MOC_FWD_NB8 2
#endif
constexpr int kFwdNB = 2, kFwdNC = MOC_FWD_NC;
// token blocks per forward super-block for kernel size S
constexpr int fwd_nb(int S) { return S == 8 ? MOC_FWD_NB8 : kFwdNB; }
#ifndef MOC_BWD_WPG
#define MOC_BWD_WPG 4
#endif
constexpr int kBwdNB = 2, kBwdNC = 2, kBwdWPG = MOC_BWD_WPG;
static_assert(kLeanWPG * kLeanCW == 16 * kBwdNC * MOC_BWD_WPG,
              "the lean backward covers the channel groups of the fused pass's grid");
// the lean fused backward (moc_bwd_lean.h) for the shapes it serves; 0: bwd_tile's
#ifndef MOC_BWD_LEAN
#define MOC_BWD_LEAN 1
#endif
// Resident workgroups the grids are sized for (256 CUs).
#ifndef MOC_FWD_TARGET_WG
#define MOC_FWD_TARGET_WG 2048
#endif
constexpr int64_t kFwdTargetWG = MOC_FWD_TARGET_WG;
#ifndef MOC_BWD_TARGET_WG
#define MOC_BWD_TARGET_WG 512
#endif
constexpr int64_t kBwdTargetWG = MOC_BWD_TARGET_WG;

struct Grid2 {
  unsigned gx, gy;
  int n_sb;        // super-blocks per range (at most)
  int gy1 = 0;      // backward: ranges y < gy1 share the first n_old super-blocks,
  int n_old = 0;    // the others the remaining n_total - n_old; the counts of a
  int n_total = 0;  // tier's ranges differ by at most one
};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Route chunks of 16 the kernels are built for: 1, 2 or 4 (K <= 64; K in
// (32, 64] is padded to 64 routes).  Four chunks in the backward with bf16
// data only: the fp32 fused backward at four chunks crashes LLVM's AGPR-copy
// rewrite, so the fp32 backward with K > 32 runs in route parts
// (moc_routesplit.hip).
inline int route_chunks(int64_t K) { return K <= 16 ? 1 : (K <= 32 ? 2 : 4); }
template <int KC, bool BF>
constexpr bool kcOK = KC <= 2 || BF;
// the forward also takes fp32 with 64 routes up to 8 taps (236-434 VGPRs, no
// spills; past 8 taps it spills)
template <int S, int KC, bool BF>
constexpr bool kcOKFwd = kcOK<KC, BF> || S <= 8;

// Forward: about kFwdTargetWG workgroups, each wave walking at most
// kFwdMaxSb super-blocks; larger problems get more workgroups rather than
// longer ones (measured: D 4096, 32768 tokens, 161 -> 141 us).
constexpr int64_t kFwdMaxSb = 4;

// Channels of one forward / backward workgroup (grid x counts these groups).
constexpr int64_t kFwdCW = 4 * 16 * kFwdNC, kBwdCW = kBwdWPG * 16 * kBwdNC;
// Taps pass of the two-pass backward: kTapsWPG waves per workgroup, half of them
// per tap half, so a workgroup covers kTapsCW channels; kTapsPerCU of its
// workgroups fit a CU's LDS at once.
#ifndef MOC_TAPS_WPG
#define MOC_TAPS_WPG 8
#endif
constexpr int kTapsWPG = MOC_TAPS_WPG;
constexpr int64_t kTapsCW = (kTapsWPG / 2) * 16 * kBwdNC;
constexpr int kTapsPerCU = kTapsWPG >= 8 ? 1 : 2;

// Forward grid over gx channel groups (the sum over the layers of a grouped launch).
inline Grid2 fwd_grid_gx(int64_t N, int64_t gx, int64_t S) {
  const int64_t n_super = cdiv(N, 16 * fwd_nb(static_cast<int>(S)));
  int64_t gy_target = kFwdTargetWG / gx;
  if (gy_target < 1) gy_target = 1;
  int64_t n_sb = cdiv(n_super, gy_target);
  if (n_sb > kFwdMaxSb) n_sb = kFwdMaxSb;
  // grid.y stays within the 65535 launch limit: longer ranges instead
  if (cdiv(n_super, n_sb) > 65535) n_sb = cdiv(n_super, 65535);
  return Grid2{static_cast<unsigned>(gx), static_cast<unsigned>(cdiv(n_super, n_sb)),
               static_cast<int>(n_sb)};
}

inline Grid2 fwd_grid(int64_t N, int64_t D, int64_t S) { return fwd_grid_gx(N, cdiv(D, kFwdCW), S); }

// Backward grid over gx channel groups; D is the widest layer's channel count
// (it bounds the token range of a workgroup's buffers).
// Own rows per super-block: the fused and dx passes recompute the last S-1 rows
// of each super-block in the next one (their dx needs later rows' g); the taps
// pass owns all of them.
inline int64_t bwd_eown(int64_t S, bool taps = false) { return taps ? 16 * kBwdNB : 16 * kBwdNB - (S - 1); }

inline Grid2 bwd_grid_gx(int64_t N, int64_t gx, int64_t D, int64_t S,
                         int64_t target_wg = kBwdTargetWG, bool taps = false) {
  const int64_t eown = bwd_eown(S, taps);
  const int64_t n_super = cdiv(N, eown);
  int64_t gy_target = target_wg / gx;
  if (gy_target < 1) gy_target = 1;
  int64_t n_sb = cdiv(n_super, gy_target);
  // a workgroup's x / dy buffers span its token range: keep them under 2^30
  // bytes (4-byte elements assumed), i.e. more, shorter ranges for long inputs
  const int64_t max_sb = ((int64_t(1) << 30) / (D * 4) - 16 * kBwdNB) / eown;
  if (n_sb > max_sb) n_sb = max_sb > 1 ? max_sb : 1;
  Grid2 g{static_cast<unsigned>(gx), static_cast<unsigned>(cdiv(n_super, n_sb)),
          static_cast<int>(n_sb)};
  g.gy1 = static_cast<int>(g.gy);
  g.n_old = static_cast<int>(n_sb * static_cast<int64_t>(g.gy));
  g.n_total = g.n_old;
  return g;
}

inline Grid2 bwd_grid(int64_t N, int64_t D, int64_t S, int64_t target_wg = kBwdTargetWG) {
  return bwd_grid_gx(N, cdiv(D, kBwdCW), D, S, target_wg);
}

// Number of compute units of the current device (cached per device).
inline int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Backward ranges in two tiers.  A grid of 2 n_cu workgroups with two of them
// resident per CU is dispatched one per CU first: workgroups y < gy1 = n_cu / gx
// are the older of each CU's pair, and the SIMD issues the older wave first
// whenever both are ready.  Measured on the headline shape: the older wave
// takes 3.6 us per super-block, the younger 5.4 us while both run and 3.3 us
// alone, so with equal ranges the younger workgroups run their last quarter
// alone.  The older ranges share kBwdOldShare percent of the super-blocks
// instead, so that both tiers finish at about the same time.  Other grids, or
// a CU count that gx does not divide, keep equal ranges.
#ifndef MOC_BWD_OLD_SHARE
#define MOC_BWD_OLD_SHARE 62
#endif
constexpr int64_t kBwdOldShare = MOC_BWD_OLD_SHARE;

inline Grid2 bwd_grid_tiered(int64_t N, int64_t gx, int64_t D, int64_t S, int n_cu) {
  Grid2 g = bwd_grid_gx(N, gx, D, S);
  if (n_cu <= 0 || n_cu % static_cast<int64_t>(g.gx) != 0) return g;
  const int64_t gy1 = n_cu / static_cast<int64_t>(g.gx);
  const int64_t gy = g.gy;
  if (gy != 2 * gy1) return g;
  const int64_t eown = bwd_eown(S);
  const int64_t n_super = cdiv(N, eown);
  const int64_t max_sb = ((int64_t(1) << 30) / (D * 4) - 16 * kBwdNB) / eown;
  const int64_t n_old = (n_super * kBwdOldShare + 50) / 100;
  const int64_t n1 = cdiv(n_old, gy1), n2 = cdiv(n_super - n_old, gy - gy1);
  if (n1 > max_sb || n2 < 1 || n2 > n1) return g;
  g.n_sb = static_cast<int>(n1);
  g.gy1 = static_cast<int>(gy1);
  g.n_old = static_cast<int>(n_old);
  g.n_total = static_cast<int>(n_super);
  return g;
}

// The backward in two passes (bwd_kernel modes kBwdDx, then kBwdTaps with the
// taps split in halves) where the fused pass does not fit two waves per SIMD
// and no activation needs P: bf16, 32 routes and 4 to 8 taps, 16 routes and 7
// or 8 taps (measured against the fused pass at every kernel size: below those
// the fused pass is faster).
// fp32 (the same two passes on fp32 operands, with and without the activation):
// 16 routes from 5 taps (4 without the activation) to 16, 32 routes from 4 to
// 8 taps.  Past 8 taps the fused fp32 tile does not build (its register file);
// below, measured against the fused pass (B4 T4096 D2048, backward entry, us,
// without / with SiLU): 16 routes, 4 taps 234 / 290 -> 222 / 295, 6 taps
// 323 / 414 -> 275 / 356, 8 taps 463 / 562 -> 354 / 461; 32 routes, 4 taps
// 381 / 464 -> 324 / 415, 6 taps 1177 / 1427 -> 450 / 615, 8 taps
// 1046 / 1425 -> 704 / 986.
constexpr bool f32_two_pass(int S, int KC, bool act) {
  return (KC == 1 && (S >= 5 || (S == 4 && !act))) || (KC == 2 && S >= 4 && S <= 8);
}
constexpr bool bwd_two_pass(int S, int KC, bool act, bool bf) {
  return !act && ((bf && ((KC == 2 && S >= 4) || (KC == 1 && S >= 7))) || (!bf && f32_two_pass(S, KC, act)));
}
// With the activation, the two passes where the fused pass spills or forms the
// same work per route chunk (bf16: 32 routes and 5 to 8 taps, 16 routes and 8,
// 64 routes and 3 to 8; measured against the fused pass at each size): the dx
// pass forms g = dy silu'(P) and leaves it in the workspace (fp32 [N, D]) for the
// taps pass.  Single launches only (the grouped launch keeps the fused pass).
constexpr bool bwd_two_pass_g(int S, int KC, bool act, bool bf) {
  return act && ((bf && ((KC == 2 && S >= 5) || (KC == 1 && S >= 8) || (KC == 4 && S >= 3))) ||
                 (!bf && f32_two_pass(S, KC, act)));
}
// The prefill runs those two passes (the dx pass's P reading the cache) with 32
// routes and 6-8 taps and with 64 routes; elsewhere its fused pass measured
// faster (B4 T4096 D2048 with SiLU: 32 routes, 5 taps 216 against 242 us; 16
// routes, 8 taps 232 against 262; 32 routes, 6 / 7 / 8 taps 365 / 610 / 970 ->
// 257 / 335 / 429).
constexpr bool pre_two_pass_g(int S, int KC) { return (KC == 2 && S >= 6) || KC == 4; }
// (the prefill passes are built for bf16: fp32 prefill keeps the fused pass)
inline bool bwd_two_pass_g(const Problem& p) {
  const int S = static_cast<int>(p.S), KC = route_chunks(p.K);
  return (!p.pre || (pre_two_pass_g(S, KC) && p.x_dt == DT_BF16)) &&
         bwd_two_pass_g(S, KC, p.activation != 0, p.x_dt == DT_BF16);
}
// 64 routes without activation: the two passes, the taps pass split in route
// halves (two workgroups per tile, each forming the tile's m products for two of
// the four route chunks; the fused pass forms them once per chunk).  Every
// kernel size.
constexpr bool bwd_two_pass_r(int S, int KC, bool act, bool bf) { return bf && !act && KC == 4; }
constexpr bool pre_two_pass_r(int S) { return S >= 2; }
inline bool bwd_two_pass(const Problem& p) {
  const int S = static_cast<int>(p.S), KC = route_chunks(p.K);
  const bool act = p.activation != 0, bf = p.x_dt == DT_BF16;
  return (bwd_two_pass(S, KC, act, bf) && (bf || !p.pre)) || bwd_two_pass_g(p) ||
         ((!p.pre || pre_two_pass_r(S)) && bwd_two_pass_r(S, KC, act, bf));
}
// route parts of the taps pass's grid (halves with 64 routes), whose single
// round of workgroups then covers half as many tiles
constexpr int taps_route_parts(int KC) { return KC == 4 ? 2 : 1; }

// The taps pass holds one workgroup per CU (its LDS), so it runs as one round
// of n_cu workgroups, with ranges twice as long as the default grid's.  Two
// rounds measured slower: each round pays a prologue of about 6 us, and the
// second round's workgroups started 15-20 us after the first round's ended.
inline Grid2 bwd_taps_grid(int64_t N, int64_t gx, int64_t D, int64_t S, int n_cu) {
  return bwd_grid_gx(N, gx, D, S, n_cu > 0 ? int64_t(n_cu) * kTapsPerCU : kBwdTargetWG / 2, true);
}

// The grid whose workgroups own the dalpha / dbasis partials (workspace,
// stage 2): the taps pass's for the two-pass form, else the fused pass's.
inline Grid2 bwd_partials_grid(const Problem& p) {
  return bwd_two_pass(p) ? bwd_taps_grid(p.n_tokens, cdiv(p.D, kTapsCW), p.D, p.S,
                                         device_cu_count() / taps_route_parts(route_chunks(p.K)))
                         : bwd_grid_gx(p.n_tokens, cdiv(p.D, kBwdCW), p.D, p.S);
}

// Operands of one layer of a grouped launch (after operand preparation); the
// layers share Problem's token axis, K, S, activation and dtypes.
struct LayerOps {
  const void* x;
  const void* a_c;
  const void* b_c;
  void* y;           // forward output
  const void* dy;    // backward
  int64_t dys;
  void* dx;
  float* part_da;
  float* part_db;
  int64_t D;
  int act;   // the layer's activation (0 / 1)
  int kc;    // the layer's route chunks (1, 2 or 4)
  float* gbuf;  // backward, two passes with the activation: the layer's g buffer
};

template <int S, int KC, bool ACT, bool BF>
void fwd_one(const Problem& p, const void* x, const void* a_c, const void* b_c, void* y,
             hipStream_t st) {
  if constexpr (!kcOKFwd<S, KC, BF>) return;
  else {
  using E = typename CT<BF>::elem;
  const Grid2 g = fwd_grid(p.n_tokens, p.D, S);
  hipLaunchKernelGGL((fwd_kernel<S, KC, fwd_nb(S), kFwdNC, ACT, BF>), dim3(g.gx, g.gy), dim3(256), 0,
                     st, x, static_cast<const E*>(a_c), static_cast<const E*>(b_c), y, p.seq, p.D,
                     g.n_sb);
  }
}

// Fused pass with 32 or 64 routes (bf16): each workgroup accumulates dbasis /
// dalpha for one of the 16-route chunks, as the accumulators and dalpha
// operands of all would not fit in registers beside the W operands.
template <int S, int KC, bool ACT, bool BF>
void bwd_one(const Problem& p, const void* x, const void* dy, const void* a_c, const void* b_c,
             void* dx, float* part_da, float* part_db, float* gbuf, hipStream_t st) {
  if constexpr (!kcOK<KC, BF>) return;
  else {
  using E = typename CT<BF>::elem;
  constexpr bool kSplit = BF && KC >= 2;
  constexpr bool kTwo = bwd_two_pass(S, KC, ACT, BF) || bwd_two_pass_g(S, KC, ACT, BF) ||
                        bwd_two_pass_r(S, KC, ACT, BF);
  // the fused pass at four waves per SIMD (moc_bwd_lean.h) where it is built
  constexpr bool kLean = MOC_BWD_LEAN && !kTwo && bwd_lean(S, KC, BF);
  // tiers for the fused pass at two resident workgroups per CU (not split in route chunks)
  constexpr bool kTiers = !kTwo && !kSplit && kBwdMinWaves<S, KC, kBwdFused, BF> == 2;
  const int64_t gx_all = cdiv(p.D, kBwdCW);
  const Grid2 g = kTiers ? bwd_grid_tiered(p.n_tokens, gx_all, p.D, S, device_cu_count())
                         : bwd_grid(p.n_tokens, p.D, S);
  const auto* a = static_cast<const E*>(a_c);
  const auto* b = static_cast<const E*>(b_c);
  const int gx = static_cast<int>(g.gx), gy = static_cast<int>(g.gy);
  // a grid split in route chunks is 1-D: 8 KC workgroups per 8 tiles (see bwd_block)
  const dim3 halves(static_cast<unsigned>(8 * KC * cdiv(static_cast<int64_t>(gx) * gy, 8)));
  if constexpr (kTwo) {
    // (with the activation the dx pass also forms g for the taps pass, so it
    // runs without dx too)
    if (dx != nullptr || ACT)
      hipLaunchKernelGGL((bwd_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, BF, false, kBwdDx>),
                         dim3(g.gx, g.gy), dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, a, b, dx, part_da,
                         part_db, p.seq, p.D, gx, gy, g.gy1, g.n_old, g.n_total, gbuf);
    // both tap halves in one workgroup of 2 kBwdWPG waves (splitting the route
    // chunks as well forms every m product twice again: measured slower than
    // the register spills it avoids)
    // (one round of workgroups: bwd_taps_grid)
    // (64 routes: route halves on a 1-D grid, the halves of a tile 8 ids apart)
    constexpr int kParts = taps_route_parts(KC);
    const Grid2 gt = bwd_taps_grid(p.n_tokens, cdiv(p.D, kTapsCW), p.D, S, device_cu_count() / kParts);
    const dim3 tgrid = kParts > 1 ? dim3(static_cast<unsigned>(8 * kParts * cdiv(int64_t(gt.gx) * gt.gy, 8)))
                                  : dim3(gt.gx, gt.gy);
    hipLaunchKernelGGL((bwd_kernel<S, KC, kBwdNB, kBwdNC, kTapsWPG, ACT, BF, (kParts > 1), kBwdTaps>),
                       tgrid, dim3(64 * kTapsWPG), 0, st, x, dy, p.dy_stride, a, b, nullptr, part_da,
                       part_db, p.seq, p.D, static_cast<int>(gt.gx), static_cast<int>(gt.gy), gt.gy1,
                       gt.n_old, gt.n_total, gbuf);
  } else if constexpr (kLean) {
    // (the lean pass's workgroup covers the same kBwdCW channels with 8 waves)
    // (one dy element for every token and channel: its own instantiation)
    auto kern = p.dy_stride < 0 ? bwd_lean_kernel<S, ACT, true> : bwd_lean_kernel<S, ACT, false>;
    hipLaunchKernelGGL(kern, dim3(g.gx, g.gy), dim3(64 * kLeanWPG), 0, st, x, dy, p.dy_stride,
                       reinterpret_cast<const uint16_t*>(a), reinterpret_cast<const uint16_t*>(b), dx,
                       part_da, part_db, p.seq, p.D, gy, g.gy1, g.n_old, g.n_total);
  } else {
    hipLaunchKernelGGL((bwd_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, BF, kSplit, kBwdFused>),
                       kSplit ? halves : dim3(g.gx, g.gy), dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, a,
                       b, dx, part_da, part_db, p.seq, p.D, gx, gy, g.gy1, g.n_old, g.n_total);
  }
  }
}

// Grouped launches (bf16): one kernel over the layers' own grids, one after
// another on a 1-D grid (see FwdLayers / BwdLayers).  ACT: 0 / 1 when the layers
// share it, kActRuntime when each reads its own.  The forward takes layers of
// any route counts (KCM: the counts present); the backward the layers of one
// count (one launch per count present).
template <int S, int KCM, int ACT>
void fwd_layers_one(const Problem& p, const LayerOps* L, int n, hipStream_t st) {
  FwdLayers ly{};
  ly.n = n;
  int64_t blk = 0;
  for (int i = 0; i < n; ++i) {
    const Grid2 g = fwd_grid(p.n_tokens, L[i].D, S);
    ly.l[i] = FwdLayer{L[i].x, L[i].a_c, L[i].b_c, L[i].y, L[i].D, static_cast<int>(g.gx),
                       g.n_sb, static_cast<int>(blk), L[i].act, L[i].kc};
    blk += static_cast<int64_t>(g.gx) * g.gy;
  }
  hipLaunchKernelGGL((fwd_layers_kernel<S, KCM, fwd_nb(S), kFwdNC, ACT, true>),
                     dim3(static_cast<unsigned>(blk)), dim3(256), 0, st, ly, p.seq);
}

// 0 / 1: every layer's activation; kActRuntime: mixed
inline int layers_act(const LayerOps* L, int n) {
  bool any = false, all = true;
  for (int i = 0; i < n; ++i) {
    any = any || L[i].act != 0;
    all = all && L[i].act != 0;
  }
  return all ? 1 : (any ? kActRuntime : 0);
}

template <int S, int KC, int ACT>
void bwd_layers_one(const Problem& p, const LayerOps* L, int n, hipStream_t st) {
  constexpr bool kSplit = KC >= 2;
  // (mixed activations run the fused pass: grouping admits them only where
  // both activations' single launches run it).  The two passes as the single
  // launches run them: without the activation as bwd_two_pass / bwd_two_pass_r,
  // with it as bwd_two_pass_g (the dx pass then forms g for every layer, also
  // those without dx); with 64 routes the taps pass in route halves
  constexpr bool kTwoG = ACT == 1 && bwd_two_pass_g(S, KC, true, true);
  constexpr bool kTwo = (ACT == 0 && (bwd_two_pass(S, KC, false, true) ||
                                      bwd_two_pass_r(S, KC, false, true))) ||
                        kTwoG;
  constexpr int kParts = kTwo ? taps_route_parts(KC) : 1;
  constexpr bool kTiers = !kTwo && !kSplit && kBwdMinWaves<S, KC, kBwdFused, true> == 2;
  const int n_cu = device_cu_count();
  // each layer's grid as bwd_one forms it (the taps pass has its own)
  BwdLayers ly{}, lt{};
  ly.n = lt.n = n;
  int64_t blk = 0, blkt = 0;
  bool any_dx = false;
  for (int i = 0; i < n; ++i) {
    const int64_t gx_l = cdiv(L[i].D, kBwdCW);
    const Grid2 g = kTiers ? bwd_grid_tiered(p.n_tokens, gx_l, L[i].D, S, n_cu)
                           : bwd_grid(p.n_tokens, L[i].D, S);
    ly.l[i] = BwdLayer{L[i].x, L[i].dy, L[i].dys, L[i].a_c, L[i].b_c, L[i].dx, L[i].part_da,
                       L[i].part_db, L[i].D, static_cast<int>(g.gx), static_cast<int>(g.gy),
                       g.gy1, g.n_old, g.n_total, static_cast<int>(blk), L[i].act,
                       kTwoG ? L[i].gbuf : nullptr};
    const int64_t tiles = static_cast<int64_t>(g.gx) * g.gy;
    // the dx pass of the two-pass form without the activation skips layers
    // without dx (no blocks: layer_index then never selects them)
    blk += kSplit && !kTwo ? 8 * KC * cdiv(tiles, 8)
                           : (kTwo && !kTwoG && L[i].dx == nullptr ? 0 : tiles);
    any_dx = any_dx || L[i].dx != nullptr;
    if constexpr (kTwo) {
      const Grid2 gt = bwd_taps_grid(p.n_tokens, cdiv(L[i].D, kTapsCW), L[i].D, S, n_cu / kParts);
      lt.l[i] = ly.l[i];
      lt.l[i].dx = nullptr;
      lt.l[i].gx = static_cast<int>(gt.gx);
      lt.l[i].gy = static_cast<int>(gt.gy);
      lt.l[i].gy1 = gt.gy1;
      lt.l[i].n_old = gt.n_old;
      lt.l[i].n_total = gt.n_total;
      lt.l[i].blk0 = static_cast<int>(blkt);
      const int64_t tiles_t = static_cast<int64_t>(gt.gx) * gt.gy;
      // (route halves: the 1-D split grid, the halves of a tile 8 ids apart)
      blkt += kParts > 1 ? 8 * kParts * cdiv(tiles_t, 8) : tiles_t;
    }
  }
  if constexpr (kTwo) {
    if (any_dx || kTwoG)
      hipLaunchKernelGGL((bwd_layers_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, true, false, kBwdDx>),
                         dim3(static_cast<unsigned>(blk)), dim3(64 * kBwdWPG), 0, st, ly, p.seq);
    hipLaunchKernelGGL((bwd_layers_kernel<S, KC, kBwdNB, kBwdNC, kTapsWPG, ACT, true, (kParts > 1), kBwdTaps>),
                       dim3(static_cast<unsigned>(blkt)), dim3(64 * kTapsWPG), 0, st, lt, p.seq);
  } else if constexpr (MOC_BWD_LEAN && bwd_lean(S, KC, true)) {
    // (layers whose dy is one element each, or none of them: one instantiation
    // per form; mixed forms keep every layer's rows by the general one)
    bool all_one = true;
    for (int i = 0; i < n; ++i) all_one = all_one && L[i].dys < 0;
    if (all_one)
      hipLaunchKernelGGL((bwd_lean_layers_kernel<S, ACT, true>), dim3(static_cast<unsigned>(blk)),
                         dim3(64 * kLeanWPG), 0, st, ly, p.seq);
    else
      hipLaunchKernelGGL((bwd_lean_layers_kernel<S, ACT, false>), dim3(static_cast<unsigned>(blk)),
                         dim3(64 * kLeanWPG), 0, st, ly, p.seq);
  } else {
    hipLaunchKernelGGL((bwd_layers_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, true, kSplit, kBwdFused>),
                       dim3(static_cast<unsigned>(blk)), dim3(64 * kBwdWPG), 0, st, ly, p.seq);
  }
}

template <int S>
void launch_fwd_layers(const Problem& p, const LayerOps* L, int n, hipStream_t st) {
  int mask = 0;
  for (int i = 0; i < n; ++i) mask |= L[i].kc;
  const int act = layers_act(L, n);
#define MOC_FWDL(M_)                                                          \
  case M_:                                                                    \
    if constexpr (M_ == 1 || M_ == 2 || M_ == 4) {                            \
      if (act == 0) fwd_layers_one<S, M_, 0>(p, L, n, st);                    \
      else if (act == 1) fwd_layers_one<S, M_, 1>(p, L, n, st);               \
      else fwd_layers_one<S, M_, kActRuntime>(p, L, n, st);                   \
    } else {                                                                  \
      fwd_layers_one<S, M_, kActRuntime>(p, L, n, st);                        \
    }                                                                         \
    break;
  switch (mask) {
    MOC_FWDL(1)
    MOC_FWDL(2)
    MOC_FWDL(3)
    MOC_FWDL(4)
    MOC_FWDL(5)
    MOC_FWDL(6)
    MOC_FWDL(7)
    default: break;
  }
#undef MOC_FWDL
}

// The layers here share their route chunks (L[0].kc).
template <int S>
void launch_bwd_layers(const Problem& p, const LayerOps* L, int n, hipStream_t st) {
  const int act = layers_act(L, n);
#define MOC_BWDL(KC_)                                              \
  if (L[0].kc == KC_) {                                            \
    if (act == 0) bwd_layers_one<S, KC_, 0>(p, L, n, st);          \
    else if (act == 1) bwd_layers_one<S, KC_, 1>(p, L, n, st);     \
    else bwd_layers_one<S, KC_, kActRuntime>(p, L, n, st);         \
    return;                                                        \
  }
  MOC_BWDL(1)
  MOC_BWDL(2)
  MOC_BWDL(4)
#undef MOC_BWDL
}

// Dispatch over (KC, activation, dtype) for one S.
template <int S>
void launch_fwd(const Problem& p, const void* x, const void* a_c, const void* b_c, void* y,
                hipStream_t st) {
  const int kc = route_chunks(p.K);
  const bool bf = p.x_dt == DT_BF16, act = p.activation != 0;
#define MOC_FWD(KC_)                                              \
  if (kc == KC_) {                                                \
    if (bf) {                                                     \
      if (act) fwd_one<S, KC_, true, true>(p, x, a_c, b_c, y, st); \
      else fwd_one<S, KC_, false, true>(p, x, a_c, b_c, y, st);   \
    } else {                                                      \
      if (act) fwd_one<S, KC_, true, false>(p, x, a_c, b_c, y, st); \
      else fwd_one<S, KC_, false, false>(p, x, a_c, b_c, y, st);  \
    }                                                             \
    return;                                                       \
  }
  MOC_FWD(1)
  MOC_FWD(2)
  MOC_FWD(4)
#undef MOC_FWD
}

template <int S>
void launch_bwd(const Problem& p, const void* x, const void* dy, const void* a_c, const void* b_c,
                void* dx, float* part_da, float* part_db, float* gbuf, hipStream_t st) {
  const int kc = route_chunks(p.K);
  const bool bf = p.x_dt == DT_BF16, act = p.activation != 0;
  // 9 to 16 taps: up to 16 routes (the two-pass form; with more routes bf16
  // runs backward_chunks and fp32 the route parts of moc_routesplit.hip: the
  // forms over more routes spill past what the compiler handles)
  if constexpr (S > 8) {
    if (kc == 1) {
      if (bf) {
        if (act) bwd_one<S, 1, true, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st);
        else bwd_one<S, 1, false, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st);
      } else {
        if (act) bwd_one<S, 1, true, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st);
        else bwd_one<S, 1, false, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st);
      }
    }
  } else {
#define MOC_BWD(KC_)                                                                          \
  if (kc == KC_) {                                                                            \
    if (bf) {                                                                                 \
      if (act) bwd_one<S, KC_, true, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st); \
      else bwd_one<S, KC_, false, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st);  \
    } else {                                                                                  \
      if (act) bwd_one<S, KC_, true, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st); \
      else bwd_one<S, KC_, false, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, gbuf, st); \
    }                                                                                         \
    return;                                                                                   \
  }
  MOC_BWD(1)
  MOC_BWD(2)
  MOC_BWD(4)
#undef MOC_BWD
  }
}

// Pieces of the backward of bf16 layers with 9 to 16 taps and 17 to 64 routes
// (backward_chunks): the dx pass over every route (dx, and with the activation
// g = dy silu'(P) into gbuf), and the taps pass of one 16-route chunk on its
// own operands (a_c16 [N, 16], b_c16 [16, S, D]), into the partials of a
// 16-route problem's plan.  (The one-pass and route-split forms do not fit
// these sizes: spills past what the compiler handles, LDS past 160 KB.)
template <int S>
void launch_dx_pass(const Problem& p, const void* x, const void* dy, const uint16_t* a_c,
                    const uint16_t* b_c, void* dx, float* gbuf, hipStream_t st) {
  if constexpr (S > 8) {
    const Grid2 g = bwd_grid(p.n_tokens, p.D, S);
    const int gx = static_cast<int>(g.gx), gy = static_cast<int>(g.gy);
    const bool act = p.activation != 0;
    auto run = [&](auto kct, auto actt) {
      constexpr int KC = decltype(kct)::value;
      constexpr bool ACT = decltype(actt)::value;
      hipLaunchKernelGGL((bwd_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, true, false, kBwdDx>),
                         dim3(g.gx, g.gy), dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, a_c, b_c, dx,
                         nullptr, nullptr, p.seq, p.D, gx, gy, g.gy1, g.n_old, g.n_total, gbuf);
    };
    if (dx == nullptr && !act) return;
    if (route_chunks(p.K) == 2) {
      if (act) run(std::integral_constant<int, 2>{}, std::true_type{});
      else run(std::integral_constant<int, 2>{}, std::false_type{});
    } else {
      if (act) run(std::integral_constant<int, 4>{}, std::true_type{});
      else run(std::integral_constant<int, 4>{}, std::false_type{});
    }
  }
}

template <int S>
void launch_taps_chunk(const Problem& p, const void* x, const void* dy, const uint16_t* a_c16,
                       const uint16_t* b_c16, float* part_da, float* part_db, float* gbuf,
                       hipStream_t st) {
  if constexpr (S > 8) {
    const Grid2 gt = bwd_taps_grid(p.n_tokens, cdiv(p.D, kTapsCW), p.D, S, device_cu_count());
    const int gx = static_cast<int>(gt.gx), gy = static_cast<int>(gt.gy);
    if (p.activation != 0)
      hipLaunchKernelGGL((bwd_kernel<S, 1, kBwdNB, kBwdNC, kTapsWPG, true, true, false, kBwdTaps>),
                         dim3(gt.gx, gt.gy), dim3(64 * kTapsWPG), 0, st, x, dy, p.dy_stride, a_c16, b_c16,
                         nullptr, part_da, part_db, p.seq, p.D, gx, gy, gt.gy1, gt.n_old, gt.n_total, gbuf);
    else
      hipLaunchKernelGGL((bwd_kernel<S, 1, kBwdNB, kBwdNC, kTapsWPG, false, true, false, kBwdTaps>),
                         dim3(gt.gx, gt.gy), dim3(64 * kTapsWPG), 0, st, x, dy, p.dy_stride, a_c16, b_c16,
                         nullptr, part_da, part_db, p.seq, p.D, gx, gy, gt.gy1, gt.n_old, gt.n_total, gbuf);
  }
}

// Prefill from a cache (Pre, fixed-length sequences): the forward on
// fwd_kernel's grid; the backward's fused pass (for every K, activation and
// dtype) on the grid that owns the partials, so the workspace and stage 2 are
// those of moc_backward.
template <int S, int KC, bool ACT, bool BF>
void fwd_pre_one(const Problem& p, const void* x, const void* a_c, const void* b_c, void* y,
                 const Pre& pre, hipStream_t st) {
  if constexpr (!kcOK<KC, BF>) return;
  else {
  using E = typename CT<BF>::elem;
  const Grid2 g = fwd_grid(p.n_tokens, p.D, S);
  hipLaunchKernelGGL((fwd_pre_kernel<S, KC, fwd_nb(S), kFwdNC, ACT, BF>), dim3(g.gx, g.gy), dim3(256),
                     0, st, x, static_cast<const E*>(a_c), static_cast<const E*>(b_c), y, p.seq,
                     p.D, g.n_sb, pre);
  }
}

template <int S, int KC, bool ACT, bool BF>
void bwd_pre_one(const Problem& p, const void* x, const void* dy, const void* a_c,
                 const void* b_c, void* dx, float* part_da, float* part_db, const Pre& pre,
                 hipStream_t st) {
  if constexpr (!kcOK<KC, BF>) return;
  else {
  using E = typename CT<BF>::elem;
  const Grid2 g = bwd_partials_grid(p);
  // the two-pass shapes of the plain backward: without the activation all of
  // them; with it those of pre_two_pass_g
  constexpr bool kTwo = BF && (bwd_two_pass(S, KC, ACT, BF) ||
                               (bwd_two_pass_r(S, KC, ACT, BF) && pre_two_pass_r(S)) ||
                               (bwd_two_pass_g(S, KC, ACT, BF) && pre_two_pass_g(S, KC)));
  if constexpr (kTwo) {
    // the dx pass: without the activation the plain one (dx reads no cache);
    // with it bwd_pre_dx_kernel, which forms P with the cache and writes g to
    // pre.g (also without dx).  Then the taps pass with the cache (reading g in
    // place of dy with the activation; g is the taps grid here), with 64 routes
    // in route halves on a 1-D grid as bwd_one runs it.
    const auto* a = static_cast<const E*>(a_c);
    const auto* b = static_cast<const E*>(b_c);
    const Grid2 gd = bwd_grid(p.n_tokens, p.D, S);
    if constexpr (ACT) {
      hipLaunchKernelGGL((bwd_pre_dx_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, BF>),
                         dim3(gd.gx, gd.gy), dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, a, b, dx,
                         p.seq, p.D, static_cast<int>(gd.gx), static_cast<int>(gd.gy), gd.gy1,
                         gd.n_old, gd.n_total, pre);
    } else if (dx != nullptr) {
      hipLaunchKernelGGL((bwd_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, BF, false, kBwdDx>),
                         dim3(gd.gx, gd.gy), dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, a, b, dx,
                         part_da, part_db, p.seq, p.D, static_cast<int>(gd.gx),
                         static_cast<int>(gd.gy), gd.gy1, gd.n_old, gd.n_total);
    }
    constexpr int kParts = taps_route_parts(KC);
    const dim3 tgrid = kParts > 1 ? dim3(static_cast<unsigned>(8 * kParts * cdiv(int64_t(g.gx) * g.gy, 8)))
                                  : dim3(g.gx, g.gy);
    hipLaunchKernelGGL((bwd_pre_taps_kernel<S, KC, kBwdNB, kBwdNC, kTapsWPG, ACT, BF, (kParts > 1)>),
                       tgrid, dim3(64 * kTapsWPG), 0, st, x, dy, p.dy_stride, a, b, part_da, part_db,
                       p.seq, p.D, static_cast<int>(g.gx), static_cast<int>(g.gy), g.gy1, g.n_old,
                       g.n_total, pre);
  } else {
    // the fused pass; 64 routes (with SiLU and 2 taps, or 8 taps without):
    // split in route chunks on a 1-D grid, as bwd_one does
    constexpr bool kSplit = BF && KC >= 4;
    const dim3 grid = kSplit ? dim3(static_cast<unsigned>(8 * KC * cdiv(int64_t(g.gx) * g.gy, 8)))
                             : dim3(g.gx, g.gy);
    hipLaunchKernelGGL((bwd_pre_kernel<S, KC, kBwdNB, kBwdNC, kBwdWPG, ACT, BF, kSplit>), grid,
                       dim3(64 * kBwdWPG), 0, st, x, dy, p.dy_stride, static_cast<const E*>(a_c),
                       static_cast<const E*>(b_c), dx, part_da, part_db, p.seq, p.D,
                       static_cast<int>(g.gx), static_cast<int>(g.gy), g.gy1, g.n_old, g.n_total,
                       pre);
  }
  }
}

template <int S>
void launch_fwd_pre(const Problem& p, const void* x, const void* a_c, const void* b_c, void* y,
                    const Pre& pre, hipStream_t st) {
  const int kc = route_chunks(p.K);
  const bool bf = p.x_dt == DT_BF16, act = p.activation != 0;
#define MOC_FWD(KC_)                                                        \
  if (kc == KC_) {                                                          \
    if (bf) {                                                               \
      if (act) fwd_pre_one<S, KC_, true, true>(p, x, a_c, b_c, y, pre, st); \
      else fwd_pre_one<S, KC_, false, true>(p, x, a_c, b_c, y, pre, st);    \
    } else {                                                                \
      if (act) fwd_pre_one<S, KC_, true, false>(p, x, a_c, b_c, y, pre, st); \
      else fwd_pre_one<S, KC_, false, false>(p, x, a_c, b_c, y, pre, st);   \
    }                                                                       \
    return;                                                                 \
  }
  MOC_FWD(1)
  MOC_FWD(2)
  MOC_FWD(4)
#undef MOC_FWD
}

template <int S>
void launch_bwd_pre(const Problem& p, const void* x, const void* dy, const void* a_c,
                    const void* b_c, void* dx, float* part_da, float* part_db, const Pre& pre,
                    hipStream_t st) {
  const int kc = route_chunks(p.K);
  const bool bf = p.x_dt == DT_BF16, act = p.activation != 0;
#define MOC_BWD(KC_)                                                                                \
  if (kc == KC_) {                                                                                  \
    if (bf) {                                                                                       \
      if (act) bwd_pre_one<S, KC_, true, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, pre, st);  \
      else bwd_pre_one<S, KC_, false, true>(p, x, dy, a_c, b_c, dx, part_da, part_db, pre, st);     \
    } else {                                                                                        \
      if (act) bwd_pre_one<S, KC_, true, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, pre, st); \
      else bwd_pre_one<S, KC_, false, false>(p, x, dy, a_c, b_c, dx, part_da, part_db, pre, st);    \
    }                                                                                               \
    return;                                                                                         \
  }
  MOC_BWD(1)
  MOC_BWD(2)
  MOC_BWD(4)
#undef MOC_BWD
}

#define MOC_DECLARE_S(S_)                                                                     \
  extern template void launch_fwd<S_>(const Problem&, const void*, const void*, const void*, \
                                      void*, hipStream_t);                                    \
  extern template void launch_bwd<S_>(const Problem&, const void*, const void*, const void*, \
                                      const void*, void*, float*, float*, float*, hipStream_t); \
  extern template void launch_fwd_layers<S_>(const Problem&, const LayerOps*, int, hipStream_t); \
  extern template void launch_bwd_layers<S_>(const Problem&, const LayerOps*, int, hipStream_t); \
  extern template void launch_fwd_pre<S_>(const Problem&, const void*, const void*, const void*, \
                                          void*, const Pre&, hipStream_t);                    \
  extern template void launch_bwd_pre<S_>(const Problem&, const void*, const void*, const void*, \
                                          const void*, void*, float*, float*, const Pre&,     \
                                          hipStream_t);
MOC_DECLARE_S(2)
MOC_DECLARE_S(3)
MOC_DECLARE_S(4)
MOC_DECLARE_S(5)
MOC_DECLARE_S(6)
MOC_DECLARE_S(7)
MOC_DECLARE_S(8)
#undef MOC_DECLARE_S
// 9 to 16 taps: the single-layer forward and backward only
#define MOC_DECLARE_S_LONG(S_)                                                                \
  extern template void launch_fwd<S_>(const Problem&, const void*, const void*, const void*, \
                                      void*, hipStream_t);                                    \
  extern template void launch_bwd<S_>(const Problem&, const void*, const void*, const void*, \
                                      const void*, void*, float*, float*, float*, hipStream_t); \
  extern template void launch_dx_pass<S_>(const Problem&, const void*, const void*,           \
                                          const uint16_t*, const uint16_t*, void*, float*,   \
                                          hipStream_t);                                       \
  extern template void launch_taps_chunk<S_>(const Problem&, const void*, const void*,        \
                                             const uint16_t*, const uint16_t*, float*, float*, \
                                             float*, hipStream_t);
MOC_DECLARE_S_LONG(9)
MOC_DECLARE_S_LONG(10)
MOC_DECLARE_S_LONG(11)
MOC_DECLARE_S_LONG(12)
MOC_DECLARE_S_LONG(13)
MOC_DECLARE_S_LONG(14)
MOC_DECLARE_S_LONG(15)
MOC_DECLARE_S_LONG(16)
#undef MOC_DECLARE_S_LONG

}  // namespace mfma
}  // namespace moc
