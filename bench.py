#!/usr/bin/env python3
"""MoC hot-path benchmark on one MI355X.

Headline: the MoC layer forward + backward at
B=4, T=4096, D=2048, z_dim=2048, K=16, S=4, bf16, softmax routing, fused SiLU,
basis init_std=0.002, router ~ N(0, 0.02), loss = y.sum(), gradients of x, z,
router and basis.  One step = zero grads, forward, backward on synthetic
inputs already resident in HBM.  Printed as one JSON line:

  value         tokens/s (millions) of the full layer step (router GEMMs + MoC)
  roofline      HBM roofline of the dominant entry (the fused backward)
  kernel_scope  forward / backward entry times alone (no router GEMMs)
  prefill       a headline-shape chunk continuing from a cache (bench_prefill)
  config3_varlen, config5_qkv  BASELINE configs[2] and configs[4] (the
                `--config 3` / `--config 5` measurements)
  shapes        forward / backward entry us at other kernel sizes (8, 12, 16
                taps) and an even channel count that is not a multiple of 4
  decode        configs[3]: batch-256 single-token steps: us per MoC.step call
                (host-synchronised each step, and back to back), per MoC.step
                replayed from a HIP graph, and per launch of the one-launch
                decode step alone (graph-replayed); the 512 steps as one
                MoC.forward call from the prompt's cache (inputs known up front);
                and (update_us) moc_update per launch in bf16 / fp32 with a
                contiguous or slot-major cache (matrix-core and generic kernels)
                and at 12 / 16 taps
  cpu_baseline  the CPU oracle on a bounded slice of the same workload

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]
       python bench.py --config 3|5     (BASELINE configs[2] / configs[4] instead)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "mixture-of-convolutions_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "fwd+bwd Mtok/s + roofline % (B4 T4096 D2048 K16 S4 bf16); decode us/step"
HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
CFG = dict(B=4, T=4096, D=2048, Z=2048, K=16, S=4)
# HBM bytes per launch of the backward stage-1 kernel at CFG: rocprofv3
# FETCH_SIZE (69220 KiB) and WRITE_SIZE (99410 KiB) per dispatch of
# `bench.py --counters bwd`, each scaled by what the counter reads for a copy of
# 128 MiB (`--counters copy`: FETCH_SIZE 65548 KiB -> factor 2.0, WRITE_SIZE
# 131072 KiB -> factor 1.0); profiles/traffic_fwd_bwd_config2.md
TRAFFIC_BWD = 243_558_400
# input sets the timed loops cycle through: 3 x (x, z) = 402 MB at CFG, more
# than the 256 MB last-level cache, so each step reads its inputs from HBM
ROTATE = 3
DECODE = dict(B=256, D=2048, Z=2048, K=16, S=4, prompt=1024, steps=512)


def bytes_fwd(N, D, K, S, ex=2, ea=2, eb=2):
    return 2 * N * D * ex + N * K * ea + K * S * D * eb


def bytes_bwd(N, D, K, S, ex=2, ea=2, eb=2):
    return 3 * N * D * ex + 2 * N * K * ea + 2 * K * S * D * eb


def flops_fwd(N, D, K, S):
    return 2 * N * D * S * (K + 1)


def flops_bwd(N, D, K, S, silu=True):
    return N * D * S * (6 * K + 3 + 2 * int(silu))


def build_layer(dev, dtype=torch.bfloat16, cfg=CFG, seed=0, n_sets=1):
    """The headline layer and ``n_sets`` input pairs (x, z): the first drawn
    from the seeded CPU generator (the BASELINE configs[1] recipe), the others
    on the GPU (same distribution, only there to rotate through)."""
    import moc
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    m = moc.MoC(cfg["D"], cfg["Z"], cfg["S"], cfg["K"], activation="silu", init_std=0.002)
    with torch.no_grad():
        m.router.copy_(torch.randn(cfg["K"], cfg["Z"], generator=g) * 0.02)
    m = m.to(dev, dtype)
    x = (torch.randn(cfg["B"], cfg["T"], cfg["D"], generator=g)).to(dev, dtype).requires_grad_()
    z = (torch.randn(cfg["B"], cfg["T"], cfg["Z"], generator=g)).to(dev, dtype).requires_grad_()
    sets = [(x, z)]
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    for _ in range(n_sets - 1):
        xi = torch.randn(x.shape, generator=gd, device=dev).to(dtype).requires_grad_()
        zi = torch.randn(z.shape, generator=gd, device=dev).to(dtype).requires_grad_()
        sets.append((xi, zi))
    return m, sets


class _Cycle:
    """Round-robin over a list (the input sets of a timed loop)."""

    def __init__(self, items):
        self.items, self.i = items, 0

    def next(self):
        v = self.items[self.i % len(self.items)]
        self.i += 1
        return v


def time_region(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms


def bench_layer(dev, steps, warmup, rotate=ROTATE):
    m, sets = build_layer(dev, n_sets=rotate)
    cyc = _Cycle(sets)

    def step():
        x, z = cyc.next()
        m.zero_grad(set_to_none=True)
        x.grad = None
        z.grad = None
        y, _ = m(x, z)
        y.sum().backward()

    return time_region(step, steps, warmup)


class _HipEvents:
    """hipEvent_t pairs from libamdhip64 (ctypes), for the profiling hook of
    libmoc_hip.so (moc_profile_events): times one kernel on its own stream."""

    def __init__(self, n):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float),
                                                 ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.pairs = []
        for _ in range(n):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            assert self.hip.hipEventCreate(ctypes.byref(a)) == 0
            assert self.hip.hipEventCreate(ctypes.byref(b)) == 0
            self.pairs.append((a, b))

    def total_ms(self):
        import ctypes
        tot = 0.0
        for a, b in self.pairs:
            ms = ctypes.c_float()
            assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
            tot += ms.value
        return tot

    def close(self):
        for a, b in self.pairs:
            self.hip.hipEventDestroy(a)
            self.hip.hipEventDestroy(b)


def time_kernel(fn, steps, warmup):
    """Average duration (ms) of the main kernel of the C-ABI call fn()."""
    from moc import _lib
    L = _lib.lib()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = _HipEvents(steps)
    for a, b in ev.pairs:
        L.moc_profile_events(a, b)
        fn()
    L.moc_profile_events(None, None)
    torch.cuda.synchronize()
    ms = ev.total_ms() / steps
    ev.close()
    return ms


def entry_calls(dev, rotate=ROTATE):
    """The forward and backward C-ABI entries as the layer calls them, as two
    zero-argument callables (fwd, bwd): on the routing weights the router
    kernel forms (softmax of the bf16 logits), routing "softmax weights given",
    so the backward returns the logits gradient.  The backward gets a full
    (contiguous) dy, the general case, not the broadcast row of y.sum().  Each
    call takes the next of ``rotate`` input sets."""
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX, ROUTE_SOFTMAX_WEIGHTS
    m, sets = build_layer(dev, n_sets=rotate)
    basis = m.conv_bases.detach()
    args = []
    with torch.no_grad():
        for x, z in sets:
            weights = ops.router_forward(z, m.router, routing=ROUTE_SOFTMAX)
            xd = x.detach()
            args.append((xd, weights, torch.ones_like(xd)))
    cf, cb = _Cycle(args), _Cycle(args)

    def fwd():
        xd, w, _ = cf.next()
        return ops.launch_forward(xd, w, basis, activation_flag=1, routing=ROUTE_SOFTMAX_WEIGHTS)

    def bwd():
        xd, w, dy = cb.next()
        return ops.launch_backward(xd, w, basis, dy, activation_flag=1, need_x=True,
                                   routing=ROUTE_SOFTMAX_WEIGHTS)
    return fwd, bwd


SHAPES = (("bf16 S4 D2048", torch.bfloat16, 4, 2048, 16), ("bf16 S4 D2050", torch.bfloat16, 4, 2050, 16),
          ("bf16 S8 D2048", torch.bfloat16, 8, 2048, 16), ("bf16 S12 D2048", torch.bfloat16, 12, 2048, 16),
          ("bf16 S16 D2048", torch.bfloat16, 16, 2048, 16), ("fp32 S8 D2048", torch.float32, 8, 2048, 16),
          ("fp32 S12 D2048", torch.float32, 12, 2048, 16), ("fp32 S16 D2048", torch.float32, 16, 2048, 16),
          ("fp32 S8 K32 D2048", torch.float32, 8, 2048, 32), ("fp32 S4 K32 D2048", torch.float32, 4, 2048, 32),
          ("fp32 S4 K64 D2048", torch.float32, 4, 2048, 64), ("bf16 S12 K32 D2048", torch.bfloat16, 12, 2048, 32))


def shape_calls(dev):
    """Forward and backward entries (moc_forward / moc_backward) at the headline
    token count (B 4 x T 4096), SiLU, softmax weights given, full dy, for the
    kernel sizes, channel counts and route counts of SHAPES: the headline shape,
    an even channel count that is not a multiple of 4, 8 / 12 / 16 taps (bf16
    and fp32), fp32 with 32 routes (4 and 8 taps) and 64, and bf16 with 12 taps
    and 32 routes.
    Returns [(label, fwd, bwd)]."""
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX_WEIGHTS
    B, T = CFG["B"], CFG["T"]
    out = []
    for label, dt, S, D, K in SHAPES:
        g = torch.Generator().manual_seed(S * 10000 + D)
        x = torch.randn(B, T, D, generator=g).to(dev, dt)
        w = torch.softmax(torch.randn(B, T, K, generator=g), -1).to(dev, dt)
        b = ((torch.rand(K, S, D, generator=g) * 2 - 1) * 0.002 * 3 ** 0.5).to(dev, dt)
        dy = torch.randn(B, T, D, generator=g).to(dev, dt)
        out.append((label,
                    lambda x=x, w=w, b=b: ops.launch_forward(x, w, b, activation_flag=1,
                                                             routing=ROUTE_SOFTMAX_WEIGHTS),
                    lambda x=x, w=w, b=b, dy=dy: ops.launch_backward(
                        x, w, b, dy, activation_flag=1, need_x=True, routing=ROUTE_SOFTMAX_WEIGHTS)))
    return out


def bench_shapes(dev, steps, warmup):
    """us per forward / backward entry for each of shape_calls."""
    res = {}
    for label, fwd, bwd in shape_calls(dev):
        res[label] = {"fwd_us": round(time_region(fwd, steps, warmup) * 1e3, 2),
                      "bwd_us": round(time_region(bwd, steps, warmup) * 1e3, 2)}
    torch.cuda.empty_cache()
    return res


def bench_prefill(dev, steps, warmup, rotate=ROTATE):
    """A chunk of the headline layer shape continuing from a cache (chunked
    prefill, moc/api.py:299-309): B=4 x T=4096 new tokens per sequence at D=2048,
    K=16, S=4, SiLU, softmax routing.  Times (us, inputs rotated):
      fwd_kernel_us / plain_fwd_kernel_us  the prefill forward kernel (cache
          halo, final state written) and the plain forward kernel on the same
          x and weights without a cache;
      bwd_us  moc_backward_prefill (stage 1, stage 2, cache gradient);
      module_fwd_us  MoC.forward(x, z, cache=..., output_final_state=True)
          without autograd: router GEMM + the prefill forward launch."""
    pre_fwd, plain_fwd, pre_bwd, module_fwd = prefill_calls(dev, rotate, parts=True)
    return {"B": CFG["B"], "T": CFG["T"], "D": CFG["D"], "K": CFG["K"], "S": CFG["S"],
            "fwd_kernel_us": round(time_kernel(pre_fwd, steps, warmup) * 1e3, 2),
            "plain_fwd_kernel_us": round(time_kernel(plain_fwd, steps, warmup) * 1e3, 2),
            "bwd_us": round(time_region(pre_bwd, steps, warmup) * 1e3, 2),
            "module_fwd_us": round(time_region(module_fwd, steps, warmup) * 1e3, 2)}


def prefill_calls(dev, rotate=ROTATE, parts=False):
    """The calls bench_prefill times, on ``rotate`` input sets: (prefill forward
    entry, plain forward entry, prefill backward entry, module forward) with
    parts, else one callable running the module forward and the backward entry."""
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX, ROUTE_SOFTMAX_WEIGHTS
    m, sets = build_layer(dev, n_sets=rotate)
    basis = m.conv_bases.detach()
    B, D, S = CFG["B"], CFG["D"], CFG["S"]
    g = torch.Generator(device=dev).manual_seed(7)
    args = []
    with torch.no_grad():
        for x, z in sets:
            w = ops.router_forward(z, m.router, routing=ROUTE_SOFTMAX)
            c = torch.randn(B, D, S, generator=g, device=dev).to(torch.bfloat16)
            args.append((x.detach(), z.detach(), w, c, torch.ones_like(x)))
    cyc = _Cycle(args)

    def pre_fwd():
        x, _, w, c, _ = cyc.next()
        return ops.launch_forward_prefill(x, w, basis, c, activation_flag=1, final_state=True,
                                          routing=ROUTE_SOFTMAX_WEIGHTS)

    def plain_fwd():
        x, _, w, _, _ = cyc.next()
        return ops.launch_forward(x, w, basis, activation_flag=1, routing=ROUTE_SOFTMAX_WEIGHTS)

    def pre_bwd():
        x, _, w, c, dy = cyc.next()
        return ops.launch_backward_prefill(x, w, basis, c, dy, activation_flag=1, need_x=True,
                                           need_cache=True, routing=ROUTE_SOFTMAX_WEIGHTS)

    def module_fwd():
        x, z, _, c, _ = cyc.next()
        with torch.no_grad():
            return m(x, z, cache=c, output_final_state=True)

    if parts:
        return pre_fwd, plain_fwd, pre_bwd, module_fwd

    def both():
        module_fwd()
        pre_bwd()
    return both


def bench_entries(dev, steps, warmup, rotate=ROTATE):
    """Forward and backward C-ABI entries alone, as the layer calls them:
    (entry ms fwd, entry ms bwd, main-kernel ms fwd, main-kernel ms bwd)."""
    fwd, bwd = entry_calls(dev, rotate)
    return (time_region(fwd, steps, warmup), time_region(bwd, steps, warmup),
            time_kernel(fwd, steps, warmup), time_kernel(bwd, steps, warmup))


def counter_run(dev, which, reps=3):
    """A short program for profiler passes (rocprofv3 --pmc or --kernel-trace):
    `reps` calls, after two untimed ones, of
      fwd / bwd  one C-ABI entry at the headline config (entry_calls);
      step       the headline layer step (bench_layer's step, inputs rotated);
      decode     the one-launch decode step of configs[3] (batch 256);
      update     moc_update at configs[3]'s layer shape in the four forms of
                 update_calls (matrix-core and generic decode kernels);
      shapes     the forward and backward entries of shape_calls (other kernel
                 sizes and channel counts at the headline token count);
      c3         the configs[2] varlen layer step (config3_step);
      c5         the configs[4] QKV triple step through MoCGroup;
      prefill    a headline-shape chunk continuing from a cache: the module
                 forward (router + prefill launch), then the prefill backward
                 entry (bench_prefill's workload);
      copy       a bf16 copy of 128 MiB, the kernel of known traffic that
                 calibrates FETCH_SIZE and WRITE_SIZE."""
    if which == "copy":
        a = torch.randn(64 * 1024 * 1024, device=dev).bfloat16()
        b = torch.empty_like(a)
        fn = lambda: b.copy_(a)  # noqa: E731
    elif which in ("fwd", "bwd"):
        fwd, bwd = entry_calls(dev, 1)
        fn = fwd if which == "fwd" else bwd
    elif which == "step":
        m, sets = build_layer(dev, n_sets=ROTATE)
        cyc = _Cycle(sets)

        def fn():
            x, z = cyc.next()
            m.zero_grad(set_to_none=True)
            x.grad = None
            z.grad = None
            y, _ = m(x, z)
            y.sum().backward()
    elif which == "decode":
        fn = decode_step_call(dev)
    elif which == "update":
        calls = [f for _, f in update_calls(dev)]

        def fn():
            for f in calls:
                f()
    elif which == "shapes":
        calls = [f for _, fw, bw in shape_calls(dev) for f in (fw, bw)]

        def fn():
            for f in calls:
                f()
    elif which == "prefill":
        fn = prefill_calls(dev, 1)
    elif which == "c3":
        fn = config3_step(dev)[0]
    else:
        fn = config5_step(dev)[0](True)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    print(f"counter run: {reps} x {which}", flush=True)


def decode_step_call(dev):
    """One launch of the decode step MoC.step runs at configs[3] (batch 256,
    D 2048, z_dim 2048, K 16, S 4, softmax, SiLU) on a scratch cache."""
    import moc
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX
    c = DECODE
    g = torch.Generator().manual_seed(0)
    m = moc.MoC(c["D"], c["Z"], c["S"], c["K"], activation="silu")
    with torch.no_grad():
        m.router.copy_(torch.randn(c["K"], c["Z"], generator=g) * 0.02)
    m = m.to(dev, torch.bfloat16)
    xt = torch.randn(c["B"], c["D"], generator=g).to(dev, torch.bfloat16)
    zt = torch.randn(c["B"], c["Z"], generator=g).to(dev, torch.bfloat16)
    cache = torch.randn(c["B"], c["D"], c["S"], generator=g).to(dev, torch.bfloat16)
    basis, router = m.conv_bases.detach(), m.router.detach()
    return lambda: ops.launch_decode_step(xt, zt, router, basis, cache, activation_flag=1,
                                          routing=ROUTE_SOFTMAX)


UPDATE_FORMS = (("bf16", "contiguous", 4), ("fp32", "contiguous", 4), ("bf16", "slot-major", 4),
                ("fp32", "slot-major", 4), ("bf16", "contiguous", 12), ("fp32", "contiguous", 16))


def update_calls(dev):
    """moc_update (one decode step from given logits) at configs[3]'s layer
    shape (batch 256, D 2048, K 16, S 4, softmax, SiLU) in four forms: bf16 with
    a contiguous [B, D, S] cache (the matrix-core decode kernel), and fp32 data
    or a slot-major cache ([B, D, S] view of a [B, S, D] store), which take the
    generic tile kernel; and the tile kernel at 12 taps (bf16) and 16 taps
    (fp32).  Returns [(label, fn)]."""
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX
    c = DECODE
    B, D, K = c["B"], c["D"], c["K"]
    calls = []
    for dt_name, layout, S in UPDATE_FORMS:
        dt = torch.bfloat16 if dt_name == "bf16" else torch.float32
        g = torch.Generator().manual_seed(0)
        x = torch.randn(B, D, generator=g).to(dev, dt)
        lg = torch.randn(B, K, generator=g).to(dev, dt)
        b = (torch.randn(K, S, D, generator=g) * 0.2).to(dev, dt)
        cache = torch.randn(B, D, S, generator=g).to(dev, dt)
        if layout == "slot-major":
            cache = cache.transpose(1, 2).contiguous().transpose(1, 2)
        calls.append((f"{dt_name} {layout}" + ("" if S == c["S"] else f" S{S}"),
                      lambda x=x, lg=lg, b=b, cache=cache: ops.launch_update(
                          x, lg, b, cache, activation_flag=1, routing=ROUTE_SOFTMAX)))
    return calls


def bench_update(dev):
    """us per moc_update launch in each form of update_calls, from a HIP graph
    of 32 launches replayed 20 times (best of 3)."""
    out = {}
    for label, fn in update_calls(dev):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(32):
                fn()
        ms = min(time_region(graph.replay, 20, 3) for _ in range(3))
        out[label] = round(ms * 1e3 / 32, 2)
    return out


def bench_decode(dev):
    """prefill a 1024-token prompt, then 512 single-token steps."""
    import moc
    from moc import ops
    from moc._lib import ROUTE_SOFTMAX
    c = DECODE
    g = torch.Generator().manual_seed(0)
    torch.manual_seed(0)
    m = moc.MoC(c["D"], c["Z"], c["S"], c["K"], activation="silu")
    with torch.no_grad():
        m.router.copy_(torch.randn(c["K"], c["Z"], generator=g) * 0.02)
    m = m.to(dev, torch.bfloat16)
    with torch.no_grad():
        xp = torch.randn(c["B"], c["prompt"], c["D"], generator=g).to(dev, torch.bfloat16)
        zp = torch.randn(c["B"], c["prompt"], c["Z"], generator=g).to(dev, torch.bfloat16)
        _, cache = m(xp, zp, output_final_state=True)
        del xp, zp
        # step t's inputs as a decode loop holds them: the current token's
        # activations, each a contiguous [B, 1, D] / [B, 1, Z] tensor
        xs = torch.randn(c["steps"], c["B"], 1, c["D"], generator=g).to(dev, torch.bfloat16)
        zs = torch.randn(c["steps"], c["B"], 1, c["Z"], generator=g).to(dev, torch.bfloat16)
        for t in range(8):  # warm-up on a scratch copy
            m.step(xs[t], zs[t], cache=cache.clone())
        torch.cuda.synchronize()
        per_step = []
        for t in range(c["steps"]):
            t0 = time.perf_counter()
            y, _ = m.step(xs[t], zs[t], cache=cache, output_final_state=True)
            torch.cuda.synchronize()
            per_step.append((time.perf_counter() - t0) * 1e6)
        # back to back, one synchronisation at the end: what a decode loop sees
        # when it does not wait for each token on the host
        t0 = time.perf_counter()
        for t in range(c["steps"]):
            m.step(xs[t], zs[t], cache=cache)
        torch.cuda.synchronize()
        async_us = (time.perf_counter() - t0) * 1e6 / c["steps"]
        # MoC.step itself captured in a HIP graph (static x / z buffers, cache
        # updated in place): 32 module steps per graph launch
        xin = xs[0].clone()
        zin = zs[0].clone()
        gcache = cache.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                m.step(xin, zin, cache=gcache)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        mgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(mgraph):
            for _ in range(32):
                m.step(xin, zin, cache=gcache)
        module_graph_us = time_region(mgraph.replay, 20, 3) * 1e3 / 32
        # kernel-only: 32 launches of the one-launch decode step that MoC.step
        # runs (router GEMM + softmax + update), captured in one HIP graph
        xt = xs[0, :, 0].contiguous()
        zt = zs[0, :, 0].contiguous()
        basis = m.conv_bases.detach()
        router = m.router.detach()
        scratch = cache.clone()
        step = lambda: ops.launch_decode_step(xt, zt, router, basis, scratch,  # noqa: E731
                                              activation_flag=1, routing=ROUTE_SOFTMAX)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        n_in_graph = 32
        with torch.cuda.graph(graph):
            for _ in range(n_in_graph):
                step()
        ms = time_region(graph.replay, 20, 3)
    # the 512 steps as one call, their inputs known up front (teacher forcing,
    # speculative verification, this workload's pre-drawn steps): MoC.forward
    # continuing from the prompt's cache, one router and one prefill launch
    with torch.no_grad():
        xw = xs[:, :, 0].transpose(0, 1).contiguous()
        zw = zs[:, :, 0].transpose(0, 1).contiguous()
        c0 = cache.clone()
        one_call = lambda: m(xw, zw, cache=c0, output_final_state=True)  # noqa: E731
        loop_ms = time_region(one_call, 5, 2)
        del xw, zw
    # x, y, cache slots read (S-1) and written (S), z, router, basis
    kbytes = (c["B"] * c["D"] * 2 * (1 + 1 + (c["S"] - 1) + c["S"]) + c["B"] * c["Z"] * 2
              + c["K"] * c["Z"] * 2 + c["K"] * c["S"] * c["D"] * 2)
    kernel_us = ms * 1e3 / n_in_graph
    return dict(B=c["B"], D=c["D"], K=c["K"], S=c["S"], prompt=c["prompt"], steps=c["steps"],
                step_us_median=round(statistics.median(per_step), 2),
                step_us_p10=round(sorted(per_step)[len(per_step) // 10], 2),
                step_us_async=round(async_us, 2),
                step_us_graph=round(module_graph_us, 2),
                steps_in_one_call_us_per_step=round(loop_ms * 1e3 / c["steps"], 3),
                kernel_us=round(kernel_us, 3),
                kernel_GBps=round(kbytes / (kernel_us * 1e-6) / 1e9, 1),
                kernel_roofline_us=round(kbytes / HBM_PEAK * 1e6, 3),
                update_us=bench_update(dev))


def cpu_baseline(seconds):
    """The CPU oracle (oracle/moc_oracle.py) on a bounded slice of the headline
    workload: one sequence of 2048 tokens at D=Z=2048, K=16, S=4, fp32, layer
    forward + backward (router GEMM + softmax + MoC), all host cores."""
    from oracle import moc_oracle as O
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    T = 2048
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, T, CFG["D"], generator=g).requires_grad_()
    z = torch.randn(1, T, CFG["Z"], generator=g).requires_grad_()
    router = (torch.randn(CFG["K"], CFG["Z"], generator=g) * 0.02).requires_grad_()
    basis = ((torch.rand(CFG["K"], CFG["S"], CFG["D"], generator=g) * 2 - 1)
             * 0.002 * 3 ** 0.5).requires_grad_()

    def step():
        for t in (x, z, router, basis):
            t.grad = None
        a = O.route(torch.nn.functional.linear(z, router), "softmax")
        O.moc_ref(x, a, basis, "silu").sum().backward()

    step()
    reps, t0 = 0, time.perf_counter()
    while True:
        step()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= 2:
            break
    tok_s = reps * T / el
    return {"value": round(tok_s / 1e6, 5), "unit": "Mtok/s", "cores": cores, "kind": "port",
            "sample": f"CPU oracle, layer fwd+bwd on B=1 T={T} D={CFG['D']} Z={CFG['Z']} "
                      f"K={CFG['K']} S={CFG['S']} fp32, {reps} reps in {el:.1f}s",
            "configs0_forward": cpu_configs0_forward(min(seconds, 5.0))}


def cpu_configs0_forward(seconds):
    """BASELINE configs[0] on the CPU oracle: the reference's CPU-runnable
    forward (B=2, T=512, D=256, z_dim=256, K=4, S=4, fp32; x, z ~ N(0,1) seed 0,
    router ~ N(0, 0.02), basis ~ N(0, 0.002), softmax routing, no SiLU)."""
    from oracle import moc_oracle as O
    B, T, D, Z, K, S = 2, 512, 256, 256, 4, 4
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, T, D, generator=g)
    z = torch.randn(B, T, Z, generator=g)
    router = torch.randn(K, Z, generator=g) * 0.02
    basis = torch.randn(K, S, D, generator=g) * 0.002

    def fwd():
        return O.moc_ref(x, O.route(torch.nn.functional.linear(z, router), "softmax"), basis, None)

    with torch.no_grad():
        fwd()
        reps, t0 = 0, time.perf_counter()
        while True:
            fwd()
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds and reps >= 2:
                break
    return {"value": round(reps * B * T / el / 1e6, 5), "unit": "Mtok/s",
            "ms_per_call": round(el / reps * 1e3, 3),
            "sample": f"CPU oracle forward (router + softmax + MoC) at configs[0], {reps} reps in {el:.1f}s"}


def config3_step(dev):
    """(step, total tokens, number of sequences): the configs[2] layer step,
    packed varlen fwd+bwd, 32768 tokens in sequences of lengths uniform in
    [16, 4096] (seeded, cu_seqlens int32), D=4096, z_dim=2048, K=16, S=4, bf16,
    exp routing, no SiLU, dy ~ N(0, 1)."""
    import moc
    g = torch.Generator().manual_seed(0)
    total, lengths = 32768, []
    while sum(lengths) < total:
        lengths.append(int(torch.randint(16, 4097, (1,), generator=g)))
    lengths[-1] -= sum(lengths) - total
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32).to(dev)
    D, Z, K, S = 4096, 2048, 16, 4
    m = moc.MoC(D, Z, S, K, init_std=0.002, router_activation="exp")
    with torch.no_grad():
        m.router.copy_(torch.randn(K, Z, generator=g) * 0.02)
    m = m.to(dev, torch.bfloat16)
    x = torch.randn(total, D, generator=g).to(dev, torch.bfloat16).requires_grad_()
    z = torch.randn(total, Z, generator=g).to(dev, torch.bfloat16).requires_grad_()
    dy = torch.randn(total, D, generator=g).to(dev, torch.bfloat16)

    def step():
        m.zero_grad(set_to_none=True)
        x.grad = None
        z.grad = None
        y, _ = m(x, z, cu_seqlens=cu, max_seqlen=max(lengths))
        y.backward(dy)

    return step, total, len(lengths)


def bench_config3(dev, steps, warmup):
    """the varlen layer step of config3_step."""
    step, total, n_seqs = config3_step(dev)
    D, Z, K, S = 4096, 2048, 16, 4
    ms = time_region(step, steps, warmup)
    return {"metric": "configs[2] varlen layer fwd+bwd Mtok/s", "value": round(total / (ms * 1e-3) / 1e6, 3),
            "unit": "Mtok/s", "ms_per_step": round(ms, 4), "n_seqs": n_seqs,
            "config": {"workload": "MoC layer fwd+bwd, BASELINE configs[2]", "tokens": total, "D": D,
                       "z_dim": Z, "K": K, "S": S, "routing": "exp", "activation": None}}


def config5_step(dev):
    """(step(grouped) -> callable, B, T, Dm): the configs[4] QKV triple step,
    three MoC layers (q 4096, k 1024, v 1024 channels) on one routing input
    x_norm [2, 8192, 4096], K=32, S=8, bf16, exp routing for q and k, softmax
    for v, no SiLU, fan-in init, loss = sum of the three y.sum(); the layers
    called one by one (grouped False) or as one MoCGroup."""
    import moc
    g = torch.Generator().manual_seed(0)
    torch.manual_seed(0)
    B, T, Dm = 2, 8192, 4096
    layers = []
    for dim, route in ((4096, "exp"), (1024, "exp"), (1024, "softmax")):
        m = moc.MoC(dim, Dm, 8, 32, router_activation=route)
        with torch.no_grad():
            m.router.copy_(torch.randn(32, Dm, generator=g) * 0.02)
        layers.append(m.to(dev, torch.bfloat16))
    xn = torch.randn(B, T, Dm, generator=g).to(dev, torch.bfloat16).requires_grad_()
    vs = [torch.randn(B, T, m.dim, generator=g).to(dev, torch.bfloat16).requires_grad_()
          for m in layers]
    grp = moc.MoCGroup(*layers)

    def step(grouped):
        def run():
            for m in layers:
                m.zero_grad(set_to_none=True)
            for v in vs:
                v.grad = None
            xn.grad = None
            outs = grp(vs, xn) if grouped else [m(v, xn) for m, v in zip(layers, vs)]
            sum(y.sum() for y, _ in outs).backward()
        return run

    return step, B, T, Dm


def bench_config5(dev, steps, warmup):
    """the QKV triple step (config5_step), the layers one by one and
    as one MoCGroup."""
    step, B, T, Dm = config5_step(dev)
    ms_sep = time_region(step(False), steps, warmup)
    ms_grp = time_region(step(True), steps, warmup)
    return {"metric": "configs[4] QKV triple fwd+bwd Mtok/s (MoCGroup)",
            "value": round(B * T / (ms_grp * 1e-3) / 1e6, 3), "unit": "Mtok/s",
            "ms_per_step": round(ms_grp, 4), "ms_per_step_separate_layers": round(ms_sep, 4),
            "config": {"workload": "QKV triple, BASELINE configs[4]", "B": B, "T": T, "d_model": Dm,
                       "dims": [4096, 1024, 1024], "K": 32, "S": 8,
                       "routing": ["exp", "exp", "softmax"], "activation": None}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the configs[2] / configs[4] objects of the default line")
    ap.add_argument("--config", type=int, choices=(2, 3, 5), default=2,
                    help="2: the headline line (default); 3 / 5: one JSON line for BASELINE "
                         "configs[2] (varlen) / configs[4] (QKV triple) instead")
    ap.add_argument("--rotate", type=int, default=ROTATE,
                    help="input sets the timed loops cycle through (1: one set reused, "
                         "which the last-level cache partly holds across steps)")
    ap.add_argument("--counters", choices=("fwd", "bwd", "step", "decode", "update", "shapes", "c3", "c5",
                                           "prefill", "copy"),
                    default=None,
                    help="only run --reps calls of one workload (see counter_run) for a "
                         "rocprofv3 --pmc or --kernel-trace pass; prints no JSON")
    ap.add_argument("--reps", type=int, default=3, help="calls of the --counters workload")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.counters:
        counter_run(dev, args.counters, args.reps)
        return
    if args.config != 2:
        fn = bench_config3 if args.config == 3 else bench_config5
        out = fn(dev, min(args.steps, 20), min(args.warmup, 5))
        out.update({"n_gpus": 1, "dtype": "bf16", "data": "synthetic (seeded)"})
        print(json.dumps(out), flush=True)
        return
    N = CFG["B"] * CFG["T"]
    D, K, S = CFG["D"], CFG["K"], CFG["S"]

    ms = bench_layer(dev, args.steps, args.warmup, args.rotate)
    t_fwd, t_bwd, k_fwd, k_bwd = bench_entries(dev, args.steps, args.warmup, args.rotate)
    fb, bb = bytes_fwd(N, D, K, S), bytes_bwd(N, D, K, S)
    roof_us = (max(fb / HBM_PEAK, flops_fwd(N, D, K, S) / 2.5e15)
               + max(bb / HBM_PEAK, flops_bwd(N, D, K, S) / 2.5e15)) * 1e6
    # dominant kernel: the fused backward stage 1; its algorithmic bytes are x, dy
    # and dx, the routing weights and the basis (dalpha / dbasis leave it as
    # partial sums that the stage-2 reduction turns into the outputs)
    kb = 3 * N * D * 2 + N * K * 2 + K * S * D * 2
    achieved = kb / (k_bwd * 1e-3)
    out = {
        "metric": METRIC,
        "value": round(N / (ms * 1e-3) / 1e6, 3),
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x, z; router N(0,0.02); basis U(+-0.002*sqrt(3)))",
        "input_sets": args.rotate,
        "config": {"workload": "MoC layer fwd+bwd, BASELINE configs[1]", "B": CFG["B"],
                   "T": CFG["T"], "D": D, "z_dim": CFG["Z"], "K": K, "S": S,
                   "activation": "silu", "routing": "softmax", "loss": "y.sum()"},
        "roofline": {"bound": "hbm", "kernel": "moc::mfma::bwd_lean_kernel (fused backward stage 1)",
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": TRAFFIC_BWD, "algorithmic_bytes": kb,
                     "kernel_us": round(k_bwd * 1e3, 2)},
        "kernel_scope": {"fwd_us": round(t_fwd * 1e3, 2), "bwd_us": round(t_bwd * 1e3, 2),
                         "fwd_kernel_us": round(k_fwd * 1e3, 2),
                         "fwd_kernel_GBps": round(fb / (k_fwd * 1e-3) / 1e9, 1),
                         "mtok_s": round(N / ((t_fwd + t_bwd) * 1e-3) / 1e6, 3),
                         "fwd_GBps": round(fb / (t_fwd * 1e-3) / 1e9, 1),
                         "bwd_GBps": round(bb / (t_bwd * 1e-3) / 1e9, 1),
                         "hbm_roofline_us": round(roof_us, 2),
                         "roofline_frac": round(roof_us / ((t_fwd + t_bwd) * 1e3), 4)},
    }
    if not args.no_prefill:
        out["prefill"] = bench_prefill(dev, min(args.steps, 20), min(args.warmup, 5), args.rotate)
    if not args.no_decode:
        out["decode"] = bench_decode(dev)
    if not args.no_configs:
        out["shapes"] = bench_shapes(dev, min(args.steps, 20), min(args.warmup, 5))
    if not args.no_configs:
        # BASELINE configs[2] (varlen) and configs[4] (QKV triple), as the
        # `--config 3` / `--config 5` lines report them
        for key, fn in (("config3_varlen", bench_config3), ("config5_qkv", bench_config5)):
            r = fn(dev, min(args.steps, 20), min(args.warmup, 5))
            out[key] = {k: r[k] for k in r if k not in ("metric",)}
            torch.cuda.empty_cache()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
