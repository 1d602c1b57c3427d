"""GPU parity at the BASELINE.json configurations.

At these sizes the oracle (oracle/moc_oracle.py, plain torch) runs in fp32 on
the GPU itself; it is the same restatement the CPU tests pin.  Every HIP result
is also compared with the other kernel family (MFMA vs generic VALU kernels,
selected with moc_set_kernel_path), and the decode loop is checked against the full
forward with the cache compared bit for bit.  Tolerances: tests/_parity.py.
"""
from __future__ import annotations

import itertools

import pytest
import torch

import moc
from moc import MoC, _lib, moc_triton
from oracle import moc_oracle as O
from tests._parity import assert_close, gen, randn, ulp_allowance

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(D, Z, K, S, act, route, init_std, dtype, seed=0):
    torch.manual_seed(seed)
    m = MoC(D, Z, S, K, activation=act, init_std=init_std, router_activation=route)
    g = gen(seed + 1)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.02))
    return m.to(DEV, dtype), g


def _oracle_layer(m, x, z, dy, route, act, cu=None):
    """The layer with the MoC op replaced by the fp32 oracle.  The logits are
    the module's own router GEMM (moc.router_linear, on the GPU), so the
    oracle and the module route identically; the router activation is rounded
    to the logits' dtype with torch's gradient rule; dz and drouter are fp32
    products of the oracle's d(logits) rounded to the logits' dtype, the value
    the module's router backward consumes.  Returns y and the gradients of x,
    z, router, basis."""
    with torch.no_grad():
        logits = moc.router_linear(z, m.router)
    lf = logits.float().requires_grad_()
    rx = x.detach().float().requires_grad_()
    rb = m.conv_bases.detach().float().requires_grad_()
    alpha = O.route(lf, route, out_dtype=logits.dtype)
    if cu is None:
        y = O.moc_ref(rx, alpha, rb, act)
    else:
        y = O.moc_varlen_ref(rx, alpha, rb, cu, act)
    y.backward(dy.float())
    dl = lf.grad
    _oracle_layer.last_dlogits = dl
    K, Z = m.router.shape
    dlr = dl.to(logits.dtype).float().reshape(-1, K)
    dz = (dlr @ m.router.detach().float()).reshape(z.shape)
    drouter = dlr.T @ z.detach().float().reshape(-1, Z)
    return y.detach(), rx.grad, dz, drouter, rb.grad


def _check_layer(label, m, got, ref, dtype):
    """y, dx, dz, drouter, dbasis; dz may differ by one bf16 ulp of the logits'
    gradient propagated through the router (both sides round it to bf16)."""
    extra = None
    if dtype == torch.bfloat16:
        extra = ulp_allowance(_oracle_layer.last_dlogits, m.router)
    for n, a, b in zip(NAMES, got, ref):
        assert_close(f"{n} {label}".strip(), a, b, dtype, extra=extra if n == "dz" else None)


def _hip_layer(m, x, z, dy, **kw):
    """The layer's forward and backward on the HIP path; dy None: loss = y.sum()
    (autograd hands the backward one element expanded over y, the form the
    kernels read in place, row stride -1)."""
    m.zero_grad(set_to_none=True)
    x = x.detach().requires_grad_()
    z = z.detach().requires_grad_()
    y, _ = m(x, z, **kw)
    if dy is None:
        y.sum().backward()
    else:
        y.backward(dy)
    return y.detach(), x.grad, z.grad, m.router.grad.clone(), m.conv_bases.grad.clone()


def _with_path(path, fn):
    """fn() on the generic kernels (path "generic") through the library's
    kernel-family switch."""
    assert path == "generic"
    with _lib.kernel_path(_lib.PATH_GENERIC):
        return fn()


NAMES = ("y", "dx", "dz", "drouter", "dbasis")


def test_config1_cpu_reference_shape_fp32():
    """B2 T512 D256 Z256 K4 S4 fp32, softmax, no SiLU (oracle on CPU)."""
    m, g = _layer(256, 256, 4, 4, None, "softmax", None, torch.float32)
    with torch.no_grad():
        m.conv_bases.copy_(randn(g, 4, 4, 256, scale=0.002))
    x = randn(g, 2, 512, 256).to(DEV)
    z = randn(g, 2, 512, 256).to(DEV)
    dy = randn(g, 2, 512, 256).to(DEV)
    got = _hip_layer(m, x, z, dy)
    ref = _oracle_layer(m, x, z, dy, "softmax", None)
    _check_layer("", m, got, ref, torch.float32)


def test_config2_headline_layer():
    """B4 T4096 D2048 Z2048 K16 S4 bf16, softmax, SiLU, loss = y.sum()."""
    m, g = _layer(2048, 2048, 16, 4, "silu", "softmax", 0.002, torch.bfloat16)
    x = randn(g, 4, 4096, 2048).to(DEV, torch.bfloat16)
    z = randn(g, 4, 4096, 2048).to(DEV, torch.bfloat16)
    dy = torch.ones_like(x)
    got = _hip_layer(m, x, z, dy)
    ref = _oracle_layer(m, x, z, dy, "softmax", "silu")
    _check_layer("", m, got, ref, torch.bfloat16)
    # the same loss as y.sum(): the one-element gradient the bench's step runs
    summed = _hip_layer(m, x, z, None)
    _check_layer("(y.sum())", m, summed, ref, torch.bfloat16)
    other = _with_path("generic", lambda: _hip_layer(m, x, z, dy))
    _check_layer("(mfma vs generic)", m, got, other, torch.bfloat16)


def _varlen_lengths(total, lo, hi, seed=0):
    g = gen(seed)
    lengths = []
    while sum(lengths) < total:
        lengths.append(int(torch.randint(lo, hi + 1, (1,), generator=g)))
    lengths[-1] -= sum(lengths) - total
    return [n for n in lengths if n > 0]


def test_config3_varlen_layer():
    """32768 packed tokens, lengths U[16, 4096], D4096 Z2048 K16 S4 bf16, exp."""
    lengths = _varlen_lengths(32768, 16, 4096)
    cu = torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32, device=DEV)
    m, g = _layer(4096, 2048, 16, 4, None, "exp", 0.002, torch.bfloat16)
    x = randn(g, 32768, 4096).to(DEV, torch.bfloat16)
    z = randn(g, 32768, 2048).to(DEV, torch.bfloat16)
    dy = randn(g, 32768, 4096).to(DEV, torch.bfloat16)
    kw = dict(cu_seqlens=cu, max_seqlen=max(lengths))
    got = _hip_layer(m, x, z, dy, **kw)
    ref = _oracle_layer(m, x, z, dy, "exp", None, cu=cu)
    _check_layer("", m, got, ref, torch.bfloat16)


def test_config5_qkv_triple():
    """configs[4] at its stated size: q / k / v MoC layers (4096 / 1024 / 1024
    channels) routed by one x_norm [2, 8192, 4096] through MoCGroup (the path
    bench.py --config 5 times), K32 S8, fan-in init, exp routing for q and k,
    softmax for v, no SiLU, loss = sum of the three y.sum().  Each layer's y,
    dx, drouter and dbasis against the fp32 oracle layer; dz (one router
    backward over the three layers' logits gradients) against the sum of the
    three oracle router gradients."""
    B, T, Dm = 2, 8192, 4096
    specs = ((4096, "exp"), (1024, "exp"), (1024, "softmax"))
    g = gen(7)
    xn = randn(g, B, T, Dm).to(DEV, torch.bfloat16)
    layers, vs = [], []
    for dim, route in specs:
        m, g2 = _layer(dim, Dm, 32, 8, None, route, None, torch.bfloat16, seed=dim)
        layers.append(m)
        vs.append(randn(g2, B, T, dim).to(DEV, torch.bfloat16))
    grp = moc.MoCGroup(*layers)
    assert grp._grouped(vs, xn, None)
    xs = [v.detach().requires_grad_() for v in vs]
    z = xn.detach().requires_grad_()
    outs = grp(xs, z)
    sum(y.sum() for y, _ in outs).backward()
    dz_ref = torch.zeros(B, T, Dm, device=DEV)
    extra = torch.zeros(B, T, Dm, device=DEV)
    for m, v, xg, (y, _), (dim, route) in zip(layers, vs, xs, outs, specs):
        ref = _oracle_layer(m, v, xn, torch.ones_like(v), route, None)
        got = (y.detach(), xg.grad, None, m.router.grad, m.conv_bases.grad)
        for n, a, b in zip(NAMES, got, ref):
            if n != "dz":
                assert_close(f"{n} ({dim}, {route})", a, b, torch.bfloat16)
        dz_ref += ref[2]
        extra += ulp_allowance(_oracle_layer.last_dlogits, m.router)
        del ref
    assert_close("dz (group)", z.grad, dz_ref, torch.bfloat16, extra=extra)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S,K,act", [(2, 8, "silu"), (3, 16, "silu"), (4, 16, "silu"), (4, 32, "silu"),
                                     (5, 16, "silu"), (5, 32, None), (6, 16, None), (6, 32, "silu"),
                                     (7, 12, None), (7, 32, "silu"),
                                     (8, 32, "silu"), (8, 32, None), (8, 5, "silu"),
                                     (6, 32, None), (8, 16, None), (7, 32, None), (7, 16, None),
                                     (4, 32, None), (5, 32, "silu"), (8, 16, "silu"), (7, 16, "silu"),
                                     (4, 64, None), (5, 48, None), (6, 64, "silu"), (3, 48, "silu"),
                                     (4, 64, "silu"), (2, 48, None), (8, 64, None),
                                     (2, 32, None), (3, 24, "silu")])
def test_mfma_matches_generic(dtype, S, K, act):
    """Mid-size problems through both kernel families, fixed and packed, for
    every kernel size the matrix-core kernels are built for (2-8; bf16 without
    activation at 4-8 taps and 32 routes, 7-8 taps and 16 routes, and with SiLU
    at 5-8 taps and 32 routes, 8 taps and 16 routes: the two-pass backward,
    odd kernel sizes with a missing last tap in the second half; 64 routes
    without activation: the two passes with the taps pass in route halves)."""
    _mfma_vs_generic(dtype, S, K, act, 192)


@pytest.mark.parametrize("dtype,S,K,act", [
    (torch.bfloat16, 4, 16, "silu"),   # the four-wave fused pass
    (torch.bfloat16, 3, 16, None),     # fused pass
    (torch.bfloat16, 8, 32, None),     # two passes
    (torch.bfloat16, 8, 32, "silu"),   # two passes, g through the workspace
    (torch.bfloat16, 4, 64, None),     # taps pass in route halves
    (torch.bfloat16, 3, 32, "silu"),   # fused pass split in route chunks
    (torch.bfloat16, 6, 48, "silu"),   # 64-route two passes, g through the workspace
    (torch.float32, 4, 16, "silu"),
    (torch.float32, 7, 32, None),
    (torch.float32, 12, 16, "silu"),   # fp32 two passes, g through the workspace
    (torch.float32, 15, 16, None),     # fp32 two passes
])
@pytest.mark.parametrize("D", [198, 130])
def test_mfma_even_channel_tails(dtype, S, K, act, D):
    """Channel counts that are even but not a multiple of 4 (the last 16-lane
    column of a wave holds a partial group of channel pairs) run on the
    matrix-core kernels, against the oracle and the generic kernels."""
    for bwd in (0, 1):
        assert _lib.lib().moc_matrix_core_supported(3 * 333, D, K, S, _lib.dtype_code(dtype), bwd) == 1
    _mfma_vs_generic(dtype, S, K, act, D)


@pytest.mark.parametrize("dtype,S,K,act,bwd", [
    (torch.bfloat16, 9, 16, "silu", 1),
    (torch.bfloat16, 12, 8, None, 1),
    (torch.bfloat16, 13, 16, None, 1),
    (torch.bfloat16, 16, 16, "silu", 1),
    (torch.bfloat16, 16, 12, None, 1),
    (torch.bfloat16, 10, 32, "silu", 1),    # past 16 routes: dx pass, then taps per 16-route chunk
    (torch.bfloat16, 16, 64, None, 1),
    (torch.bfloat16, 12, 24, "silu", 1),
    (torch.bfloat16, 13, 48, None, 1),
    (torch.float32, 11, 16, None, 1),       # fp32 up to 16 routes: the two-pass form
    (torch.float32, 9, 16, "silu", 1),
    (torch.float32, 14, 12, "silu", 1),
    (torch.float32, 16, 16, None, 1),
    (torch.float32, 13, 8, "silu", 1),
    (torch.float32, 16, 32, "silu", 1),     # fp32 past 16 routes: parts of 16 routes
    (torch.float32, 10, 20, None, 1),
    (torch.float32, 12, 48, "silu", 1),     # and the forward in halves of 32 routes
    (torch.float32, 9, 64, None, 1),
    (torch.float32, 15, 40, "silu", 1),
    (torch.float32, 4, 48, "silu", 1),      # fp32, 33-64 routes: the backward in route halves
    (torch.float32, 8, 64, None, 1),
    (torch.float32, 3, 40, "silu", 1),
])
def test_mfma_long_kernels(dtype, S, K, act, bwd):
    """9 to 16 taps: the forward on the matrix cores for every route count, the
    backward up to 16 routes in its two-pass form (bf16 and fp32), for bf16
    past 16 routes the dx pass over every route, then the taps pass per
    16-route chunk, for fp32 past 16 routes in parts of 16 routes (dy = g from
    P, the router gradient over all routes at the end), with P and the forward
    past 32 routes as the sum of two 32-route forwards; fp32 with 33-64 routes
    up to 8 taps: the forward on the matrix cores, the backward in two route
    halves on the 32-route kernels.  Against the oracle and the generic
    kernels."""
    L = _lib.lib()
    assert L.moc_matrix_core_supported(3 * 333, 192, K, S, _lib.dtype_code(dtype), 0) == 1
    assert L.moc_matrix_core_supported(3 * 333, 192, K, S, _lib.dtype_code(dtype), 1) == bwd
    _mfma_vs_generic(dtype, S, K, act, 192)


@pytest.mark.parametrize("dtype,S,K,act,D", [
    (torch.bfloat16, 4, 16, "silu", 197),    # the lean fused pass
    (torch.bfloat16, 8, 32, None, 129),      # two passes
    (torch.float32, 6, 24, "silu", 65),
    (torch.bfloat16, 12, 16, None, 131),     # 12 taps
    (torch.bfloat16, 3, 64, "silu", 191),    # 64 routes
    (torch.float32, 12, 48, "silu", 197),    # fp32 route parts and forward halves
    (torch.bfloat16, 12, 32, "silu", 131),   # bf16 route chunks past 8 taps
])
def test_odd_channel_counts_padded(dtype, S, K, act, D):
    """Odd channel counts run the matrix-core kernels on a copy padded with a
    zero channel, against the oracle and the generic kernels, fixed and packed."""
    L = _lib.lib()
    for bwd in (0, 1):
        assert L.moc_matrix_core_supported(3 * 333, D, K, S, _lib.dtype_code(dtype), bwd) == 1
    _mfma_vs_generic(dtype, S, K, act, D)


@pytest.mark.parametrize("S,K,dtype,act,D", [
    (4, 16, torch.bfloat16, "silu", 65),     # padded copy
    (8, 32, torch.bfloat16, None, 3),        # padded copy, two passes
    (12, 32, torch.float32, "silu", 66),     # route parts of 16
    (12, 48, torch.float32, None, 130),      # route parts, forward in halves
    (6, 64, torch.float32, "silu", 4),       # route halves of 32
])
@pytest.mark.parametrize("B,T", [(1, 1), (1, 2), (2, 3), (1, 17), (3, 40)])
def test_parts_and_padding_small(S, K, dtype, act, D, B, T):
    """The padded and route-part forms at token counts below one super-block
    and small channel counts, forward and backward against the oracle."""
    L = _lib.lib()
    assert L.moc_matrix_core_supported(B * T, D, K, S, _lib.dtype_code(dtype), 1) == 1
    g = gen(S * 1000 + K * 10 + T + D)
    x = randn(g, B, T, D, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, B, T, K), -1).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.2).to(DEV, dtype)
    dy = randn(g, B, T, D).to(DEV, dtype)
    xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
    y, _ = moc_triton(xx, aa, bb, activation=act)
    y.backward(dy)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), act)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), (y, xx.grad, aa.grad, bb.grad), ref):
        assert_close(n, u, r, dtype)


@pytest.mark.parametrize("D,K,S,dtype,act", [
    (1, 1, 2, torch.bfloat16, "silu"),     # one channel (padded to 2), one route
    (2, 2, 3, torch.bfloat16, None),
    (3, 5, 2, torch.float32, "silu"),
    (2, 1, 16, torch.float32, None),       # 16 taps, two passes
    (5, 33, 4, torch.bfloat16, "silu"),    # 33 routes padded to 64
    (4, 17, 9, torch.float32, "silu"),     # fp32 route parts past 8 taps
])
def test_tiny_shapes(D, K, S, dtype, act):
    """The smallest channel and route counts on the matrix-core paths (padded
    copies, padded routes, route parts), fixed and packed, against the oracle."""
    L = _lib.lib()
    assert L.moc_matrix_core_supported(2 * 37, D, K, S, _lib.dtype_code(dtype), 1) == 1
    _mfma_vs_generic(dtype, S, K, act, D, Bt=2, T=37, lengths=(1, 2, 30, 4, 37))


@pytest.mark.parametrize("form", ["element", "row", "full"])
@pytest.mark.parametrize("S,K,act", [(12, 48, 0), (4, 64, 0), (12, 32, 1)])
def test_route_parts_broadcast_dy(form, S, K, act):
    """The fp32 route-part backward with the dy of y.sum() (one element), one dy
    row for every token and full rows: without the activation the parts read
    dy as it is; with it g = dy silu'(P) comes first.  Against the oracle."""
    from moc import ops
    g = gen(S * 100 + K)
    D = 128
    x = randn(g, 2, 150, D, scale=0.5).to(DEV, torch.float32)
    a = torch.softmax(randn(g, 2, 150, K), -1).to(DEV, torch.float32)
    b = randn(g, K, S, D, scale=0.2).to(DEV, torch.float32)
    if form == "element":
        dy = torch.ones((), device=DEV, dtype=torch.float32).expand(2, 150, D)
    elif form == "row":
        dy = randn(g, D).to(DEV, torch.float32).expand(2, 150, D)
    else:
        dy = randn(g, 2, 150, D).to(DEV, torch.float32)
    got = ops.launch_backward(x, a, b, dy, activation_flag=act, need_x=True)
    rx, ra, rb = O.reference_inputs(x, a, b, torch.float32)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu().contiguous(), "silu" if act else None)
    for n, u, r in zip(("dx", "dalpha", "dbasis"), got, ref[1:]):
        assert_close(n, u, r, torch.float32)


@pytest.mark.parametrize("form", ["element", "row"])
def test_odd_channel_count_broadcast_dy(form):
    """The padded backward with the dy of y.sum() (one element) and with one
    dy row for every token, against the oracle."""
    from moc import ops
    g = gen(7)
    D, K, S = 197, 16, 4
    x = randn(g, 2, 150, D, scale=0.5).to(DEV, torch.bfloat16)
    a = torch.softmax(randn(g, 2, 150, K), -1).to(DEV, torch.bfloat16)
    b = randn(g, K, S, D, scale=0.2).to(DEV, torch.bfloat16)
    if form == "element":
        dy = torch.ones((), device=DEV, dtype=torch.bfloat16).expand(2, 150, D)
    else:
        dy = randn(g, D).to(DEV, torch.bfloat16).expand(2, 150, D)
    got = ops.launch_backward(x, a, b, dy, activation_flag=1, need_x=True)
    rx, ra, rb = O.reference_inputs(x, a, b, torch.bfloat16)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu().contiguous(), "silu")
    for n, u, r in zip(("dx", "dalpha", "dbasis"), got, ref[1:]):
        assert_close(n, u, r, torch.bfloat16)


@pytest.mark.parametrize("dtype,S,K,act,D", [
    (torch.bfloat16, 17, 16, "silu", 192),   # past 16 taps
    (torch.bfloat16, 4, 80, None, 192),      # past 64 routes
    (torch.float32, 17, 8, "silu", 197),     # past 16 taps, odd channel count
])
def test_generic_path_matches_oracle(dtype, S, K, act, D):
    """The shapes outside the matrix-core kernels (forward and backward) run
    the generic kernels, against the oracle, fixed and packed."""
    L = _lib.lib()
    for bwd in (0, 1):
        assert L.moc_matrix_core_supported(3 * 333, D, K, S, _lib.dtype_code(dtype), bwd) == 0
    _mfma_vs_generic(dtype, S, K, act, D)


def _mfma_vs_generic(dtype, S, K, act, D, Bt=3, T=333, lengths=(1, 2, 70, 3, 200, 17, 400, 5, 301)):
    g = gen(S * 100 + K)
    x = randn(g, Bt, T, D, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, Bt, T, K), -1).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.2).to(DEV, dtype)
    dy = randn(g, Bt, T, D).to(DEV, dtype)

    def run(**kw):
        xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
        if "cu_seqlens" in kw:
            y, _ = moc_triton(xx.view(-1, D), aa.view(-1, K), bb, activation=act, **kw)
            y.backward(dy.view(-1, D))
        else:
            y, _ = moc_triton(xx, aa, bb, activation=act)
            y.backward(dy)
        return y.detach().reshape(x.shape), xx.grad, aa.grad, bb.grad

    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), act)
    got = run()
    other = _with_path("generic", run)
    for n, u, v, r in zip(("y", "dx", "dalpha", "dbasis"), got, other, ref):
        assert_close(n, u, r, dtype)
        assert_close(n + " (mfma vs generic)", u, v, dtype)
    cu = torch.tensor([0, *itertools.accumulate(lengths)], device=DEV, dtype=torch.int64)
    assert cu[-1] == Bt * T
    gv = run(cu_seqlens=cu, max_seqlen=max(lengths))
    refv = O.moc_varlen_grads_ref(rx.detach().view(-1, D), ra.detach().view(-1, K), rb.detach(),
                                  cu.cpu(), dy.float().cpu().view(-1, D), act)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), gv, refv):
        assert_close("varlen " + n, u.reshape(r.shape), r, dtype)


@pytest.mark.parametrize("form", ["rows", "element"])
@pytest.mark.parametrize("S,K,dtype", [(8, 32, torch.bfloat16), (8, 16, torch.bfloat16),
                                       (12, 16, torch.float32)])
def test_two_pass_silu_without_dx(form, S, K, dtype):
    """With SiLU the two-pass backward's dx pass also forms g for the taps pass:
    without dx (need_x false) dalpha and dbasis are those of the call with dx,
    bit for bit, for a full dy and for the one-element dy of y.sum()."""
    from moc import ops
    g = gen(S * 10 + K)
    x = randn(g, 2, 150, 192, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, 2, 150, K), -1).to(DEV, dtype)
    b = randn(g, K, S, 192, scale=0.2).to(DEV, dtype)
    if form == "rows":
        dy = randn(g, 2, 150, 192).to(DEV, dtype)
    else:
        dy = torch.ones((), device=DEV, dtype=dtype).expand(2, 150, 192)
    with_dx = ops.launch_backward(x, a, b, dy, activation_flag=1, need_x=True)
    no_dx = ops.launch_backward(x, a, b, dy, activation_flag=1, need_x=False)
    assert no_dx[0] is None
    assert torch.equal(with_dx[1], no_dx[1]) and torch.equal(with_dx[2], no_dx[2])
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu().expand(2, 150, 192).contiguous(), "silu")
    for n, u, r in zip(("dx", "dalpha", "dbasis"), with_dx, ref[1:]):
        assert_close(n, u, r, dtype)


@pytest.mark.parametrize("S,K,dtype", [(5, 32, torch.bfloat16), (7, 32, torch.bfloat16),
                                       (8, 16, torch.bfloat16), (7, 16, torch.bfloat16),
                                       (12, 16, torch.float32), (9, 8, torch.float32)])
@pytest.mark.parametrize("B,T,D", [(1, 1, 64), (1, 2, 4), (2, 3, 132), (1, 17, 260), (3, 40, 68)])
def test_two_pass_small_and_ragged(S, K, dtype, B, T, D):
    """The two-pass backward (no activation; bf16, and fp32 past 8 taps) at
    token counts below one super-block and channel counts that leave partial
    channel groups, against the oracle."""
    g = gen(S * 1000 + K * 10 + T)
    x = randn(g, B, T, D, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, B, T, K), -1).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.2).to(DEV, dtype)
    dy = randn(g, B, T, D).to(DEV, dtype)
    xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
    y, _ = moc_triton(xx, aa, bb)
    y.backward(dy)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), None)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), (y, xx.grad, aa.grad, bb.grad), ref):
        assert_close(n, u, r, dtype)


@pytest.mark.parametrize("S,K", [(2, 8), (3, 16), (4, 16), (4, 20), (8, 32), (8, 5), (5, 16), (6, 24),
                                 (7, 32), (4, 48), (8, 64), (9, 16), (12, 32), (13, 8), (16, 64)])
@pytest.mark.parametrize("route", [None, "softmax", "exp"])
@pytest.mark.parametrize("D", [196, 198])
def test_decode_kernel_matches_oracle_and_generic(S, K, route, D):
    """Decode steps through the matrix-core kernel and the generic kernel: y
    against the oracle step (routing weights formed from the same logits),
    caches bit-exact and identical between the two."""
    g = gen(S * 1000 + K)
    Bt, steps = 37, 5                              # ragged batch and channel counts
    x = randn(g, Bt, steps, D, scale=0.5).to(DEV, torch.bfloat16)
    lg = randn(g, Bt, steps, K).to(DEV, torch.bfloat16)
    b = randn(g, K, S, D, scale=0.2).to(DEV, torch.bfloat16)
    if route is None:
        lg = torch.softmax(lg.float(), -1).to(torch.bfloat16)
    start = randn(g, Bt, D, S).to(DEV, torch.bfloat16)

    def run():
        cache = start.clone()
        ys = []
        for t in range(steps):
            if route is None:
                y, _ = moc_triton(x[:, t:t + 1], lg[:, t:t + 1], b, cache=cache, activation="silu")
            else:
                y = moc.ops.launch_update(x[:, t], lg[:, t], b, cache, activation_flag=1,
                                          routing=moc.api._ROUTING_CODES[route])[:, None]
            ys.append(y)
        return torch.cat(ys, 1), cache

    got_y, got_c = run()
    gen_y, gen_c = _with_path("generic", run)
    assert torch.equal(got_c, gen_c)
    assert torch.equal(got_c, torch.cat((start, x.transpose(1, 2)), -1)[..., -S:])
    alpha = lg.float() if route is None else O.route(lg.float(), route, out_dtype=torch.bfloat16)
    ref = O.moc_ref(torch.cat((start.transpose(1, 2).float(), x.float()), 1),
                    alpha_pad(alpha, S), b.float().to(torch.bfloat16).float(), "silu")[:, S:]
    assert_close("decode y", got_y, ref, torch.bfloat16)
    assert_close("decode y (mfma vs generic)", got_y, gen_y, torch.bfloat16)


@pytest.mark.parametrize("S,K,route,act", [(4, 16, "softmax", "silu"), (2, 8, "exp", None),
                                              (8, 32, "softmax", None), (3, 20, "exp", "silu"),
                                              (12, 16, "softmax", "silu"), (16, 32, "exp", None)])
def test_fused_decode_step_matches_router_then_update(S, K, route, act):
    """MoC.step through the one-launch decode step (router GEMM + activation +
    update) against the router kernel followed by the update kernel: identical
    logits, so y and the cache agree bit for bit."""
    g = gen(S * 31 + K)
    Bt, D, Z = 45, 260, 192
    m = MoC(D, Z, S, K, activation=act, init_std=0.1, router_activation=route)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.05))
    m = m.to(DEV, torch.bfloat16)
    x = randn(g, Bt, 1, D).to(DEV, torch.bfloat16)
    z = randn(g, Bt, 1, Z).to(DEV, torch.bfloat16)
    start = randn(g, Bt, D, S).to(DEV, torch.bfloat16)
    c1, c2 = start.clone(), start.clone()
    assert moc.ops.decode_step_supported(x, z, m.router, m.conv_bases, c1)
    with torch.no_grad():
        y1, st = m.step(x, z, cache=c1, output_final_state=True)
        logits = moc.router_linear(z[:, 0], m.router)
        y2 = moc.ops.launch_update(x[:, 0], logits, m.conv_bases, c2,
                                   activation_flag=int(act is not None),
                                   routing=moc.api._ROUTING_CODES[route])[:, None]
    assert st is c1
    assert torch.equal(c1, c2)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("S,K,act", [(8, 64, None), (8, 48, None), (4, 64, None)])
def test_route_half_taps_pass_multi_range(S, K, act):
    """The plain backward's taps pass in route halves (bf16, 64 routes without
    activation) at a token count whose token ranges hold many super-blocks
    each (the shape sweep above runs single super-block ranges): gradients
    against the oracle."""
    g = gen(S * 7 + K)
    B, T, D = 2, 4096, 192
    x = randn(g, B, T, D, scale=0.5).to(DEV, torch.bfloat16)
    a = torch.softmax(randn(g, B, T, K), -1).to(DEV, torch.bfloat16)
    b = randn(g, K, S, D, scale=0.2).to(DEV, torch.bfloat16)
    dy = randn(g, B, T, D).to(DEV, torch.bfloat16)
    xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
    y, _ = moc_triton(xx, aa, bb, activation=act)
    y.backward(dy)
    rx, ra, rb = O.reference_inputs(x, a, b, torch.bfloat16)
    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), act)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), (y, xx.grad, aa.grad, bb.grad), ref):
        assert_close(n, u, r, torch.bfloat16)


def alpha_pad(alpha, S):
    """Routing weights for the S history rows prepended to the steps (their
    outputs are dropped, so any weights do)."""
    return torch.cat((torch.zeros_like(alpha[:, :1]).expand(-1, S, -1), alpha), 1)


@pytest.mark.parametrize("xdt,adt,bdt,layout,S,K,route", [
    (torch.float32, torch.float32, torch.float32, "contiguous", 4, 16, "softmax"),
    (torch.float32, torch.bfloat16, torch.float32, "slot-major", 8, 32, "exp"),
    (torch.float32, torch.float16, torch.float16, "contiguous", 3, 12, None),
    (torch.bfloat16, torch.bfloat16, torch.float32, "slot-major", 5, 20, "softmax"),
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, "padded", 4, 64, "softmax"),
    (torch.float32, torch.float32, torch.float32, "padded", 2, 7, "exp"),
    (torch.bfloat16, torch.bfloat16, torch.float32, "contiguous", 4, 16, "softmax"),
    (torch.bfloat16, torch.float32, torch.bfloat16, "contiguous", 6, 24, "exp"),
    (torch.float32, torch.float32, torch.float32, "contiguous", 8, 64, "softmax"),
    (torch.float32, torch.bfloat16, torch.float32, "aligned-padded", 4, 40, "softmax"),
    (torch.bfloat16, torch.bfloat16, torch.float32, "aligned-padded", 8, 16, None),
    (torch.float32, torch.float32, torch.float32, "contiguous", 9, 16, "softmax"),   # 9 to 16 taps
    (torch.bfloat16, torch.bfloat16, torch.float32, "contiguous", 12, 32, "softmax"),
    (torch.bfloat16, torch.bfloat16, torch.float32, "contiguous", 11, 16, "exp"),
    (torch.bfloat16, torch.float32, torch.bfloat16, "slot-major", 16, 64, "softmax"),
    (torch.float32, torch.float32, torch.float32, "padded", 16, 20, "exp"),
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, "aligned-padded", 14, 16, None),
    (torch.float32, torch.float32, torch.float32, "slot-major", 4, 80, "exp"),       # 80 routes, 17 taps:
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, "contiguous", 17, 8, "softmax"),  # the per-row kernel
])
def test_decode_other_dtypes_and_strided_caches(xdt, adt, bdt, layout, S, K, route):
    """Decode steps (moc_update) on what the matrix-core decode kernel does not
    take: fp32 data, mixed storage dtypes (fp16 / bf16 weights or basis), caches with any strides, a
    channel count that is not a multiple of 4, up to 64 routes and 16 taps (the
    tile kernel, with whole-row cache accesses where the rows are contiguous and
    aligned and per-slot ones otherwise), and past them (the per-row kernel).  y against the oracle
    step with the weights and basis rounded as the kernels round them; the
    cache bit-exact."""
    g = gen(S * 100 + K)
    Bt, D, steps = 37, 198, 4                      # ragged batch, D % 4 == 2
    x = randn(g, Bt, steps, D, scale=0.5).to(DEV, xdt)
    lg = randn(g, Bt, steps, K).to(DEV, adt)
    if route is None:
        lg = torch.softmax(lg.float(), -1).to(adt)
    b = randn(g, K, S, D, scale=0.2).to(DEV, bdt)
    start = randn(g, Bt, D, S).to(DEV, xdt)
    if layout == "contiguous":
        cache = start.clone()
    elif layout == "slot-major":                   # [B, D, S] view of a [B, S, D] store
        cache = start.transpose(1, 2).contiguous().transpose(1, 2)
    elif layout == "padded":                       # a window of a larger buffer
        big = torch.zeros(Bt, D + 8, S + 3, device=DEV, dtype=xdt)
        cache = big[:, 4:4 + D, 1:1 + S]
        cache.copy_(start)
    else:                                          # padded rows that keep whole-row alignment
        big = torch.zeros(Bt, D + 8, 2 * S, device=DEV, dtype=xdt)
        cache = big[:, 4:4 + D, :S]
        cache.copy_(start)
    code = _lib.ROUTE_ALPHA if route is None else moc.api._ROUTING_CODES[route]
    ys = [moc.ops.launch_update(x[:, t], lg[:, t], b, cache, activation_flag=1, routing=code)[:, None]
          for t in range(steps)]
    y = torch.cat(ys, 1)
    assert torch.equal(cache, torch.cat((start, x.transpose(1, 2)), -1)[..., -S:])
    if layout == "padded":                         # nothing outside the window written
        assert not big[:, :4].any() and not big[:, 4 + D:].any()
        assert not big[..., :1].any() and not big[..., 1 + S:].any()
    if layout == "aligned-padded":
        assert not big[:, :4].any() and not big[:, 4 + D:].any() and not big[..., S:].any()
    alpha = lg.float() if route is None else O.route(lg.float(), route, out_dtype=adt)
    alpha = alpha.to(xdt).float()
    ref = O.moc_ref(torch.cat((start.transpose(1, 2).float(), x.float()), 1).cpu(),
                    alpha_pad(alpha, S).cpu(), b.to(xdt).float().cpu(), "silu")[:, S:]
    assert_close("decode y", y, ref, xdt)


def test_config4_decode():
    """configs[3] at its stated size: a batch-256 layer (D 2048, z_dim 2048, K16,
    S4, softmax, SiLU) prefilled from a 1024-token prompt, then 512 single-token
    steps; every step's y on every batch row against the fp32 oracle forward
    over all 1536 tokens, the final cache bit-exact (the last S inputs); the
    same steps as one MoC.forward call from the prompt's cache likewise."""
    B, D, Z, K, S, P, steps = 256, 2048, 2048, 16, 4, 1024, 512
    m, _ = _layer(D, Z, K, S, "silu", "softmax", None, torch.bfloat16)
    gd = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(B, P + steps, D, generator=gd, device=DEV).to(torch.bfloat16)
    z = torch.randn(B, P + steps, Z, generator=gd, device=DEV).to(torch.bfloat16)
    y_steps = torch.empty(B, steps, D, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        _, cache = m(x[:, :P], z[:, :P], output_final_state=True)
        for i, t in enumerate(range(P, P + steps)):
            y, c2 = m.step(x[:, t:t + 1], z[:, t:t + 1], cache=cache, output_final_state=True)
            assert c2 is cache
            y_steps[:, i:i + 1] = y
    assert torch.equal(cache, x[:, -S:].transpose(1, 2))
    # the same 512 steps as one call (their inputs known up front): MoC.forward
    # continuing from the prompt's cache, i.e. one router launch and one prefill
    # launch; y against the same oracle, the final cache bit-exact
    with torch.no_grad():
        _, cache_p = m(x[:, :P], z[:, :P], output_final_state=True)
        y_call, cache_call = m(x[:, P:], z[:, P:], cache=cache_p, output_final_state=True)
    assert torch.equal(cache_call, cache)
    basis = m.conv_bases.detach().float()
    for r0 in range(0, B, 64):   # the oracle in row blocks (its W is [rows, T, D, S] fp32)
        rows = slice(r0, r0 + 64)
        with torch.no_grad():
            logits = moc.router_linear(z[rows], m.router)
            alpha = O.route(logits.float(), "softmax", out_dtype=logits.dtype)
            full = O.moc_ref(x[rows].float(), alpha, basis, "silu")
        assert_close(f"decode y rows {r0}..{r0 + 63}", y_steps[rows], full[:, P:], torch.bfloat16)
        assert_close(f"one-call y rows {r0}..{r0 + 63}", y_call[rows], full[:, P:], torch.bfloat16)
        del full, alpha, logits


def test_module_step_graph_capture():
    """MoC.step captured in a HIP graph (static x / z buffers, the cache updated
    in place by the captured launch) and replayed once per token: each replay
    matches the eager step bit for bit (y and cache), with eager work and a
    synchronisation between replays."""
    B, D, Z, K, S, steps = 64, 512, 256, 16, 4, 6
    g = gen(77)
    m = MoC(D, Z, S, K, activation="silu", init_std=0.1)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.05))
    m = m.to(DEV, torch.bfloat16)
    xs = randn(g, B, steps, D).to(DEV, torch.bfloat16)
    zs = randn(g, B, steps, Z).to(DEV, torch.bfloat16)
    cache0 = randn(g, B, D, S).to(DEV, torch.bfloat16)
    assert moc.ops.decode_step_supported(xs[:, :1], zs[:, :1], m.router, m.conv_bases, cache0)
    ce, ye = cache0.clone(), []
    with torch.no_grad():
        for t in range(steps):
            y, _ = m.step(xs[:, t:t + 1], zs[:, t:t + 1], cache=ce)
            ye.append(y.clone())
    xin = torch.empty(B, 1, D, device=DEV, dtype=torch.bfloat16)
    zin = torch.empty(B, 1, Z, device=DEV, dtype=torch.bfloat16)
    cg = cache0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.no_grad():
        scratch = cache0.clone()
        for _ in range(2):
            m.step(xin.zero_(), zin.zero_(), cache=scratch)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        yg, _ = m.step(xin, zin, cache=cg)
    assert torch.equal(cg, cache0)  # capture records, it does not run
    for t in range(steps):
        xin.copy_(xs[:, t:t + 1])
        zin.copy_(zs[:, t:t + 1])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ye[t]), t
        (xs.float() * 2).sum().item()  # eager work between replays
    assert torch.equal(cg, ce)


def test_bwd_two_tier_ranges():
    """A backward grid of two workgroups per CU on a 256-CU part (D 2048: 16
    channel groups; 1827 tokens: 63 super-blocks over 32 ranges) runs with the
    ranges in two tiers, here of 2-3 and 1-2 super-blocks: fixed-length and
    packed inputs against the oracle."""
    dtype, D, K, S, act = torch.bfloat16, 2048, 16, 4, "silu"
    g = gen(1827)
    N = 1827
    x = randn(g, 1, N, D, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, 1, N, K), -1).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.2).to(DEV, dtype)
    dy = randn(g, 1, N, D).to(DEV, dtype)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)

    def run(**kw):
        xx, aa, bb = (t.clone().requires_grad_() for t in (x, a, b))
        if "cu_seqlens" in kw:
            y, _ = moc_triton(xx.view(-1, D), aa.view(-1, K), bb, activation=act, **kw)
            y.backward(dy.view(-1, D))
        else:
            y, _ = moc_triton(xx, aa, bb, activation=act)
            y.backward(dy)
        return y.detach().reshape(x.shape), xx.grad, aa.grad, bb.grad

    ref = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), act)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), run(), ref):
        assert_close(n, u, r, dtype)
    lengths = [300, 1, 640, 29, 857]
    cu = torch.tensor([0, *itertools.accumulate(lengths)], device=DEV, dtype=torch.int64)
    assert cu[-1] == N
    refv = O.moc_varlen_grads_ref(rx.detach().view(-1, D), ra.detach().view(-1, K), rb.detach(),
                                  cu.cpu(), dy.float().cpu().view(-1, D), act)
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), run(cu_seqlens=cu, max_seqlen=857), refv):
        assert_close("varlen " + n, u.reshape(r.shape), r, dtype)
