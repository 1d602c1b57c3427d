"""GPU parity of the router GEMM kernels (logits = z . router^T and its
backward), which replace the F.linear(z, router) of MoC.forward
(moc/api.py:383-388) for bf16 layers.

References are plain fp32 products of the same bf16 inputs; the bf16 outputs
are held to the bf16 rule of tests/_parity.py.  Shapes cover single tokens,
token counts that are not multiples of the 16-token tiles, every supported k
class (k % 4 == 0 up to 96, one to six 16-route chunks) and the
BASELINE sizes.
"""
from __future__ import annotations

import pytest
import torch

import moc
from moc import MoC, ops
from tests._parity import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16

SHAPES = [
    (1, 64, 16), (15, 64, 4), (16, 128, 16), (17, 192, 12), (50, 64, 20), (77, 320, 28),
    (333, 256, 32), (1000, 2048, 16), (4096, 4096, 32), (16384, 2048, 16),
    (70, 128, 36), (129, 192, 48), (33, 64, 64), (300, 256, 80), (1000, 512, 96),
    (16384, 4096, 96),
]


def _inputs(N, Z, K, seed):
    g = gen(seed)
    z = randn(g, N, Z).to(DEV, BF)
    r = randn(g, K, Z, scale=0.02).to(DEV, BF)
    dl = randn(g, N, K, scale=0.05).to(DEV, BF)
    return z, r, dl


@pytest.mark.parametrize("N,Z,K", SHAPES)
def test_router_forward_and_backward(N, Z, K):
    z, r, dl = _inputs(N, Z, K, N * 7 + Z + K)
    assert ops.router_supported(z, r)
    logits = ops.router_forward(z, r)
    assert logits.shape == (N, K) and logits.dtype == BF
    assert_close("logits", logits, z.float() @ r.float().T, BF)
    dz, dr = ops.router_backward(z, r, dl, True, True)
    assert_close("dz", dz, dl.float() @ r.float(), BF)
    assert_close("drouter", dr, dl.float().T @ z.float(), BF)
    # either output alone gives the same values; drouter is reduced in a fixed order
    dz_only, none_r = ops.router_backward(z, r, dl, True, False)
    none_z, dr_only = ops.router_backward(z, r, dl, False, True)
    assert none_r is None and none_z is None
    assert torch.equal(dz_only, dz)
    assert torch.equal(dr_only, dr)


def test_router_batched_input_and_autograd():
    B, T, Z, K = 3, 37, 128, 16
    g = gen(5)
    z = randn(g, B, T, Z).to(DEV, BF).requires_grad_()
    r = randn(g, K, Z, scale=0.05).to(DEV, BF).requires_grad_()
    dl = randn(g, B, T, K, scale=0.1).to(DEV, BF)
    logits = moc.router_linear(z, r)
    assert type(logits.grad_fn).__name__.startswith("_RouterLinear")
    logits.backward(dl)
    zf, rf = z.detach().float(), r.detach().float()
    assert_close("logits", logits, zf @ rf.T, BF)
    assert_close("dz", z.grad, dl.float() @ rf, BF)
    assert_close("drouter", r.grad, dl.float().reshape(-1, K).T @ zf.reshape(-1, Z), BF)


@pytest.mark.parametrize("Z,K,dtype", [(48, 16, BF), (64, 6, BF), (64, 100, BF), (64, 16, torch.float32)])
def test_router_unsupported_shapes_use_torch(Z, K, dtype):
    g = gen(Z + K)
    z = randn(g, 5, Z).to(DEV, dtype)
    r = randn(g, K, Z, scale=0.1).to(DEV, dtype)
    assert not ops.router_supported(z, r)
    out = moc.router_linear(z, r)
    assert torch.equal(out, torch.nn.functional.linear(z, r))


@pytest.mark.parametrize("route", ["softmax", "exp"])
def test_module_router_kernels_match_torch_gemm(route):
    """The bf16 layer with the router kernels against the same layer whose
    router GEMM is torch's (F.linear): y and every gradient within bf16 rules."""
    torch.manual_seed(0)
    D, Z, K, S, B, T = 128, 256, 16, 4, 2, 80
    m = MoC(D, Z, S, K, activation="silu", init_std=0.05, router_activation=route)
    g = gen(9)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.05))
    m = m.to(DEV, BF)
    x = randn(g, B, T, D).to(DEV, BF)
    z = randn(g, B, T, Z).to(DEV, BF)
    dy = randn(g, B, T, D, scale=0.1).to(DEV, BF)

    def run(use_kernels):
        m.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_()
        zi = z.clone().requires_grad_()
        if use_kernels:
            y, _ = m(xi, zi)
        else:
            logits = torch.nn.functional.linear(zi, m.router)
            y, _ = moc.api._dispatch(xi, logits, m.conv_bases, None, False, m.activation,
                                     m.router_activation, None, None, None, None)
        y.backward(dy)
        return y.detach(), xi.grad, zi.grad, m.router.grad.clone(), m.conv_bases.grad.clone()

    got, ref = run(True), run(False)
    for name, a, b in zip(("y", "dx", "dz", "drouter", "dbasis"), got, ref):
        assert_close(name, a, b.float(), BF)


@pytest.mark.parametrize("K,S,route,act,varlen", [
    (16, 4, "softmax", "silu", False), (16, 4, "exp", None, False),
    (16, 3, "softmax", "silu", True), (12, 4, "softmax", "silu", False),
    (32, 8, "exp", "silu", False), (20, 2, "softmax", None, True),
])
def test_layer_function_matches_logits_path(K, S, route, act, varlen):
    """MoC.forward as one autograd node (the router kernel forms the weights,
    the MoC kernels take them as given and return d(logits)) against the
    two-node path (router logits, the MoC kernels form the weights): both run
    the same arithmetic in the same order, so y and every gradient agree bit
    for bit.  K = 16 takes the kernels' in-place operand path, other K the
    prepared-operand path."""
    D, Z, B, T = 192, 128, 2, 77
    torch.manual_seed(K + S)
    m = MoC(D, Z, S, K, activation=act, init_std=0.1, router_activation=route)
    g = gen(K * 10 + S)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.1))
    m = m.to(DEV, BF)
    if varlen:
        lengths = [1, 30, 2, 77, 44]
        cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32,
                          device=DEV)
        shape, kw = (sum(lengths),), dict(cu_seqlens=cu, max_seqlen=max(lengths))
    else:
        shape, kw = (B, T), {}
    x = randn(g, *shape, D).to(DEV, BF)
    z = randn(g, *shape, Z).to(DEV, BF)
    dy = randn(g, *shape, D, scale=0.1).to(DEV, BF)

    def run(one_node):
        m.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_()
        zi = z.clone().requires_grad_()
        if one_node:
            y, _ = m(xi, zi, **kw)
            assert type(y.grad_fn).__name__.startswith("_MoCLayerFunction")
        else:
            logits = moc.router_linear(zi, m.router)
            y, _ = moc.api._dispatch(xi, logits, m.conv_bases, None, False, m.activation,
                                     m.router_activation, kw.get("cu_seqlens"),
                                     kw.get("max_seqlen"), None, None)
        y.backward(dy)
        return y.detach(), xi.grad, zi.grad, m.router.grad.clone(), m.conv_bases.grad.clone()

    got, ref = run(True), run(False)
    for name, a, b in zip(("y", "dx", "dz", "drouter", "dbasis"), got, ref):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("K", [4, 16, 20, 32])
@pytest.mark.parametrize("route", ["softmax", "exp"])
def test_router_forward_routed_weights(K, route):
    """The router kernel's fused activation against torch's softmax / exp of
    the kernel's own bf16 logits (torch rounds the activation to bf16 once)."""
    N, Z = 333, 192
    z, r, _ = _inputs(N, Z, K, K + 3)
    code = moc.api._ROUTING_CODES[route]
    w = ops.router_forward(z, r, routing=code)
    logits = ops.router_forward(z, r)
    ref = torch.softmax(logits.float(), -1) if route == "softmax" else torch.exp(logits.float())
    assert w.dtype == BF and w.shape == (N, K)
    # one bf16 ulp: torch's exp / division may round differently in fp32
    assert_close("weights", w, ref, BF)


def _qkv_layers(specs, Z, seed):
    """MoC layers (dim, k, S, activation, router_activation) on one z_dim, bf16;
    router and basis drawn from the seeded generator."""
    g = gen(seed)
    layers = []
    for D, K, S, act, route in specs:
        m = MoC(D, Z, S, K, activation=act, init_std=0.1, router_activation=route)
        with torch.no_grad():
            m.router.copy_(randn(g, K, Z, scale=0.05))
            m.conv_bases.copy_(randn(g, K, S, D, scale=0.1))
        layers.append(m.to(DEV, BF))
    return layers, g


def _bf16_ulp(t):
    a = t.detach().float().abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


def _run_layers(layers, xs, z, dys, grouped, **kw):
    """Outputs and gradients; separately (grouped False) each layer gets its own
    z leaf, and dz is their fp32 sum with, as a second value, the rounding of
    the per-layer bf16 dz (half an ulp each) as an allowance."""
    for m in layers:
        m.zero_grad(set_to_none=True)
    xi = [x.clone().requires_grad_() for x in xs]
    if grouped:
        zi = z.clone().requires_grad_()
        outs = moc.MoCGroup(*layers)(xi, zi, **kw)
    else:
        zs = [z.clone().requires_grad_() for _ in layers]
        outs = [m(x, zl, **kw) for m, x, zl in zip(layers, xi, zs)]
    torch.autograd.backward([y for y, _ in outs], dys)
    if grouped:
        dz = zi.grad
    else:
        dz = (sum(zl.grad.float() for zl in zs), sum(0.5 * _bf16_ulp(zl.grad) for zl in zs))
    return ([y.detach() for y, _ in outs], [x.grad for x in xi], dz,
            [m.router.grad.clone() for m in layers], [m.conv_bases.grad.clone() for m in layers])


QKV_SPECS = [
    [(256, 32, 8, None, "exp"), (64, 32, 8, None, "exp"), (64, 32, 8, None, "softmax")],
    [(192, 16, 4, "silu", "softmax"), (128, 16, 4, "silu", "exp"), (64, 16, 4, "silu", "softmax")],
    [(256, 32, 4, "silu", "exp"), (96, 32, 4, "silu", "softmax")],
    [(192, 16, 4, "silu", "softmax"), (128, 20, 3, None, "exp")],
    [(128, 8, 2, "silu", "softmax"), (64, 4, 4, None, "exp"), (64, 12, 4, None, "softmax"),
     (32, 32, 8, "silu", "exp")],
    # one S, each layer its own K and activation (one grouped call)
    [(192, 16, 4, "silu", "softmax"), (128, 32, 4, None, "exp"), (64, 12, 4, "silu", "softmax")],
    [(256, 32, 6, None, "exp"), (64, 16, 6, "silu", "exp"), (128, 16, 6, None, "softmax")],
]


@pytest.mark.parametrize("specs", QKV_SPECS)
@pytest.mark.parametrize("varlen", [False, True])
def test_group_matches_separate_layers(specs, varlen):
    """MoCGroup (one router pass over the concatenated routers, one grouped
    forward and backward call over all layers when they share S, one router
    backward) against the same layers called one by one: y, dx,
    drouter and dbasis bit for bit (every workgroup does the work of its own
    layer's launch, same reduction order); dz, which the group sums over all
    routes in fp32 and rounds once, against the fp32 sum of the layers' own bf16
    dz, within the bf16 rule plus half an ulp of each rounding."""
    Z, B, T = 128, 2, 61
    layers, g = _qkv_layers(specs, Z, sum(s[0] + s[1] for s in specs) + 10 * len(specs) + varlen)
    if varlen:
        lengths = [5, 40, 1, 70, 7]
        cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32,
                          device=DEV)
        lead, kw = (sum(lengths),), dict(cu_seqlens=cu, max_seqlen=max(lengths))
    else:
        lead, kw = (B, T), {}
    xs = [randn(g, *lead, D).to(DEV, BF) for D, *_ in specs]
    z = randn(g, *lead, Z).to(DEV, BF)
    dys = [randn(g, *lead, D, scale=0.1).to(DEV, BF) for D, *_ in specs]
    assert moc.ops.router_grouped_supported(z, [m.router for m in layers])
    got = _run_layers(layers, xs, z, dys, True, **kw)
    ref = _run_layers(layers, xs, z, dys, False, **kw)
    for name, a, b in (("y", got[0], ref[0]), ("dx", got[1], ref[1]), ("drouter", got[3], ref[3]),
                       ("dbasis", got[4], ref[4])):
        for i, (u, v) in enumerate(zip(a, b)):
            assert torch.equal(u, v), f"{name}[{i}]"
    ref_dz, rounding = ref[2]
    assert_close("dz", got[2], ref_dz, BF, extra=rounding + 0.5 * _bf16_ulp(ref_dz))


def test_group_falls_back_to_layers():
    """fp32 layers (no router kernels): the group runs the layers one by one."""
    Z = 64
    g = gen(3)
    layers = [MoC(64, Z, 4, 8, init_std=0.1).to(DEV), MoC(32, Z, 4, 8, init_std=0.1).to(DEV)]
    for m in layers:
        with torch.no_grad():
            m.router.copy_(randn(g, 8, Z, scale=0.1))
    xs = [randn(g, 2, 9, 64).to(DEV), randn(g, 2, 9, 32).to(DEV)]
    z = randn(g, 2, 9, Z).to(DEV)
    assert not moc.ops.router_grouped_supported(z, [m.router for m in layers])
    outs = moc.MoCGroup(*layers)(xs, z, output_final_state=True)
    for (y, st), m, x in zip(outs, layers, xs):
        y2, st2 = m(x, z, output_final_state=True)
        assert torch.equal(y, y2) and torch.equal(st, st2)


@pytest.mark.parametrize("ks,routes", [([32, 32, 32], [2, 2, 1]), ([16, 20], [1, 0]),
                                       ([4, 8, 12, 28], [1, 2, 1, 2])])
def test_router_forward_grouped_matches_per_router(ks, routes):
    """The grouped router pass against one router launch per group: bit for bit
    (routing 0 gives the group's logits)."""
    N, Z = 301, 192
    g = gen(sum(ks))
    z = randn(g, N, Z).to(DEV, BF)
    rs = [randn(g, k, Z, scale=0.05).to(DEV, BF) for k in ks]
    outs = ops.router_forward_grouped(z, torch.cat(rs, 0), ks, routes)
    for o, r, code in zip(outs, rs, routes):
        assert torch.equal(o, ops.router_forward(z, r, routing=code))
