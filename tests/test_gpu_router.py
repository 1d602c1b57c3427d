"""GPU parity of the router GEMM kernels (logits = z . router^T and its
backward), which replace the F.linear(z, router) of MoC.forward
(moc/api.py:383-388) for bf16 layers.

References are plain fp32 products of the same bf16 inputs; the bf16 outputs
are held to the bf16 rule of tests/_parity.py.  Shapes cover single tokens,
token counts that are not multiples of the 16-token tiles, every supported k
class (k % 4 == 0 up to 32, with and without a second 16-route half) and the
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


@pytest.mark.parametrize("Z,K,dtype", [(48, 16, BF), (64, 6, BF), (64, 36, BF), (64, 16, torch.float32)])
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
