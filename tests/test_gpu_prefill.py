"""GPU parity of the prefill entries (moc_forward_prefill / moc_backward_prefill,
through moc.ops -> ctypes): a fixed-length batch continuing from a cache
(moc/api.py:299-309) with its final state (moc/api.py:218-227).

Checked against
  * the oracle's formulation (moc_prefill_ref: the cache prepended to x, zero
    routing weights prepended to alpha, the first S outputs dropped) by autograd
    on fp32 CPU leaves, under the tolerance rule of tests/_parity.py;
  * the same kernels run on that concatenated formulation: y bit for bit (each
    output's taps are summed in the same order, cache values where the
    concatenation has its rows);
  * O.final_state of the concatenation: the final state bit for bit.
"""
from __future__ import annotations

import pytest
import torch

from moc import moc_triton, ops
from moc._lib import ROUTE_ALPHA, ROUTE_EXP, ROUTE_SOFTMAX
from oracle import moc_oracle as O
from tests._parity import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF, F32 = torch.bfloat16, torch.float32


def _inputs(seed, B, T, D, K, S, dtype, logits=False):
    g = gen(seed)
    x = randn(g, B, T, D, scale=0.5).to(DEV, dtype)
    raw = randn(g, B, T, K)
    a = (raw if logits else torch.softmax(raw, -1)).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.1).to(DEV, dtype)
    c = randn(g, B, D, S, scale=0.5).to(DEV, dtype)
    dy = randn(g, B, T, D, scale=0.1).to(DEV, dtype)
    return x, a, b, c, dy


def _concat(x, a, c):
    B, _, _ = x.shape
    S = c.shape[-1]
    return torch.cat((c.transpose(1, 2), x), 1), torch.cat((a.new_zeros(B, S, a.shape[-1]), a), 1)


CASES = [  # S, K, activation, dtype, T (T >= S-1: the prefill entries' range)
    (4, 16, "silu", BF, 37),
    (4, 16, None, BF, 3),
    (4, 16, "silu", F32, 5),
    (2, 16, "silu", BF, 1),
    (2, 32, None, BF, 19),
    (3, 16, "silu", BF, 2),
    (3, 5, "silu", F32, 41),
    (8, 32, None, BF, 7),
    (8, 32, None, BF, 70),
    (7, 32, None, BF, 9),
    (5, 32, None, BF, 12),
    (7, 16, None, BF, 33),
    (4, 32, None, BF, 20),
    (8, 32, "silu", BF, 40),
    (8, 16, "silu", F32, 9),
    (8, 16, None, BF, 64),
    (4, 32, "silu", BF, 33),
    (4, 12, None, F32, 8),
    (5, 16, "silu", BF, 9),
    (6, 32, None, BF, 5),
    (7, 16, "silu", F32, 6),
    (4, 64, "silu", BF, 21),
    (3, 48, None, BF, 7),
    (5, 32, "silu", BF, 12),
    (7, 32, "silu", BF, 70),
    (6, 24, "silu", BF, 5),
    (8, 16, "silu", BF, 50),
    (8, 64, None, BF, 40),
    (7, 64, None, BF, 70),
    (5, 48, None, BF, 40),
    (6, 48, "silu", BF, 9),
    (8, 64, "silu", BF, 70),
    (2, 64, "silu", BF, 5),
]


@pytest.mark.parametrize("S,K,act,dtype,T", CASES)
def test_prefill_entries_against_oracle(S, K, act, dtype, T):
    _prefill_case(S, K, act, dtype, T, 192)


@pytest.mark.parametrize("S,K,act,dtype,T", [(4, 16, "silu", BF, 40), (8, 32, None, BF, 33),
                                              (7, 16, "silu", F32, 9), (4, 64, "silu", BF, 21)])
def test_prefill_even_channel_tail(S, K, act, dtype, T):
    """An even channel count that is not a multiple of 4 (198)."""
    _prefill_case(S, K, act, dtype, T, 198)


def _prefill_case(S, K, act, dtype, T, D):
    B = 3
    x, a, b, c, dy = _inputs(S * 100 + K + T, B, T, D, K, S, dtype)
    flag = 1 if act else 0
    assert ops.prefill_supported(x, b, with_cache=True)
    y, fin = ops.launch_forward_prefill(x, a, b, c, activation_flag=flag, final_state=True)
    fx, fa = _concat(x, a, c)
    y_cat = ops.launch_forward(fx, fa, b, activation_flag=flag)[:, S:]
    assert torch.equal(y, y_cat)
    assert torch.equal(fin, O.final_state(fx, None, S))
    dx, da, db, dc = ops.launch_backward_prefill(x, a, b, c, dy, activation_flag=flag,
                                                 need_x=True, need_cache=True)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, ra, rb, rc, act)
    ry.backward(dy.float().cpu())
    assert_close("prefill y", y, ry, dtype)
    assert_close("prefill dx", dx, rx.grad, dtype)
    assert_close("prefill dalpha", da, ra.grad, dtype)
    assert_close("prefill dbasis", db, rb.grad, dtype)
    assert_close("prefill dcache", dc, rc.grad, dtype)
    assert torch.all(dc[:, :, 0] == 0)


@pytest.mark.parametrize("S,K", [(8, 32), (6, 32), (7, 24), (4, 64), (8, 48)])
def test_prefill_two_pass_silu_without_dx(S, K):
    """With SiLU at these shapes the prefill backward runs two passes, the first
    forming g = dy silu'(P) with P over the cache: without dx, dalpha, dbasis
    and dcache equal those of the call with dx bit for bit."""
    B, T, D = 3, 45, 192
    x, a, b, c, dy = _inputs(S * 10 + K, B, T, D, K, S, BF)
    full = ops.launch_backward_prefill(x, a, b, c, dy, activation_flag=1, need_x=True,
                                       need_cache=True)
    part = ops.launch_backward_prefill(x, a, b, c, dy, activation_flag=1, need_x=False,
                                       need_cache=True)
    assert part[0] is None
    for n, u, v in zip(("dalpha", "dbasis", "dcache"), full[1:], part[1:]):
        assert torch.equal(u, v), n


@pytest.mark.parametrize("T,S", [(2, 4), (4, 4), (9, 4), (1, 8), (30, 8)])
def test_final_state_without_cache(T, S):
    """cache = NULL: y is the plain forward's bit for bit, and the final state
    is the last S inputs with zeros before the first token (any T)."""
    B, D, K = 2, 128, 16
    x, a, b, _, _ = _inputs(T + S, B, T, D, K, S, BF)
    assert ops.prefill_supported(x, b, with_cache=False)
    y, fin = ops.launch_forward_prefill(x, a, b, None, activation_flag=1, final_state=True)
    assert torch.equal(y, ops.launch_forward(x, a, b, activation_flag=1))
    assert torch.equal(fin, O.final_state(x, None, S))


@pytest.mark.parametrize("routing,name", [(ROUTE_SOFTMAX, "softmax"), (ROUTE_EXP, "exp")])
def test_prefill_with_router_logits(routing, name):
    """alpha as router logits whose softmax / exp the kernels form: y and the
    logits gradient against the oracle on weights rounded like torch's."""
    B, T, D, K, S, dtype = 2, 29, 128, 16, 4, BF
    x, lg, b, c, dy = _inputs(7 + routing, B, T, D, K, S, dtype, logits=True)
    lg = lg * 0.5
    y, fin = ops.launch_forward_prefill(x, lg, b, c, activation_flag=1, final_state=False,
                                        routing=routing)
    assert fin is None
    dx, dl, db, dc = ops.launch_backward_prefill(x, lg, b, c, dy, activation_flag=1,
                                                 need_x=True, need_cache=True, routing=routing)
    rx = x.detach().float().cpu().requires_grad_()
    rl = lg.detach().float().cpu().requires_grad_()
    rb = b.detach().float().cpu().requires_grad_()
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, O.route(rl, name, out_dtype=dtype), rb, rc, "silu")
    ry.backward(dy.float().cpu())
    assert_close("y", y, ry, dtype)
    assert_close("dx", dx, rx.grad, dtype)
    assert_close("dlogits", dl, rl.grad, dtype)
    assert_close("dbasis", db, rb.grad, dtype)
    assert_close("dcache", dc, rc.grad, dtype)


@pytest.mark.parametrize("T,S,dtype", [(20, 4, BF), (3, 4, BF), (11, 8, F32), (7, 8, BF)])
def test_moc_triton_prefill_autograd(T, S, dtype):
    """moc_triton with a cache on the prefill entries: gradients of a loss on y
    and on the final state (moc/api.py:218-227: a slice of x and, for T < S,
    of the cache) for x, alpha, basis and the cache against the oracle."""
    B, D, K = 2, 96, 16
    x, a, b, c, dy = _inputs(T * 3 + S, B, T, D, K, S, dtype)
    assert ops.prefill_supported(x, b, with_cache=True)
    dst = randn(gen(5), B, D, S, scale=0.2).to(DEV, dtype)
    xs, as_, bs, cs = (t.clone().requires_grad_() for t in (x, a, b, c))
    y, st = moc_triton(xs, as_, bs, cache=cs, output_final_state=True, activation="silu")
    ((y.float() * dy.float()).sum() + (st.float() * dst.float()).sum()).backward()
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, ra, rb, rc, "silu")
    rst = O.final_state(torch.cat((rc.transpose(1, 2), rx), 1), None, S)
    ((ry * dy.float().cpu()).sum() + (rst * dst.float().cpu()).sum()).backward()
    assert_close("y", y, ry, dtype)
    assert torch.equal(st.detach().float().cpu(), rst.detach())
    assert_close("dx", xs.grad, rx.grad, dtype)
    assert_close("dalpha", as_.grad, ra.grad, dtype)
    assert_close("dbasis", bs.grad, rb.grad, dtype)
    assert_close("dcache", cs.grad, rc.grad, dtype)


def test_prefill_broadcast_dy_matches_full_dy():
    """The gradient of y.sum() (one broadcast row, row stride 0) gives the
    results of the same gradient as a contiguous tensor, bit for bit."""
    B, T, D, K, S = 2, 50, 256, 16, 4
    x, a, b, c, _ = _inputs(11, B, T, D, K, S, BF)
    ones = torch.ones(B, T, D, device=DEV, dtype=BF)
    got = ops.launch_backward_prefill(x, a, b, c, torch.ones((), device=DEV, dtype=BF).expand(B, T, D),
                                      activation_flag=1, need_x=True, need_cache=True)
    ref = ops.launch_backward_prefill(x, a, b, c, ones, activation_flag=1, need_x=True,
                                      need_cache=True)
    for u, v in zip(got, ref):
        assert torch.equal(u, v)


def test_prefill_headline_shape():
    """configs[1]'s layer shape (D 2048, K 16, S 4, SiLU, bf16) continuing from a
    cache, B 4 x T 1024: y bit for bit against the concatenated formulation on
    the same kernels, the final state exact, gradients against the oracle."""
    B, T, D, K, S, dtype = 4, 1024, 2048, 16, 4, BF
    x, a, b, c, dy = _inputs(2048, B, T, D, K, S, dtype)
    y, fin = ops.launch_forward_prefill(x, a, b, c, activation_flag=1, final_state=True)
    fx, fa = _concat(x, a, c)
    assert torch.equal(y, ops.launch_forward(fx, fa, b, activation_flag=1)[:, S:])
    assert torch.equal(fin, O.final_state(fx, None, S))
    dx, da, db, dc = ops.launch_backward_prefill(x, a, b, c, dy, activation_flag=1,
                                                 need_x=True, need_cache=True)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, ra, rb, rc, "silu")
    ry.backward(dy.float().cpu())
    assert_close("y", y, ry, dtype)
    assert_close("dx", dx, rx.grad, dtype)
    assert_close("dalpha", da, ra.grad, dtype)
    assert_close("dbasis", db, rb.grad, dtype)
    assert_close("dcache", dc, rc.grad, dtype)


def test_backward_8_taps_32_routes_silu():
    """The plain backward with SiLU at 8 taps and 32 routes (bf16): its fused
    pass needs more workspace than the two-pass plan of the same shape without
    the activation, and moc_backward_workspace_bytes sizes for both."""
    B, T, D, K, S, dtype = 2, 300, 256, 32, 8, BF
    x, a, b, _, dy = _inputs(88, B, T, D, K, S, dtype)
    xs, as_, bs = (t.clone().requires_grad_() for t in (x, a, b))
    y, _ = moc_triton(xs, as_, bs, activation="silu")
    y.backward(dy)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    ry, rdx, rda, rdb = O.moc_grads_ref(rx, ra, rb, dy.float().cpu(), "silu")
    assert_close("y", y, ry, dtype)
    assert_close("dx", xs.grad, rdx, dtype)
    assert_close("dalpha", as_.grad, rda, dtype)
    assert_close("dbasis", bs.grad, rdb, dtype)


@pytest.mark.parametrize("route", ["softmax", "exp"])
def test_module_prefill_gradients(route):
    """MoC.forward continuing from a cache on its kernel path (router epilogue +
    prefill entries, one autograd node): y, the final state and the gradients
    of x, z, router, basis and the cache against the oracle chain on the
    module's own bf16 logits."""
    from moc import MoC, router_linear
    from tests._parity import ulp_allowance
    B, T, D, Z, K, S, bf = 2, 40, 128, 64, 16, 4, torch.bfloat16
    g = gen(31)
    m = MoC(D, Z, S, K, activation="silu", init_std=0.1, router_activation=route)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.1))
    m = m.to(DEV, bf)
    x = randn(g, B, T, D, scale=0.5).to(DEV, bf).requires_grad_()
    z = randn(g, B, T, Z).to(DEV, bf).requires_grad_()
    c = randn(g, B, D, S, scale=0.5).to(DEV, bf).requires_grad_()
    dy = randn(g, B, T, D, scale=0.1).to(DEV, bf)
    y, st = m(x, z, cache=c, output_final_state=True)
    y.backward(dy)
    with torch.no_grad():
        logits = router_linear(z, m.router).cpu()
    lf = logits.float().requires_grad_()
    rx = x.detach().float().cpu().requires_grad_()
    rb = m.conv_bases.detach().float().cpu().requires_grad_()
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, O.route(lf, route, out_dtype=bf), rb, rc, "silu")
    ry.backward(dy.float().cpu())
    dl = lf.grad.to(bf).float().reshape(-1, K)
    rz = (dl @ m.router.detach().float().cpu()).reshape(B, T, Z)
    rr = dl.T @ z.detach().float().cpu().reshape(-1, Z)
    assert_close("y", y, ry, bf)
    assert torch.equal(st, O.final_state(torch.cat((c.detach().transpose(1, 2), x.detach()), 1),
                                         None, S))
    assert_close("dx", x.grad, rx.grad, bf)
    assert_close("dz", z.grad, rz, bf, extra=ulp_allowance(lf.grad, m.router.cpu()))
    assert_close("drouter", m.router.grad, rr, bf)
    assert_close("dbasis", m.conv_bases.grad, rb.grad, bf)
    assert_close("dcache", c.grad, rc.grad, bf)


@pytest.mark.parametrize("K,act", [(16, "silu"), (64, None)])
def test_prefill_backward_multi_range_workspace(K, act):
    """The prefill backward at a token count that spans many token ranges, at
    shapes whose plain backward runs the two-pass form while the prefill keeps
    the fused pass (8 taps: 16 routes with SiLU, 64 without activation), so the
    two plans' partial grids differ: the workspace the size query returns
    serves the prefill call, and the gradients match the oracle."""
    B, T, D, S, dtype = 2, 4096, 128, 8, BF
    x, a, b, c, dy = _inputs(K + S, B, T, D, K, S, dtype)
    flag = 1 if act else 0
    dx, da, db, dc = ops.launch_backward_prefill(x, a, b, c, dy, activation_flag=flag,
                                                 need_x=True, need_cache=True)
    rx, ra, rb = O.reference_inputs(x, a, b, dtype)
    rc = c.detach().float().cpu().requires_grad_()
    ry = O.moc_prefill_ref(rx, ra, rb, rc, act)
    ry.backward(dy.float().cpu())
    assert_close("dx", dx, rx.grad, dtype)
    assert_close("dalpha", da, ra.grad, dtype)
    assert_close("dbasis", db, rb.grad, dtype)
    assert_close("dcache", dc, rc.grad, dtype)
