"""GPU parity: the HIP kernels (through moc -> ctypes -> libmoc_hip.so) against
the CPU oracle on identical seeded inputs.

Covers the reference's verify.py matrix (moc/../verify.py:243-285: {bf16, fp32} x
S in {2,4} x {plain, SiLU} x {fixed, varlen in both forms, step} plus mixed
storage dtypes) and what it leaves out: the MoC module with
softmax / exp routing, prefill from a cache, final states, need_x=False, int64
cu_seqlens, sequences shorter than S, D not a multiple of any tile, odd K and
S, bitwise varlen isolation, bitwise determinism.  Tolerances: tests/_parity.py.
"""
from __future__ import annotations

import itertools

import pytest
import torch

import moc
from moc import MoC, moc_triton
from oracle import moc_oracle as O
from tests._parity import assert_close, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

B, T, D, K = 2, 64, 64, 8
VARLEN_LENGTHS = [31, 17, 5, 23]
STEP_T = 8


def _verify_inputs(seed=0):
    g = gen(seed)
    x = randn(g, B, T, D, scale=0.5)
    alpha = torch.softmax(randn(g, B, T, K), -1)
    dy = randn(g, B, T, D, scale=0.1)
    N = sum(VARLEN_LENGTHS)
    xv = randn(g, N, D, scale=0.5)
    av = torch.softmax(randn(g, N, K), -1)
    dyv = randn(g, N, D, scale=0.1)
    return g, x, alpha, dy, xv, av, dyv


def _cu(lengths, dtype=torch.int32):
    return torch.tensor([0, *itertools.accumulate(lengths)], dtype=dtype)


def _run_fixed(x, a, b, dy, dtype, a_dt, b_dt, act):
    kx = x.to(DEV, dtype).requires_grad_()
    ka = a.to(DEV, a_dt).requires_grad_()
    kb = b.to(DEV, b_dt).requires_grad_()
    y, st = moc_triton(kx, ka, kb, activation=act)
    assert st is None and y.dtype == dtype
    y.backward(dy.to(DEV, dtype))
    rx, ra, rb = O.reference_inputs(kx, ka, kb, dtype)
    ry, rdx, rda, rdb = O.moc_grads_ref(rx, ra, rb, dy.to(dtype).float(), act)
    assert_close("y", y, ry, dtype)
    assert_close("dx", kx.grad, rdx, dtype)
    assert_close("dalpha", ka.grad, rda, dtype)
    assert_close("dbasis", kb.grad, rdb, dtype)
    assert kx.grad.dtype == dtype and ka.grad.dtype == a_dt and kb.grad.dtype == b_dt


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S", [2, 4])
@pytest.mark.parametrize("act", [None, "silu"])
def test_fixed(dtype, S, act):
    g, x, a, dy, *_ = _verify_inputs()
    b = randn(g, K, S, D, scale=0.1)
    _run_fixed(x, a, b, dy, dtype, dtype, dtype, act)


@pytest.mark.parametrize("dtype,a_dt,b_dt", [
    (torch.bfloat16, torch.float32, torch.float16),
    (torch.float32, torch.bfloat16, torch.float16),
    (torch.bfloat16, torch.float64, torch.float32),
])
def test_mixed_storage_dtypes(dtype, a_dt, b_dt):
    g, x, a, dy, *_ = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1)
    _run_fixed(x, a, b, dy, dtype, a_dt, b_dt, None)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S", [2, 4])
@pytest.mark.parametrize("act", [None, "silu"])
@pytest.mark.parametrize("cu_dt", [torch.int32, torch.int64])
def test_varlen(dtype, S, act, cu_dt):
    g, _, _, _, xv, av, dyv = _verify_inputs()
    b = randn(g, K, S, D, scale=0.1)
    cu = _cu(VARLEN_LENGTHS, cu_dt).to(DEV)
    kx = xv.to(DEV, dtype).requires_grad_()
    ka = av.to(DEV, dtype).requires_grad_()
    kb = b.to(DEV, dtype).requires_grad_()
    y, st = moc_triton(kx, ka, kb, cu_seqlens=cu, max_seqlen=max(VARLEN_LENGTHS), activation=act)
    assert st is None
    y.backward(dyv.to(DEV, dtype))
    rx, ra, rb = O.reference_inputs(kx, ka, kb, dtype)
    ry, rdx, rda, rdb = O.moc_varlen_grads_ref(rx, ra, rb, cu.cpu(), dyv.to(dtype).float(), act)
    assert_close("y", y, ry, dtype)
    assert_close("dx", kx.grad, rdx, dtype)
    assert_close("dalpha", ka.grad, rda, dtype)
    assert_close("dbasis", kb.grad, rdb, dtype)
    y3, _ = moc_triton(kx.detach()[None], ka.detach()[None], kb.detach(), cu_seqlens=cu,
                       max_seqlen=max(VARLEN_LENGTHS), activation=act)
    assert y3.shape == (1, *y.shape)
    assert torch.equal(y3[0], y.detach())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S", [2, 4])
@pytest.mark.parametrize("act", [None, "silu"])
def test_step(dtype, S, act):
    g, x, a, *_ = _verify_inputs()
    b = randn(g, K, S, D, scale=0.1)
    kx = x[:, :STEP_T].to(DEV, dtype)
    ka = a[:, :STEP_T].to(DEV, dtype)
    kb = b.to(DEV, dtype)
    ref = O.moc_ref(kx.float().cpu(), ka.float().cpu(), kb.float().cpu(), act)
    cache = torch.zeros(B, D, S, device=DEV, dtype=dtype)
    outs = []
    for t in range(STEP_T):
        y, cache2 = moc_triton(kx[:, t:t + 1], ka[:, t:t + 1], kb, cache=cache,
                               output_final_state=True, activation=act)
        assert cache2 is cache            # the same object, mutated in place
        outs.append(y)
    assert_close("step y", torch.cat(outs, 1), ref, dtype)
    assert torch.equal(cache, kx[:, -S:].transpose(1, 2))


def test_step_with_strided_cache_and_no_final_state():
    g, x, a, *_ = _verify_inputs()
    S = 4
    b = randn(g, K, S, D, scale=0.1).to(DEV, torch.bfloat16)
    store = torch.zeros(B, S, D, device=DEV, dtype=torch.bfloat16)
    cache = store.transpose(1, 2)        # [B, D, S] view with non-unit slot stride
    kx = x[:, :6].to(DEV, torch.bfloat16)
    ka = a[:, :6].to(DEV, torch.bfloat16)
    for t in range(6):
        y, st = moc_triton(kx[:, t:t + 1], ka[:, t:t + 1], b, cache=cache)
        assert st is None
    assert torch.equal(cache, kx[:, -S:].transpose(1, 2))


@pytest.mark.parametrize("route", ["softmax", "exp"])
@pytest.mark.parametrize("act", [None, "silu"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_module_routed_fwd_bwd(route, act, dtype):
    torch.manual_seed(0)
    Z = 48
    m = MoC(dim=D, z_dim=Z, kernel_size=4, k=K, activation=act, init_std=0.1,
            router_activation=route)
    g = gen(3)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.2))
    m = m.to(DEV, dtype)
    x = randn(g, B, T, D, scale=0.5).to(DEV, dtype).requires_grad_()
    z = randn(g, B, T, Z).to(DEV, dtype).requires_grad_()
    dy = randn(g, B, T, D, scale=0.1).to(DEV, dtype)
    y, _ = m(x, z)
    y.backward(dy)

    # oracle layer: the module's own router GEMM (same dtype, on the GPU), the
    # router activation rounded like torch's, the MoC op by the CPU oracle
    lz = z.detach().requires_grad_()
    lr = m.router.detach().requires_grad_()
    logits = torch.nn.functional.linear(lz, lr)
    rx = x.detach().float().cpu().requires_grad_()
    rb = m.conv_bases.detach().float().cpu().requires_grad_()
    alpha = O.route(logits.float().cpu(), route, out_dtype=dtype)
    ry = O.moc_ref(rx, alpha, rb, act)
    ry.backward(dy.float().cpu())
    rz, rr = lz, lr
    assert_close("y", y, ry, dtype)
    assert_close("dx", x.grad, rx.grad, dtype)
    assert_close("dz", z.grad, rz.grad, dtype)
    assert_close("drouter", m.router.grad, rr.grad, dtype)
    assert_close("dbasis", m.conv_bases.grad, rb.grad, dtype)


@pytest.mark.parametrize("T1,T2", [(10, 7), (2, 9), (3, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_from_cache_and_final_state(T1, T2, dtype):
    """Prefill continuing from a cache (moc/api.py:299-309): y, the final states
    and the gradients of x, alpha, basis and the cache against autograd of the
    oracle's formulation (moc_prefill_ref: the cache prepended to x, zero
    weights prepended to alpha, the first S outputs dropped)."""
    S, act = 4, "silu"
    g, x, a, dy, *_ = _verify_inputs()
    b = randn(g, K, S, D, scale=0.1).to(DEV, dtype)
    kx = x[:, :T1 + T2].to(DEV, dtype)
    ka = a[:, :T1 + T2].to(DEV, dtype)
    y1, st1 = moc_triton(kx[:, :T1], ka[:, :T1], b, output_final_state=True, activation=act)
    assert torch.equal(st1, O.final_state(kx[:, :T1], None, S))
    x2, a2, b2, c2 = (t.clone().requires_grad_() for t in (kx[:, T1:], ka[:, T1:], b, st1))
    y2, st2 = moc_triton(x2, a2, b2, cache=c2, output_final_state=True, activation=act)
    assert torch.equal(st2, O.final_state(kx, None, S))
    dy2 = dy[:, :T2].to(DEV, dtype)
    y2.backward(dy2)
    ref = O.moc_ref(kx.float().cpu(), ka.float().cpu(), b.float().cpu(), act)
    assert_close("prefill y", y2, ref[:, T1:], dtype)
    assert_close("first y", y1, ref[:, :T1], dtype)
    rx, ra, rb, rc = (t.detach().float().cpu().requires_grad_() for t in (x2, a2, b2, c2))
    ry = O.moc_prefill_ref(rx, ra, rb, rc, act)
    ry.backward(dy2.float().cpu())
    assert_close("prefill y (oracle prefill)", y2, ry, dtype)
    assert_close("prefill dx", x2.grad, rx.grad, dtype)
    assert_close("prefill dalpha", a2.grad, ra.grad, dtype)
    assert_close("prefill dbasis", b2.grad, rb.grad, dtype)
    assert_close("prefill dcache", c2.grad, rc.grad, dtype)


def test_need_x_false_and_alpha_only_grads():
    g, x, a, dy, *_ = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1)
    kx = x.to(DEV, torch.float32)
    ka = a.to(DEV).requires_grad_()
    kb = b.to(DEV).requires_grad_()
    y, _ = moc_triton(kx, ka, kb, activation="silu")
    y.backward(dy.to(DEV))
    rx, ra, rb = O.reference_inputs(kx, ka, kb, torch.float32)
    _, _, rda, rdb = O.moc_grads_ref(rx, ra, rb, dy, "silu")
    assert_close("dalpha", ka.grad, rda, torch.float32)
    assert_close("dbasis", kb.grad, rdb, torch.float32)


@pytest.mark.parametrize("Dd,Kk,S,Tt", [
    (67, 5, 3, 11), (16, 1, 1, 5), (130, 17, 5, 9), (96, 33, 8, 20), (40, 16, 4, 3),
    (200, 32, 8, 37), (64, 12, 6, 2),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_odd_shapes(Dd, Kk, S, Tt, dtype):
    g = gen(Dd * 31 + Kk)
    x = randn(g, 3, Tt, Dd, scale=0.5)
    a = torch.softmax(randn(g, 3, Tt, Kk), -1)
    b = randn(g, Kk, S, Dd, scale=0.2)
    dy = randn(g, 3, Tt, Dd, scale=0.1)
    _run_fixed(x, a, b, dy, dtype, dtype, dtype, "silu")


def test_varlen_short_sequences_and_empty_ones():
    # lengths below S, length-1 and zero-length sequences
    lengths = [1, 0, 2, 3, 0, 9, 1]
    dtype = torch.float32
    g = gen(5)
    N = sum(lengths)
    xv = randn(g, N, D)
    av = torch.softmax(randn(g, N, K), -1)
    b = randn(g, K, 4, D, scale=0.2)
    dyv = randn(g, N, D)
    cu = _cu(lengths).to(DEV)
    kx = xv.to(DEV).requires_grad_()
    ka = av.to(DEV).requires_grad_()
    kb = b.to(DEV).requires_grad_()
    y, _ = moc_triton(kx, ka, kb, cu_seqlens=cu, max_seqlen=9, activation="silu")
    y.backward(dyv.to(DEV))
    ry, rdx, rda, rdb = O.moc_varlen_grads_ref(xv, av, b, cu.cpu(), dyv, "silu")
    assert_close("y", y, ry, dtype)
    assert_close("dx", kx.grad, rdx, dtype)
    assert_close("dalpha", ka.grad, rda, dtype)
    assert_close("dbasis", kb.grad, rdb, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_varlen_isolation_is_bitwise(dtype):
    """Perturbing other sequences leaves y, dx and dalpha of a probed sequence
    bitwise unchanged."""
    g, _, _, _, xv, av, dyv = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1).to(DEV, dtype)
    cu = _cu(VARLEN_LENGTHS).to(DEV)
    lo, hi = 31, 48  # sequence 1

    def run(xs, as_, dys):
        kx = xs.to(DEV, dtype).requires_grad_()
        ka = as_.to(DEV, dtype).requires_grad_()
        y, _ = moc_triton(kx, ka, b, cu_seqlens=cu, max_seqlen=31, activation="silu")
        y.backward(dys.to(DEV, dtype))
        return y.detach()[lo:hi], kx.grad[lo:hi], ka.grad[lo:hi]

    base = run(xv, av, dyv)
    x2, a2, d2 = xv.clone(), av.clone(), dyv.clone()
    for sl in (slice(0, lo), slice(hi, None)):
        x2[sl] = x2[sl] * 3 + 1
        a2[sl] = a2[sl].flip(-1)
        d2[sl] = -d2[sl]
    pert = run(x2, a2, d2)
    for u, v in zip(base, pert):
        assert torch.equal(u, v)


def test_determinism_bitwise():
    g, x, a, dy, *_ = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1)
    grads = []
    for _ in range(3):
        kx = x.to(DEV, torch.bfloat16).requires_grad_()
        ka = a.to(DEV, torch.bfloat16).requires_grad_()
        kb = b.to(DEV, torch.bfloat16).requires_grad_()
        y, _ = moc_triton(kx, ka, kb, activation="silu")
        y.backward(dy.to(DEV, torch.bfloat16))
        grads.append((y.detach(), kx.grad, ka.grad, kb.grad))
    for other in grads[1:]:
        for u, v in zip(grads[0], other):
            assert torch.equal(u, v)


def test_module_decode_matches_full_forward():
    """Config-4 pattern at reduced size: prefill through forward(output_final_state),
    then single-token steps; y within tolerance of the full forward, cache
    bit-exact."""
    torch.manual_seed(0)
    Bd, Dd, Z, Kd, S, Tp, Ts = 8, 256, 64, 16, 4, 40, 24
    m = MoC(Dd, Z, S, Kd, activation="silu")
    g = gen(9)
    with torch.no_grad():
        m.router.copy_(randn(g, Kd, Z, scale=0.02))
    m = m.to(DEV, torch.bfloat16)
    x = randn(g, Bd, Tp + Ts, Dd).to(DEV, torch.bfloat16)
    z = randn(g, Bd, Tp + Ts, Z).to(DEV, torch.bfloat16)
    with torch.no_grad():
        y_pre, cache = m(x[:, :Tp], z[:, :Tp], output_final_state=True)
        steps = []
        for t in range(Tp, Tp + Ts):
            y, c2 = m.step(x[:, t:t + 1], z[:, t:t + 1], cache=cache, output_final_state=True)
            assert c2 is cache
            steps.append(y)
        y_full, _ = m(x, z)
    assert torch.equal(cache, x[:, -S:].transpose(1, 2))
    assert_close("decode y", torch.cat(steps, 1), y_full[:, Tp:], torch.bfloat16)
    assert_close("prefill y", y_pre, y_full[:, :Tp], torch.bfloat16)
    with torch.no_grad():
        y0, c0 = m.step(x[:, :1], z[:, :1])   # cache=None: zeros are created
    assert c0 is None
    assert_close("first step", y0, y_full[:, :1], torch.bfloat16)


def test_module_varlen_routed():
    torch.manual_seed(0)
    Z = 32
    m = MoC(D, Z, 4, K, router_activation="exp", init_std=0.1)
    g = gen(11)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.1))
    m = m.to(DEV)
    cu = _cu(VARLEN_LENGTHS).to(DEV)
    N = sum(VARLEN_LENGTHS)
    x = randn(g, N, D).to(DEV).requires_grad_()
    z = randn(g, N, Z).to(DEV).requires_grad_()
    y, st = m(x, z, cu_seqlens=cu, max_seqlen=31)
    assert st is None
    y.sum().backward()
    rz = z.detach().requires_grad_()
    rr = m.router.detach().requires_grad_()
    rx = x.detach().cpu().requires_grad_()
    ry = O.moc_varlen_ref(rx, O.route(torch.nn.functional.linear(rz, rr).cpu(), "exp"),
                          m.conv_bases.detach().cpu(), cu.cpu())
    ry.sum().backward()
    assert_close("y", y, ry, torch.float32)
    assert_close("dx", x.grad, rx.grad, torch.float32)
    assert_close("dz", z.grad, rz.grad, torch.float32)
    assert_close("drouter", m.router.grad, rr.grad, torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_varlen_with_cu_seqlens_cpu_and_chunk_indices(dtype):
    """Valid packed calls that pass cu_seqlens_cpu or chunk_indices
    (moc/api.py:117-128): checked as the reference checks them, then the same
    results as the call without them (bit for bit) and as the oracle."""
    from moc import ops
    g, _, _, _, xv, av, dyv = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1).to(DEV, dtype)
    cu = _cu(VARLEN_LENGTHS).to(DEV)
    extra = [dict(), dict(cu_seqlens_cpu=cu.cpu()),
             dict(chunk_indices=ops.prepare_chunk_indices(cu)),
             dict(cu_seqlens_cpu=cu.cpu().long(), chunk_indices=ops.prepare_chunk_indices(cu, 64, cu.cpu()))]
    outs = []
    for kw in extra:
        kx = xv.to(DEV, dtype).requires_grad_()
        ka = av.to(DEV, dtype).requires_grad_()
        kb = b.clone().requires_grad_()
        y, _ = moc_triton(kx, ka, kb, cu_seqlens=cu, max_seqlen=max(VARLEN_LENGTHS),
                          activation="silu", **kw)
        y.backward(dyv.to(DEV, dtype))
        outs.append((y.detach(), kx.grad, ka.grad, kb.grad))
    for other in outs[1:]:
        for u, v in zip(outs[0], other):
            assert torch.equal(u, v)
    rx, ra, rb = O.reference_inputs(xv.to(dtype), av.to(dtype), b, dtype)
    ref = O.moc_varlen_grads_ref(rx, ra, rb, cu.cpu(), dyv.to(dtype).float(), "silu")
    for n, u, r in zip(("y", "dx", "dalpha", "dbasis"), outs[0], ref):
        assert_close(n, u, r, dtype)


def test_module_varlen_with_cu_seqlens_cpu_and_chunk_indices():
    """The bf16 module on the router kernels (one autograd node) with
    cu_seqlens_cpu / chunk_indices: the same results as without them."""
    from moc import ops
    torch.manual_seed(0)
    Z = 64
    m = MoC(D, Z, 4, 16, activation="silu", init_std=0.1)
    g = gen(17)
    with torch.no_grad():
        m.router.copy_(randn(g, 16, Z, scale=0.1))
    m = m.to(DEV, torch.bfloat16)
    cu = _cu(VARLEN_LENGTHS).to(DEV)
    N = sum(VARLEN_LENGTHS)
    x = randn(g, 1, N, D).to(DEV, torch.bfloat16)
    z = randn(g, 1, N, Z).to(DEV, torch.bfloat16)
    outs = []
    for kw in (dict(), dict(cu_seqlens_cpu=cu.cpu()), dict(chunk_indices=ops.prepare_chunk_indices(cu))):
        m.zero_grad(set_to_none=True)
        xi, zi = x.clone().requires_grad_(), z.clone().requires_grad_()
        y, st = m(xi, zi, cu_seqlens=cu, max_seqlen=max(VARLEN_LENGTHS), **kw)
        assert st is None and y.shape == x.shape
        y.float().square().sum().backward()
        outs.append((y.detach(), xi.grad, zi.grad, m.router.grad, m.conv_bases.grad))
    for other in outs[1:]:
        for u, v in zip(outs[0], other):
            assert torch.equal(u, v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("varlen", [False, True])
def test_broadcast_dy_matches_materialised(dtype, varlen):
    """The gradient of y.sum() reaches the backward as one row broadcast over
    every token (stride 0); the kernels read that row in place (row stride 0)
    instead of a copied [n_tokens, D] tensor.  dx, dalpha and dbasis equal those
    from the materialised ones tensor bit for bit, and the oracle's."""
    g, x, a, _, xv, av, _ = _verify_inputs()
    b = randn(g, K, 4, D, scale=0.1).to(DEV, dtype)
    xs, as_ = (xv, av) if varlen else (x, a)
    kw = dict(cu_seqlens=_cu(VARLEN_LENGTHS).to(DEV), max_seqlen=31) if varlen else {}

    def run(broadcast):
        kx = xs.to(DEV, dtype).requires_grad_()
        ka = as_.to(DEV, dtype).requires_grad_()
        kb = b.clone().requires_grad_()
        y, _ = moc_triton(kx, ka, kb, activation="silu", **kw)
        if broadcast:
            y.sum().backward()
        else:
            y.backward(torch.ones_like(y))
        return kx.grad, ka.grad, kb.grad

    got, mat = run(True), run(False)
    for n, u, v in zip(("dx", "dalpha", "dbasis"), got, mat):
        assert torch.equal(u, v), n
    rx, ra, rb = O.reference_inputs(xs.to(dtype), as_.to(dtype), b, dtype)
    ones = torch.ones(xs.shape)
    ref = (O.moc_varlen_grads_ref(rx, ra, rb, kw["cu_seqlens"].cpu(), ones, "silu") if varlen
           else O.moc_grads_ref(rx, ra, rb, ones, "silu"))
    for n, u, r in zip(("dx", "dalpha", "dbasis"), got, ref[1:]):
        assert_close(n, u, r, dtype)


@pytest.mark.parametrize("form", ["element", "row"])
@pytest.mark.parametrize("shape", ["fused", "two_pass", "generic", "varlen"])
def test_broadcast_dy_forms_match_materialised(form, shape):
    """dy passed as one element for every token and channel (row stride -1, the
    expanded gradient of y.sum()) or as one row for every token (row stride 0)
    gives the results of the same dy as a contiguous tensor, bit for bit: on the
    fused matrix-core pass (4 taps, 16 routes, SiLU), the two-pass form (8 taps,
    32 routes, no activation), the generic kernels and a varlen call."""
    from moc import _lib, ops
    S, Kr, act, Dd = (8, 32, 0, 256) if shape == "two_pass" else (4, 16, 1, 192)
    g = gen(77)
    N = 300
    x = randn(g, N, Dd, scale=0.5).to(DEV, torch.bfloat16)
    a = torch.softmax(randn(g, N, Kr), -1).to(DEV, torch.bfloat16)
    b = randn(g, Kr, S, Dd, scale=0.1).to(DEV, torch.bfloat16)
    lead = (N,) if shape == "varlen" else (2, N // 2)   # packed [N, D] or fixed [B, T, D]
    x = x.reshape(*lead, Dd)
    if form == "element":
        dy = (randn(g, 1, scale=0.5) + 1.0).to(DEV, torch.bfloat16).reshape(()).expand(*lead, Dd)
    else:
        dy = randn(g, Dd, scale=0.5).to(DEV, torch.bfloat16).expand(*lead, Dd)
    assert dy.stride()[0] == 0
    assert ops.dy_operand(dy, torch.bfloat16)[1] == (-1 if form == "element" else 0)
    kw = dict(cu_seqlens=_cu([120, 7, 173]).to(DEV)) if shape == "varlen" else {}
    path = _lib.PATH_GENERIC if shape == "generic" else _lib.PATH_AUTO
    with _lib.kernel_path(path):
        got = ops.launch_backward(x, a, b, dy, activation_flag=act, need_x=True, **kw)
        ref = ops.launch_backward(x, a, b, dy.contiguous(), activation_flag=act, need_x=True, **kw)
    for n, u, v in zip(("dx", "dalpha", "dbasis"), got, ref):
        assert torch.equal(u, v), n


def test_moc_triton_name_is_hip_path():
    assert moc.moc_triton is moc.moc_hip


@pytest.mark.parametrize("route", ["softmax", "exp"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_routed_function_dlogits(route, dtype):
    """The logits-input autograd function directly: y, dx, d(logits), dbasis."""
    from moc import api
    g = gen(21)
    x = randn(g, B, T, D, scale=0.5).to(DEV, dtype)
    lg = randn(g, B, T, K).to(DEV, dtype)
    b = randn(g, K, 4, D, scale=0.1).to(DEV, dtype)
    dy = randn(g, B, T, D).to(DEV, dtype)
    xx, ll, bb = (t.clone().requires_grad_() for t in (x, lg, b))
    y = api._MoCRoutedFunction.apply(xx, ll, bb, "silu", route, None, None, None, None)
    y.backward(dy)
    rx = x.float().cpu().requires_grad_()
    rl = lg.float().cpu().requires_grad_()
    rb = b.float().cpu().requires_grad_()
    ry = O.moc_ref(rx, O.route(rl, route, out_dtype=dtype), rb, "silu")
    ry.backward(dy.float().cpu())
    assert_close("y", y, ry, dtype)
    assert_close("dx", xx.grad, rx.grad, dtype)
    assert_close("dlogits", ll.grad, rl.grad, dtype)
    assert_close("dbasis", bb.grad, rb.grad, dtype)


@pytest.mark.parametrize("Kr,S,route", [(48, 4, "softmax"), (64, 4, "exp"), (64, 8, "softmax"),
                                        (40, 2, "softmax")])
def test_routed_function_64_routes(Kr, S, route):
    """More than 32 routes (bf16; K in (32, 64] padded to 64 in the kernels):
    the logits-input function's y, dx, d(logits) and dbasis against the oracle,
    and the same through the generic kernels."""
    from moc import _lib, api
    dtype = torch.bfloat16
    g = gen(Kr + S)
    Bn, Tn, Dn = 2, 150, 192
    x = randn(g, Bn, Tn, Dn, scale=0.5).to(DEV, dtype)
    lg = randn(g, Bn, Tn, Kr).to(DEV, dtype)
    b = randn(g, Kr, S, Dn, scale=0.1).to(DEV, dtype)
    dy = randn(g, Bn, Tn, Dn).to(DEV, dtype)

    def run():
        xx, ll, bb = (t.clone().requires_grad_() for t in (x, lg, b))
        y = api._MoCRoutedFunction.apply(xx, ll, bb, "silu", route, None, None, None, None)
        y.backward(dy)
        return y.detach(), xx.grad, ll.grad, bb.grad

    rx = x.float().cpu().requires_grad_()
    rl = lg.float().cpu().requires_grad_()
    rb = b.float().cpu().requires_grad_()
    ry = O.moc_ref(rx, O.route(rl, route, out_dtype=dtype), rb, "silu")
    ry.backward(dy.float().cpu())
    got = run()
    with _lib.kernel_path(_lib.PATH_GENERIC):
        other = run()
    for n, u, v, r in zip(("y", "dx", "dlogits", "dbasis"), got, other,
                          (ry, rx.grad, rl.grad, rb.grad)):
        assert_close(n, u, r, dtype)
        assert_close(n + " (generic)", v, r, dtype)


@pytest.mark.parametrize("T2,S", [(10, 4), (2, 4), (3, 4), (7, 2), (5, 8), (40, 3), (4, 8)])
def test_prefill_matches_concatenated_history(T2, S):
    """Prefill from a cache against the reference's formulation of it
    (moc/api.py:299-307: the cache prepended to x, zero weights prepended to
    alpha, the first S outputs dropped) on the same kernels: y bit for bit
    (each token's output depends only on its own window); dx, dalpha, dbasis
    and dcache within the bf16 rule (partial sums are rounded separately)."""
    Bn, Dn, Kn, dtype = 3, 192, 16, torch.bfloat16
    g = gen(T2 * 10 + S)
    x = randn(g, Bn, T2, Dn).to(DEV, dtype)
    a = torch.softmax(randn(g, Bn, T2, Kn), -1).to(DEV, dtype)
    b = randn(g, Kn, S, Dn, scale=0.1).to(DEV, dtype)
    c = randn(g, Bn, Dn, S).to(DEV, dtype)
    dy = randn(g, Bn, T2, Dn, scale=0.1).to(DEV, dtype)

    def run(native):
        xi, ai, bi, ci = (t.clone().requires_grad_() for t in (x, a, b, c))
        if native:
            y, st = moc_triton(xi, ai, bi, cache=ci, output_final_state=True, activation="silu")
        else:
            hist = ci.transpose(1, 2)
            y, _ = moc_triton(torch.cat((hist, xi), 1),
                              torch.cat((ai.new_zeros(Bn, S, Kn), ai), 1), bi, activation="silu")
            y = y[:, S:]
            st = None
        y.backward(dy)
        return y.detach(), xi.grad, ai.grad, bi.grad, ci.grad, st

    got, ref = run(True), run(False)
    assert torch.equal(got[0], ref[0])
    for name, u, v in zip(("dx", "dalpha", "dbasis", "dcache"), got[1:5], ref[1:5]):
        assert_close(name, u, v.float(), dtype)
    full = torch.cat((c.transpose(1, 2), x), 1)
    assert torch.equal(got[5], O.final_state(full, None, S))


def test_module_prefill_from_cache_matches_full_forward():
    """MoC.forward continuing from a cache (router logits path): the second
    chunk's y within tolerance of the full-sequence forward, final cache bit-exact."""
    torch.manual_seed(0)
    Z = 64
    m = MoC(D, Z, 4, K, activation="silu", init_std=0.1)
    g = gen(13)
    with torch.no_grad():
        m.router.copy_(randn(g, K, Z, scale=0.1))
    m = m.to(DEV, torch.bfloat16)
    x = randn(g, B, T, D).to(DEV, torch.bfloat16)
    z = randn(g, B, T, Z).to(DEV, torch.bfloat16)
    t1 = T // 3
    with torch.no_grad():
        y_full, st_full = m(x, z, output_final_state=True)
        _, cache = m(x[:, :t1], z[:, :t1], output_final_state=True)
        y2, st2 = m(x[:, t1:], z[:, t1:], cache=cache, output_final_state=True)
    assert_close("prefill y", y2, y_full[:, t1:].float(), torch.bfloat16)
    assert torch.equal(st2, st_full)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kernels_match_golden(dtype):
    """The committed golden vectors (tests/golden/moc_golden.npz: the verify.py
    matrix class, fixed and varlen, S 2 / 4, plain / SiLU): y and the gradients
    of x, alpha and basis from the kernels against the stored fp64 oracle
    results, under the tolerance rule of the dtype."""
    from tests.test_oracle import golden_cases
    for name, S, act, a in golden_cases():
        x = torch.from_numpy(a["x"]).to(DEV, dtype).requires_grad_()
        al = torch.from_numpy(a["alpha"]).to(DEV, dtype).requires_grad_()
        b = torch.from_numpy(a["basis"]).to(DEV, dtype).requires_grad_()
        dy = torch.from_numpy(a["dy"]).to(DEV, dtype)
        if "cu_seqlens" in a:
            cu = torch.from_numpy(a["cu_seqlens"]).to(DEV)
            lengths = (cu[1:] - cu[:-1]).tolist()
            y, _ = moc_triton(x, al, b, activation=act, cu_seqlens=cu, max_seqlen=max(lengths))
        else:
            y, _ = moc_triton(x, al, b, activation=act)
        y.backward(dy)
        for key, got in (("y", y), ("dx", x.grad), ("dalpha", al.grad), ("dbasis", b.grad)):
            assert_close(f"{name} {key}", got, torch.from_numpy(a[key]), dtype)


def test_longest_token_axis_ends_match_oracle():
    """The longest token axis the backward entry accepts (65535 * 256 tokens;
    D 64, K 16, S 4, SiLU, bf16, loss y.sum()).  Every output of a token
    depends only on the S-1 tokens before it and the S-1 after it, so the first
    and last 1024 tokens are checked against the oracle run on those windows
    (the last one with its S-1 rows of history); dbasis, a sum over the whole
    axis, is checked to be finite."""
    S, Kr, Dl = 4, 16, 64
    N = 65535 * 256
    gd = torch.Generator(device=DEV).manual_seed(5)
    x = (torch.randn(1, N, Dl, generator=gd, device=DEV) * 0.5).to(torch.bfloat16).requires_grad_()
    a = torch.softmax(torch.randn(1, N, Kr, generator=gd, device=DEV), -1).to(torch.bfloat16)
    a.requires_grad_()
    b = (torch.randn(Kr, S, Dl, generator=gd, device=DEV) * 0.2).to(torch.bfloat16).requires_grad_()
    y, _ = moc_triton(x, a, b, activation="silu")
    y.sum().backward()
    torch.cuda.synchronize()
    assert torch.isfinite(b.grad.float()).all()
    L, H = 1024, S - 1
    for lo, keep in ((0, 0), (N - L - H, H)):
        hi = min(lo + L + H, N)
        rx, ra, rb = O.reference_inputs(x[:, lo:hi], a[:, lo:hi], b, torch.bfloat16)
        dy = torch.ones(1, hi - lo, Dl)
        ry, rdx, rda, _ = O.moc_grads_ref(rx, ra, rb, dy, "silu")
        rows = slice(keep, keep + L)
        sl = slice(lo + keep, lo + keep + L)
        assert_close(f"y[{lo}]", y[:, sl], ry[:, rows], torch.bfloat16)
        assert_close(f"dx[{lo}]", x.grad[:, sl], rdx[:, rows], torch.bfloat16)
        assert_close(f"dalpha[{lo}]", a.grad[:, sl], rda[:, rows], torch.bfloat16)
