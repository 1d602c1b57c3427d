"""moc_backward_noalloc against moc_backward, through the C ABI.

The no-allocation entry runs the same kernels as moc_backward on the library's
own device scratch instead of a caller workspace, so its results must equal
moc_backward's bit for bit.  Two calls in a row, the second on a smaller
problem (the scratch keeps the first call's contents), plus a packed call.
"""
from __future__ import annotations

import itertools

import pytest
import torch

from moc import _lib
from tests._parity import gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, N, D, K, S, dtype, weights):
    g = gen(seed)
    x = randn(g, N, D, scale=0.5).to(DEV, dtype)
    a = torch.softmax(randn(g, N, K), -1).to(DEV, dtype) if weights else randn(g, N, K).to(DEV, dtype)
    b = randn(g, K, S, D, scale=0.1).to(DEV, dtype)
    dy = randn(g, N, D).to(DEV, dtype)
    return x, a, b, dy


def _call(noalloc, x, a, b, dy, dy_stride, act, routing, cu=None, seq_len=None):
    """(dx, dalpha, dbasis) of one C-ABI backward call on the current stream."""
    L = _lib.lib()
    N, D = x.shape[0], b.shape[2]
    K, S = b.shape[0], b.shape[1]
    dx = torch.full_like(x, float("nan"))
    da = torch.full_like(a, float("nan"))
    db = torch.full_like(b, float("nan"))
    dt = _lib.dtype_code(x.dtype)
    seq = (None, 0, 0, N, seq_len) if cu is None else (
        cu.data_ptr(), int(cu.dtype == torch.int64), cu.numel() - 1, N, 0)
    head = (x.data_ptr(), a.data_ptr(), b.data_ptr(), dy.data_ptr(), dy_stride,
            dx.data_ptr(), da.data_ptr(), db.data_ptr(), *seq, D, K, S, dt, dt, dt, act, routing)
    stream = _lib.stream_ptr(x.device)
    if noalloc:
        rc = L.moc_backward_noalloc(*head, stream)
    else:
        nbytes = L.moc_backward_workspace_bytes(N, D, K, S, dt, routing)
        assert 0 < nbytes <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        rc = L.moc_backward(*head, ws.data_ptr(), nbytes, stream)
    _lib.check(rc, "moc_backward_noalloc" if noalloc else "moc_backward")
    torch.cuda.synchronize()
    return dx, da, db


def _same(label, got, ref):
    for n, u, v in zip(("dx", "dalpha", "dbasis"), got, ref):
        assert not torch.isnan(v).any(), f"{label} {n}: reference left unwritten elements"
        assert torch.equal(u, v), f"{label} {n}: noalloc differs from moc_backward"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_backward_matches_workspace_backward(dtype):
    # first call: 2 x 2048 tokens, D 1024, K 16, S 4, SiLU, softmax weights given
    T1 = 2048
    x, a, b, dy = _inputs(1, 2 * T1, 1024, 16, 4, dtype, True)
    ref = _call(False, x, a, b, dy, 1024, 1, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=T1)
    got = _call(True, x, a, b, dy, 1024, 1, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=T1)
    _same("call 1", got, ref)
    # second call, smaller: 3 x 100 tokens, D 256, K 8, S 2, no activation,
    # alpha given, dy one broadcast row (row stride 0)
    x, a, b, dy = _inputs(2, 300, 256, 8, 2, dtype, True)
    row = dy[:1].contiguous()
    ref = _call(False, x, a, b, row, 0, 0, _lib.ROUTE_ALPHA, seq_len=100)
    got = _call(True, x, a, b, row, 0, 0, _lib.ROUTE_ALPHA, seq_len=100)
    _same("call 2", got, ref)
    # a packed call (logits routed by exp in the kernels)
    lengths = [1, 40, 3, 77, 59]
    cu = torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32, device=DEV)
    x, a, b, dy = _inputs(3, sum(lengths), 192, 12, 3, dtype, False)
    ref = _call(False, x, a, b, dy, 192, 1, _lib.ROUTE_EXP, cu=cu)
    got = _call(True, x, a, b, dy, 192, 1, _lib.ROUTE_EXP, cu=cu)
    _same("packed", got, ref)


@pytest.mark.parametrize("D,K,S,dtype,act", [
    (197, 16, 4, torch.bfloat16, 1),    # odd channel count: the padded copy
    (192, 32, 12, torch.float32, 1),    # fp32 route parts of 16 routes
    (128, 48, 4, torch.float32, 0),     # fp32 route halves of 32 routes
    (192, 32, 12, torch.bfloat16, 1),   # bf16 route chunks past 8 taps
    (192, 64, 6, torch.bfloat16, 0),    # 64 routes in two passes, taps in route halves
])
def test_noalloc_other_backward_forms(D, K, S, dtype, act):
    """The backward forms that carve more of the workspace (padded copies, route
    parts and chunks, route-half taps) on the scratch: bit for bit with
    moc_backward, on a second call after a larger first one."""
    x, a, b, dy = _inputs(5, 2 * 300, D, K, S, dtype, True)
    ref = _call(False, x, a, b, dy, D, act, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=300)
    got = _call(True, x, a, b, dy, D, act, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=300)
    _same("call 1", got, ref)
    x, a, b, dy = _inputs(6, 2 * 77, D, K, S, dtype, True)
    ref = _call(False, x, a, b, dy, D, act, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=77)
    got = _call(True, x, a, b, dy, D, act, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=77)
    _same("call 2", got, ref)


def test_noalloc_rejects_a_problem_beyond_its_scratch():
    L = _lib.lib()
    N, D = 1 << 20, 2048
    assert L.moc_backward_workspace_bytes(N, D, 16, 4, _lib.DT_BF16, 3) > _lib.NOALLOC_SCRATCH_BYTES
    p = 0x1000   # never dereferenced: the size check comes first
    rc = L.moc_backward_noalloc(p, p, p, p, D, p, p, p, None, 0, 0, N, 4096, D, 16, 4, 1, 1, 1, 1,
                                3, _lib.stream_ptr(torch.device(DEV)))
    assert rc == -3 and b"moc_backward_noalloc holds" in L.moc_last_error()


def test_noalloc_backward_replays_in_a_captured_graph():
    """The caller the no-allocation entry is for: a HIP graph.  One eager call
    first (the library resolves its scratch address on a device's first call),
    then the call captured on a side stream and the graph replayed three times,
    with new dy values written eagerly between replays; every replay must equal
    the eager moc_backward on the same inputs bit for bit."""
    L = _lib.lib()
    T1 = 1024
    x, a, b, dy = _inputs(4, 2 * T1, 512, 16, 4, torch.bfloat16, True)
    dt = _lib.dtype_code(x.dtype)
    N, D, K, S = x.shape[0], b.shape[2], b.shape[0], b.shape[1]
    _call(True, x, a, b, dy, D, 1, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=T1)
    dx = torch.empty_like(x)
    da = torch.empty_like(a)
    db = torch.empty_like(b)
    head = (x.data_ptr(), a.data_ptr(), b.data_ptr(), dy.data_ptr(), D, dx.data_ptr(), da.data_ptr(),
            db.data_ptr(), None, 0, 0, N, T1, D, K, S, dt, dt, dt, 1, _lib.ROUTE_SOFTMAX_WEIGHTS)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        rc = L.moc_backward_noalloc(*head, _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc, "moc_backward_noalloc (captured)")
    g = gen(40)
    for rep in range(3):
        dy.copy_(randn(g, N, D).to(DEV, dy.dtype))
        for t in (dx, da, db):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _call(False, x, a, b, dy, D, 1, _lib.ROUTE_SOFTMAX_WEIGHTS, seq_len=T1)
        _same(f"replay {rep}", (dx, da, db), ref)
