"""Grouped layer launches (moc_forward_layers / moc_backward_layers) against the
single-layer entries, through the C ABI: every layer's y, dx, dalpha and dbasis
bit for bit.  The grouped kernels run each layer's own grid inside one launch,
so each workgroup does exactly the work of the single-layer launch; layers may
differ in K and activation (one forward launch; one backward stage-1 launch
per route count, and per activation where a two-pass form runs: with SiLU
each layer's g goes through its own workspace); layers that cannot share one
launch (fp32, or the generic kernels) run one by one inside the same
entry."""
from __future__ import annotations

import itertools

import pytest
import torch

from moc import _lib, ops
from tests._parity import gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (layer dims, K, S, activation, routing codes, need_x per layer, dtype); K and
# the activation are one value for every layer or a list with one per layer
CASES = [
    ([512, 256, 128], 16, 4, 1, [3, 4, 3], [True, True, True], torch.bfloat16),   # fused, tiered
    ([512, 128, 128], 32, 8, 0, [4, 4, 3], [True, False, True], torch.bfloat16),  # dx + taps passes
    ([256, 192], 32, 4, 1, [0, 3], [True, True], torch.bfloat16),                 # route halves
    ([128, 64, 96, 32], 8, 2, 0, [0, 0, 4, 3], [False, True, True, True], torch.bfloat16),
    ([96, 64], 8, 2, 1, [0, 0], [True, True], torch.float32),                     # one by one
    ([256, 128], 16, 6, 1, [3, 3], [True, True], torch.bfloat16),                 # 6 taps
    ([128, 192, 64], 32, 7, 0, [4, 0, 3], [True, True, False], torch.bfloat16),  # 7 taps, halves
    ([256, 128], 64, 4, 1, [3, 0], [True, True], torch.bfloat16),                 # 64 routes
    ([256, 128], 32, 6, 0, [4, 3], [True, False], torch.bfloat16),               # 6 taps, two passes
    ([192, 64], 32, 4, 0, [0, 4], [True, True], torch.bfloat16),                  # 4 taps, two passes
    ([128, 64], 16, 8, 0, [0, 3], [True, True], torch.bfloat16),                  # 16 routes, two passes
    # per-layer activation and K
    ([512, 256, 128], 16, 4, [1, 0, 1], [3, 4, 3], [True, True, False], torch.bfloat16),  # four-wave pass
    ([256, 128], 16, 6, [1, 0], [3, 0], [True, True], torch.bfloat16),           # fused pass, 6 taps
    ([256, 192], 32, 3, [0, 1], [4, 3], [True, True], torch.bfloat16),           # route halves
    ([256, 128, 192], [16, 32, 16], 4, [1, 0, 0], [3, 4, 0], [True, True, True],
     torch.bfloat16),                                                            # 16 | 32 (two passes)
    ([128, 256], [16, 32], 3, [0, 1], [0, 3], [False, True], torch.bfloat16),    # 16 | 32 with SiLU
    ([128, 64, 96], [32, 16, 12], 5, [1, 1, 0], [3, 3, 4], [True, True, True], torch.bfloat16),
    ([128, 64], 32, 8, [0, 1], [3, 3], [True, True], torch.bfloat16),            # two forms, two launches
    # SiLU two passes (g through each layer's workspace), grouped
    ([512, 256, 128], 32, 6, 1, [3, 4, 3], [True, True, False], torch.bfloat16),
    ([256, 192], 16, 8, 1, [3, 0], [False, True], torch.bfloat16),
    ([256, 128, 64], [32, 16, 32], 8, [1, 1, 0], [3, 3, 4], [True, False, True], torch.bfloat16),
    # 64 routes in two passes (taps pass in route halves), grouped
    ([256, 192], 64, 6, 0, [3, 4], [True, False], torch.bfloat16),
    ([128, 256], [64, 32], 5, [1, 1], [3, 0], [True, True], torch.bfloat16),
]


def _per_layer(v, n):
    return list(v) if isinstance(v, (list, tuple)) else [v] * n


def _inputs(dims, K, S, dtype, lead, seed):
    g = gen(seed)
    ks = _per_layer(K, len(dims))
    xs = [randn(g, *lead, D, scale=0.5).to(DEV, dtype) for D in dims]
    ws = [torch.softmax(randn(g, *lead, k), -1).to(DEV, dtype) for k in ks]
    bs = [randn(g, k, S, D, scale=0.1).to(DEV, dtype) for k, D in zip(ks, dims)]
    dys = [randn(g, *lead, D).to(DEV, dtype) for D in dims]
    return xs, ws, bs, dys


def _check(dims, K, S, act, codes, need, dtype, lead, cu=None, generic=False):
    xs, ws, bs, dys = _inputs(dims, K, S, dtype, lead, sum(dims) + sum(_per_layer(K, 1)) + S)
    acts = _per_layer(act, len(dims))
    ctx = _lib.kernel_path(_lib.PATH_GENERIC) if generic else _lib.kernel_path(_lib.PATH_AUTO)
    with ctx:
        ys = ops.launch_forward_layers(xs, ws, bs, activation_flags=acts, routings=codes,
                                       cu_seqlens=cu)
        grads = ops.launch_backward_layers(xs, ws, bs, dys, activation_flags=acts, routings=codes,
                                           need_xs=need, cu_seqlens=cu)
        for i in range(len(dims)):
            y1 = ops.launch_forward(xs[i], ws[i], bs[i], activation_flag=acts[i], routing=codes[i],
                                    cu_seqlens=cu)
            g1 = ops.launch_backward(xs[i], ws[i], bs[i], dys[i], activation_flag=acts[i],
                                     need_x=need[i], routing=codes[i], cu_seqlens=cu)
            assert torch.equal(ys[i], y1), f"y[{i}]"
            assert (grads[i][0] is None) == (not need[i])
            for n, u, v in zip(("dx", "dalpha", "dbasis"), grads[i], g1):
                if u is not None:
                    assert torch.equal(u, v), f"{n}[{i}]"


@pytest.mark.parametrize("dims,K,S,act,codes,need,dtype", CASES)
def test_layers_match_single_layer_entries(dims, K, S, act, codes, need, dtype):
    _check(dims, K, S, act, codes, need, dtype, (3, 211))


@pytest.mark.parametrize("dims,K,S,act,codes,need,dtype", CASES[:3] + CASES[11:15] + CASES[-5:])
def test_layers_match_single_layer_entries_packed(dims, K, S, act, codes, need, dtype):
    lengths = [1, 90, 3, 250, 17, 199, 73]
    cu = torch.tensor([0, *itertools.accumulate(lengths)], dtype=torch.int32, device=DEV)
    _check(dims, K, S, act, codes, need, dtype, (sum(lengths),), cu=cu)


def test_layers_on_generic_kernels():
    """With the generic kernels forced, the layers run one by one on them."""
    _check([96, 64], 16, 4, 1, [3, 0], [True, True], torch.bfloat16, (2, 77), generic=True)


def test_layers_broadcast_dy():
    """A broadcast-row dy (the gradient of y.sum()) in a grouped backward."""
    dims, K, S = [256, 128], 16, 4
    xs, ws, bs, _ = _inputs(dims, K, S, torch.bfloat16, (2, 300), 5)
    dys = [torch.ones((), device=DEV, dtype=torch.bfloat16).expand(2, 300, D) for D in dims]
    got = ops.launch_backward_layers(xs, ws, bs, dys, activation_flags=[1, 1], routings=[3, 3],
                                     need_xs=[True, True])
    for i in range(2):
        ref = ops.launch_backward(xs[i], ws[i], bs[i], torch.ones_like(xs[i]), activation_flag=1,
                                  need_x=True, routing=3)
        for u, v in zip(got[i], ref):
            assert torch.equal(u, v)
