"""Host-side behaviour of the ``moc`` package that needs no GPU: validation
(exception types and messages of the reference, moc/api.py:18-92, 209-215,
311-314, 410-413), module parameters and init, optim helpers, chunk indices and
final-state bookkeeping."""
from __future__ import annotations

import math

import pytest
import torch

import moc
from moc import api, ops


def test_exports():
    for name in ("MoC", "moc_triton", "moc_fan_in_std", "match_lr_to_init_std",
                 "match_weight_decay_to_lr"):
        assert hasattr(moc, name)
    assert moc.moc_hip is moc.moc_triton


def test_optim_helpers_readme_values():
    std = moc.moc_fan_in_std(k=16, kernel_size=4)
    assert std == pytest.approx(1.1547005, rel=1e-6)
    lr = moc.match_lr_to_init_std(std, reference_std=0.01, reference_lr=1e-3)
    assert lr == pytest.approx(0.1154700, rel=1e-6)
    assert moc.match_weight_decay_to_lr(lr, reference_lr=1e-3, reference_weight_decay=0.1) == \
        pytest.approx(0.000866025, rel=1e-5)
    assert moc.match_lr_to_init_std(0.002) == pytest.approx(1e-3)


def test_activation_flags():
    assert api.activation_flag(None) == 0
    assert api.activation_flag("silu") == 1 and api.activation_flag("swish") == 1
    with pytest.raises(ValueError, match="unsupported activation: gelu"):
        api.activation_flag("gelu")
    api.check_router_activation("softmax")
    api.check_router_activation("exp")
    with pytest.raises(ValueError, match="unsupported router activation"):
        api.check_router_activation("sigmoid")


def test_module_parameters_and_init():
    torch.manual_seed(0)
    m = moc.MoC(dim=64, z_dim=32, kernel_size=4, k=8)
    assert tuple(m.conv_bases.shape) == (8, 4, 64)
    assert tuple(m.router.shape) == (8, 32)
    assert torch.count_nonzero(m.router) == 0
    bound = math.sqrt(8 / 12) * math.sqrt(3)
    assert m.conv_bases.abs().max() <= bound
    assert m.conv_bases.abs().max() > 0.9 * bound
    assert m.state_size == 64 * 4
    m2 = moc.MoC(dim=16, z_dim=16, kernel_size=2, k=4, init_std=0.002)
    assert m2.conv_bases.abs().max() <= 0.002 * math.sqrt(3)
    assert set(dict(m.named_parameters())) == {"conv_bases", "router"}
    with pytest.raises(ValueError):
        moc.MoC(8, 8, 4, 2, activation="relu")
    with pytest.raises(ValueError):
        moc.MoC(8, 8, 4, 2, router_activation="sigmoid")


def test_cpu_tensors_are_rejected():
    x = torch.zeros(1, 4, 8)
    a = torch.zeros(1, 4, 2)
    b = torch.zeros(2, 4, 8)
    with pytest.raises(ValueError, match="must all be CUDA tensors"):
        moc.moc_triton(x, a, b)
    with pytest.raises(ValueError, match="unsupported activation"):
        moc.moc_triton(x, a, b, activation="tanh")


@pytest.fixture
def no_device_check(monkeypatch):
    """Validators minus the CUDA-residency test, so the shape / dtype rules can
    be exercised on CPU tensors."""
    orig = api.check_common_dtypes

    def check(x, alpha, basis):
        if x.dtype not in api.SUPPORTED_DTYPES:
            raise TypeError(f"unsupported x dtype: {x.dtype}")
        if not alpha.is_floating_point():
            raise TypeError(f"alpha must be floating point, got {alpha.dtype}")
        if not basis.is_floating_point():
            raise TypeError(f"basis must be floating point, got {basis.dtype}")

    monkeypatch.setattr(api, "check_common_dtypes", check)
    yield
    monkeypatch.setattr(api, "check_common_dtypes", orig)


def test_fixed_shape_validation(no_device_check):
    x = torch.zeros(2, 5, 8)
    a = torch.zeros(2, 5, 3)
    b = torch.zeros(3, 4, 8)
    assert api.check_fixed_inputs(x, a, b) == (2, 5, 8, 3, 4)
    with pytest.raises(TypeError, match="unsupported x dtype"):
        api.check_fixed_inputs(x.half(), a, b)
    with pytest.raises(TypeError, match="alpha must be floating point"):
        api.check_fixed_inputs(x, a.long(), b)
    with pytest.raises(TypeError, match="basis must be floating point"):
        api.check_fixed_inputs(x, a, b.int())
    with pytest.raises(ValueError, match="ranks 3/3/3"):
        api.check_fixed_inputs(x[0], a, b)
    with pytest.raises(ValueError, match="batch/time shapes differ"):
        api.check_fixed_inputs(x, a[:, :4], b)
    with pytest.raises(ValueError, match="alpha/basis dimensions disagree"):
        api.check_fixed_inputs(x, a, b[:2])
    with pytest.raises(ValueError, match="must all be positive"):
        api.check_fixed_inputs(x[:, :0], a[:, :0], b)


def test_packed_shape_validation(no_device_check):
    x = torch.zeros(10, 8)
    a = torch.zeros(10, 3)
    b = torch.zeros(3, 4, 8)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    # cu_seqlens residency is checked by the packed validator itself
    with pytest.raises(ValueError, match="cu_seqlens must be a CUDA tensor"):
        api.check_packed_inputs(x, a, b, cu, 6)
    with pytest.raises(ValueError, match="ranks 2/2/3"):
        api.check_packed_inputs(x[None], a, b, cu, 6)
    with pytest.raises(ValueError, match="token counts differ"):
        api.check_packed_inputs(x, a[:9], b, cu, 6)


def test_dispatch_errors(no_device_check):
    x = torch.zeros(1, 10, 8)
    a = torch.zeros(1, 10, 3)
    b = torch.zeros(3, 4, 8)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    with pytest.raises(ValueError, match="require cu_seqlens"):
        moc.moc_triton(x, a, b, cu_seqlens_cpu=cu)
    with pytest.raises(ValueError, match="only supported for fixed-length"):
        moc.moc_triton(x, a, b, cu_seqlens=cu, max_seqlen=6, output_final_state=True)
    with pytest.raises(ValueError, match="max_seqlen is required"):
        moc.moc_triton(x, a, b, cu_seqlens=cu)
    with pytest.raises(ValueError, match=r"\[N,D\]/\[N,K\] or \[1,N,D\]/\[1,N,K\]"):
        moc.moc_triton(x.expand(2, 10, 8), a.expand(2, 10, 3), b, cu_seqlens=cu, max_seqlen=6)
    with pytest.raises(ValueError, match="cache must have shape"):
        moc.moc_triton(x, a, b, cache=torch.zeros(1, 8, 3))
    with pytest.raises(ValueError, match="same device and dtype"):
        moc.moc_triton(x, a, b, cache=torch.zeros(1, 8, 4, dtype=torch.float64))


def test_step_shape_errors():
    m = moc.MoC(8, 4, 4, 2)
    with pytest.raises(ValueError, match=r"step expects x with shape \[B, 1, D\]"):
        m.step(torch.zeros(2, 3, 8), torch.zeros(2, 3, 4))
    with pytest.raises(ValueError, match=r"step expects z with shape \[B, 1, Z\]"):
        m.step(torch.zeros(2, 1, 8), torch.zeros(3, 1, 4))


@pytest.mark.parametrize("T,S", [(7, 4), (4, 4), (2, 4), (1, 3)])
def test_final_state(T, S):
    x = torch.arange(2 * T * 3, dtype=torch.float32).reshape(2, T, 3)
    st = api._final_state(x, None, S)
    assert tuple(st.shape) == (2, 3, S)
    full = torch.cat((torch.zeros(2, S, 3), x), 1)[:, -S:].transpose(1, 2)
    assert torch.equal(st, full)
    cache = torch.full((2, 3, S), -1.0)
    st2 = api._final_state(x, cache, S)
    hist = torch.cat((cache.transpose(1, 2), x), 1)[:, -S:].transpose(1, 2)
    assert torch.equal(st2, hist)


def test_prepare_chunk_indices_closed_form_and_lru():
    ops.clear_chunk_index_cache()
    lengths = [31, 17, 5, 23, 64, 65, 1]
    cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int64)
    ch = ops.prepare_chunk_indices(cu, 16)
    expect = [(j, c) for j, n in enumerate(lengths) for c in range((n + 15) // 16)]
    assert ch.dtype == torch.int32 and ch.tolist() == [list(e) for e in expect]
    assert ops.prepare_chunk_indices(cu, 16) is ch        # LRU hit on identity + version
    cu.add_(0)                                            # bumps the version: recompute
    assert ops.prepare_chunk_indices(cu, 16) is not ch
    with pytest.raises(ValueError):
        ops.prepare_chunk_indices(cu, 0)
    with pytest.raises(TypeError):
        ops.prepare_chunk_indices(cu.float(), 16)
    with pytest.raises(ValueError, match="cu_seqlens_cpu must match"):
        ops.prepare_chunk_indices(cu, 16, cu_seqlens_cpu=cu[:-1])
    for i in range(6):
        ops.prepare_chunk_indices(torch.tensor([0, i + 1]), 16)
    assert len(ops._chunk_index_cache) == ops._CHUNK_CACHE_SIZE


def test_group_construction_and_arguments():
    """MoCGroup: layer checks, input counts, and the layers' own validation on
    the fallback path (CPU tensors never take the router kernels)."""
    assert "MoCGroup" in moc.__all__
    q = moc.MoC(16, 8, 4, 4)
    k = moc.MoC(8, 8, 4, 4)
    with pytest.raises(ValueError, match="at least one"):
        moc.MoCGroup()
    with pytest.raises(TypeError, match="takes MoC layers"):
        moc.MoCGroup(q, torch.nn.Linear(2, 2))
    with pytest.raises(ValueError, match="share z_dim"):
        moc.MoCGroup(q, moc.MoC(8, 4, 4, 4))
    grp = moc.MoCGroup(q, k)
    assert list(grp.parameters()) == list(q.parameters()) + list(k.parameters())
    z = torch.zeros(1, 3, 8)
    xs = [torch.zeros(1, 3, 16), torch.zeros(1, 3, 8)]
    with pytest.raises(ValueError, match="got 1 inputs"):
        grp(xs[:1], z)
    with pytest.raises(ValueError, match="got 3 caches"):
        grp(xs, z, cache=[None] * 3)
    assert not ops.router_grouped_supported(z, [q.router, k.router])
    with pytest.raises(ValueError, match="must all be CUDA tensors"):
        grp(xs, z)
