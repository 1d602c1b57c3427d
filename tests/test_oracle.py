"""Pins for the CPU oracle (oracle/moc_oracle.py).

Each oracle function is checked against something it does not share code or
formula with: explicit fp64 loops, torch's conv1d (one-hot routing reduces MoC
to a depthwise causal convolution), closed forms (S=1, impulse inputs),
linearity, finite differences (gradcheck), the adjoint identity, a fixed-length
batch packed as varlen, and decode / prefill round trips.  One test plants
plausible mistakes in copies of the oracle and checks that these pins catch
every one of them; the last one checks the oracle against the committed golden
vectors (tests/golden/), which the GPU parity tests also use.
"""
from __future__ import annotations

import itertools
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moc_oracle as O


def _rand(*shape, seed=0, dtype=torch.float64, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype) * scale


def _loops(x, alpha, basis, activation=None):
    """Explicit-loop MoC in fp64 (pure Python over b, t, s; vectorised over d)."""
    B, T, D = x.shape
    K, S, _ = basis.shape
    y = torch.zeros(B, T, D, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            acc = torch.zeros(D, dtype=torch.float64)
            for s in range(S):
                src = t - (S - 1 - s)
                if src < 0:
                    continue
                w = torch.zeros(D, dtype=torch.float64)
                for k in range(K):
                    w += alpha[b, t, k].double() * basis[k, s].double()
                acc += w * x[b, src].double()
            y[b, t] = acc
    if activation is not None:
        y = y * torch.sigmoid(y)
    return y


@pytest.mark.parametrize("S,K,act", [(1, 3, None), (2, 4, None), (4, 8, "silu"), (5, 2, "swish")])
def test_forward_matches_explicit_loops(S, K, act):
    x = _rand(2, 9, 5, seed=1)
    a = _rand(2, 9, K, seed=2)
    b = _rand(K, S, 5, seed=3)
    torch.testing.assert_close(O.moc_ref(x, a, b, act), _loops(x, a, b, act), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("S", [1, 2, 3, 4, 7])
def test_one_hot_routing_is_depthwise_causal_conv1d(S):
    B, T, D, K = 2, 13, 6, 5
    x = _rand(B, T, D, seed=4)
    b = _rand(K, S, D, seed=5)
    for k in range(K):
        a = torch.zeros(B, T, K, dtype=torch.float64)
        a[..., k] = 1.0
        # conv1d is cross-correlation: tap j multiplies x[t-(S-1-j)] after left padding.
        ref = F.conv1d(F.pad(x.transpose(1, 2), (S - 1, 0)), b[k].t()[:, None, :], groups=D)
        torch.testing.assert_close(O.moc_ref(x, a, b), ref.transpose(1, 2), rtol=1e-12, atol=1e-12)


def test_kernel_size_one_is_per_token_scaling():
    x = _rand(3, 7, 4, seed=6)
    a = _rand(3, 7, 5, seed=7)
    b = _rand(5, 1, 4, seed=8)
    torch.testing.assert_close(O.moc_ref(x, a, b), x * (a @ b[:, 0, :]), rtol=1e-12, atol=1e-12)


def test_impulse_reads_out_the_mixed_kernel():
    B, T, D, K, S, t0 = 1, 12, 3, 4, 4, 5
    a = _rand(B, T, K, seed=9)
    b = _rand(K, S, D, seed=10)
    x = torch.zeros(B, T, D, dtype=torch.float64)
    x[0, t0] = 1.0
    y = O.moc_ref(x, a, b)
    for t in range(T):
        lag = t - t0
        if 0 <= lag < S:
            # token t sees the impulse through tap s = S-1-lag
            expect = a[0, t] @ b[:, S - 1 - lag, :]
        else:
            expect = torch.zeros(D, dtype=torch.float64)
        torch.testing.assert_close(y[0, t], expect, rtol=1e-12, atol=1e-12)


def test_linearity_in_each_operand():
    x1, x2 = _rand(2, 8, 4, seed=11), _rand(2, 8, 4, seed=12)
    a1, a2 = _rand(2, 8, 3, seed=13), _rand(2, 8, 3, seed=14)
    b1, b2 = _rand(3, 4, 4, seed=15), _rand(3, 4, 4, seed=16)
    f = O.moc_ref
    torch.testing.assert_close(f(x1 + 2 * x2, a1, b1), f(x1, a1, b1) + 2 * f(x2, a1, b1))
    torch.testing.assert_close(f(x1, a1 - a2, b1), f(x1, a1, b1) - f(x1, a2, b1))
    torch.testing.assert_close(f(x1, a1, 3 * b1 + b2), 3 * f(x1, a1, b1) + f(x1, a1, b2))


@pytest.mark.parametrize("act", [None, "silu"])
def test_gradcheck_fp64(act):
    x = _rand(2, 6, 3, seed=17).requires_grad_()
    a = _rand(2, 6, 4, seed=18).requires_grad_()
    b = _rand(4, 3, 3, seed=19).requires_grad_()
    assert torch.autograd.gradcheck(lambda x, a, b: O.moc_ref(x, a, b, act), (x, a, b))


def test_gradcheck_varlen_and_routing_fp64():
    cu = torch.tensor([0, 4, 5, 11])
    x = _rand(11, 3, seed=20).requires_grad_()
    lg = _rand(11, 4, seed=21).requires_grad_()
    b = _rand(4, 3, 3, seed=22).requires_grad_()
    for route in ("softmax", "exp"):
        f = lambda x, lg, b: O.moc_varlen_ref(x, O.route(lg, route), b, cu, "silu")  # noqa: E731
        assert torch.autograd.gradcheck(f, (x, lg, b))


def test_adjoint_identity():
    # y is linear in x without SiLU: <y(x), dy> == <x, dx>.
    x = _rand(2, 10, 5, seed=23)
    a = _rand(2, 10, 3, seed=24)
    b = _rand(3, 4, 5, seed=25)
    dy = _rand(2, 10, 5, seed=26)
    y, dx, _, _ = O.moc_grads_ref(x, a, b, dy)
    torch.testing.assert_close((y * dy).sum(), (x * dx).sum(), rtol=1e-12, atol=1e-12)


def test_alpha_and_basis_gradients_close_forms_by_bilinearity():
    # y is linear in alpha and in basis separately: <y, dy> = <alpha, dalpha> = <basis, dbasis>.
    x = _rand(2, 10, 5, seed=27)
    a = _rand(2, 10, 3, seed=28)
    b = _rand(3, 4, 5, seed=29)
    dy = _rand(2, 10, 5, seed=30)
    y, _, da, db = O.moc_grads_ref(x, a, b, dy)
    s = (y * dy).sum()
    torch.testing.assert_close(s, (a * da).sum(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(s, (b * db).sum(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("act", [None, "silu"])
def test_equal_length_varlen_equals_fixed_batch(act):
    B, T, D, K, S = 3, 7, 4, 3, 4
    x = _rand(B, T, D, seed=31)
    a = _rand(B, T, K, seed=32)
    b = _rand(K, S, D, seed=33)
    cu = torch.arange(0, B * T + 1, T)
    y_fixed = O.moc_ref(x, a, b, act)
    y_var = O.moc_varlen_ref(x.reshape(B * T, D), a.reshape(B * T, K), b, cu, act)
    torch.testing.assert_close(y_var, y_fixed.reshape(B * T, D), rtol=1e-12, atol=1e-12)
    y_var3 = O.moc_varlen_ref(x.reshape(1, B * T, D), a.reshape(1, B * T, K), b, cu, act)
    torch.testing.assert_close(y_var3[0], y_fixed.reshape(B * T, D), rtol=1e-12, atol=1e-12)


def test_varlen_has_no_cross_sequence_leakage():
    cu = torch.tensor([0, 3, 4, 9])
    x = _rand(9, 2, seed=34)
    a = _rand(9, 3, seed=35)
    b = _rand(3, 4, 2, seed=36)
    y = O.moc_varlen_ref(x, a, b, cu)
    x2 = x.clone()
    x2[3:4] += 100.0  # perturb sequence 1 only
    y2 = O.moc_varlen_ref(x2, a, b, cu)
    assert torch.equal(y[:3], y2[:3]) and torch.equal(y[4:], y2[4:])


def test_route():
    lg = _rand(4, 6, seed=37)
    p = O.route(lg, "softmax")
    torch.testing.assert_close(p.sum(-1), torch.ones(4, dtype=torch.float64))
    torch.testing.assert_close(p, lg.exp() / lg.exp().sum(-1, keepdim=True))
    torch.testing.assert_close(O.route(lg, "exp"), lg.exp())
    with pytest.raises(ValueError):
        O.route(lg, "relu")


@pytest.mark.parametrize("act", ["softmax", "exp"])
def test_rounded_route_matches_torch_low_precision_autograd(act):
    # torch's own softmax / exp on a bf16 tensor: bf16 output, gradient formed
    # from that output; the oracle's rounded route must reproduce both.
    lg = _rand(6, 8, seed=47, dtype=torch.float32, scale=2.0)
    g = _rand(6, 8, seed=48, dtype=torch.float32)
    lb = lg.bfloat16().requires_grad_()
    ab = torch.softmax(lb, -1) if act == "softmax" else torch.exp(lb)
    ab.backward(g.bfloat16())
    lf = lg.bfloat16().float().requires_grad_()
    af = O.route(lf, act, out_dtype=torch.bfloat16)
    af.backward(g.bfloat16().float())
    torch.testing.assert_close(af, ab.float(), rtol=2 ** -7, atol=1e-6)
    torch.testing.assert_close(lf.grad, lb.grad.float(), rtol=2 ** -6, atol=1e-3 * lf.grad.abs().max().item())
    # in fp32 the rounded route is the plain route, gradient included
    l64 = _rand(5, 7, seed=49).requires_grad_()
    assert torch.autograd.gradcheck(lambda t: O.route(t, act, out_dtype=torch.float64), (l64,))
    torch.testing.assert_close(O.route(l64, act, out_dtype=torch.float64), O.route(l64, act))


@pytest.mark.parametrize("S", [1, 2, 4])
def test_decode_steps_match_full_forward_and_cache_is_last_inputs(S):
    B, T, D, K = 2, 9, 5, 3
    x = _rand(B, T, D, seed=38)
    a = _rand(B, T, K, seed=39)
    b = _rand(K, S, D, seed=40)
    full = O.moc_ref(x, a, b, "silu")
    cache = torch.zeros(B, D, S, dtype=torch.float64)
    for t in range(T):
        y, cache = O.moc_step_ref(x[:, t], a[:, t], b, cache, "silu")
        torch.testing.assert_close(y, full[:, t], rtol=1e-12, atol=1e-12)
    assert torch.equal(cache, x[:, T - S:].transpose(1, 2))


@pytest.mark.parametrize("T1,T2,S", [(6, 5, 4), (2, 3, 4), (4, 1, 3)])
def test_prefill_from_cache_and_final_state(T1, T2, S):
    B, D, K = 2, 4, 3
    x = _rand(B, T1 + T2, D, seed=41)
    a = _rand(B, T1 + T2, K, seed=42)
    b = _rand(K, S, D, seed=43)
    full = O.moc_ref(x, a, b)
    st1 = O.final_state(x[:, :T1], None, S)
    # the state holds the last S inputs, zero-padded on the left
    padded = torch.cat((torch.zeros(B, S, D, dtype=x.dtype), x[:, :T1]), 1)
    assert torch.equal(st1, padded[:, -S:].transpose(1, 2))
    y2 = O.moc_prefill_ref(x[:, T1:], a[:, T1:], b, st1)
    torch.testing.assert_close(y2, full[:, T1:], rtol=1e-12, atol=1e-12)
    st2 = O.final_state(x[:, T1:], st1, S)
    assert torch.equal(st2, O.final_state(x, None, S))


def test_reference_inputs_round_to_compute_dtype():
    x = _rand(1, 3, 2, seed=44, dtype=torch.float32)
    a = _rand(1, 3, 2, seed=45, dtype=torch.float32)
    b = _rand(2, 2, 2, seed=46, dtype=torch.float32)
    rx, ra, rb = O.reference_inputs(x, a, b, torch.bfloat16)
    assert rx.dtype == ra.dtype == rb.dtype == torch.float32 and ra.requires_grad
    assert torch.equal(ra, a.to(torch.bfloat16).float())
    assert torch.equal(rb, b.to(torch.bfloat16).float())
    assert torch.equal(rx, x)


# ---------------------------------------------------------------------------
# Planted mistakes: each mutant is a plausible slip in the oracle's forward;
# at least one of the pins above must reject it.

def _mutant_tap_reversed(x, alpha, basis, activation=None):
    return O.moc_ref(x, alpha, basis.flip(1), activation)


def _mutant_off_by_one(x, alpha, basis, activation=None):
    S = basis.shape[1]
    win = F.pad(x, (0, 0, S, 0)).unfold(1, S, 1)[:, :-1]
    w = torch.einsum("btk,ksd->btds", alpha, basis)
    return (win * w).sum(-1)


def _mutant_dropped_tap(x, alpha, basis, activation=None):
    b = basis.clone()
    b[:, 0] = 0
    return O.moc_ref(x, alpha, b, activation)


def _mutant_alpha_transposed(x, alpha, basis, activation=None):
    # routing weights taken from the previous token (index slip along time)
    return O.moc_ref(x, torch.roll(alpha, 1, 1), basis, activation)


def _pins_pass(f) -> bool:
    checks = []
    x = _rand(2, 9, 5, seed=1)
    a = _rand(2, 9, 4, seed=2)
    b = _rand(4, 4, 5, seed=3)
    checks.append(torch.allclose(f(x, a, b), _loops(x, a, b)))
    xi = torch.zeros(1, 12, 3, dtype=torch.float64)
    xi[0, 5] = 1
    ai = _rand(1, 12, 4, seed=9)
    bi = _rand(4, 4, 3, seed=10)
    yi = f(xi, ai, bi)
    for t in range(12):
        lag = t - 5
        expect = ai[0, t] @ bi[:, 3 - lag, :] if 0 <= lag < 4 else torch.zeros(3, dtype=torch.float64)
        checks.append(torch.allclose(yi[0, t], expect))
    for k in range(2):
        oh = torch.zeros(2, 9, 4, dtype=torch.float64)
        oh[..., k] = 1
        ref = F.conv1d(F.pad(x.transpose(1, 2), (3, 0)), b[k].t()[:, None, :], groups=5)
        checks.append(torch.allclose(f(x, oh, b), ref.transpose(1, 2)))
    return all(checks)


@pytest.mark.parametrize("mutant", [_mutant_tap_reversed, _mutant_off_by_one,
                                    _mutant_dropped_tap, _mutant_alpha_transposed])
def test_pins_reject_planted_mistakes(mutant):
    assert _pins_pass(O.moc_ref)
    assert not _pins_pass(mutant)


def test_grid_of_shapes_matches_loops():
    for (S, K, T) in itertools.product((1, 3), (1, 2), (1, 4)):
        x = _rand(1, T, 3, seed=S * 7 + K)
        a = _rand(1, T, K, seed=S * 11 + K)
        b = _rand(K, S, 3, seed=S * 13 + K)
        torch.testing.assert_close(O.moc_ref(x, a, b), _loops(x, a, b), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# golden fixtures (tests/golden/make_golden.py)

GOLDEN = Path(__file__).resolve().parent / "golden" / "moc_golden.npz"


def golden_cases():
    """(name, S, activation, arrays) of every case in the golden file."""
    data = np.load(GOLDEN)  # allow_pickle is False by default
    out = []
    for name in sorted({k.split("/")[0] for k in data.files}):
        S = int(name.split("_S")[1].split("_")[0])
        act = None if name.endswith("_none") else "silu"
        arrays = {k.split("/")[1]: data[k] for k in data.files if k.startswith(name + "/")}
        out.append((name, S, act, arrays))
    return out


def test_oracle_reproduces_golden():
    """The oracle, run again in fp64 on the stored inputs, reproduces the stored
    outputs (fp32 rounding of the fp64 values)."""
    cases = golden_cases()
    assert len(cases) == 8
    for name, S, act, a in cases:
        t = {k: torch.from_numpy(v).double() for k, v in a.items() if k != "cu_seqlens"}
        assert t["basis"].shape[1] == S
        if "cu_seqlens" in a:
            cu = torch.from_numpy(a["cu_seqlens"]).long()
            got = O.moc_varlen_grads_ref(t["x"], t["alpha"], t["basis"], cu, t["dy"], act)
        else:
            got = O.moc_grads_ref(t["x"], t["alpha"], t["basis"], t["dy"], act)
        for key, g in zip(("y", "dx", "dalpha", "dbasis"), got):
            ref = t[key]
            tol = 1e-6 * ref.abs().max().item() + 1e-12
            assert (g - ref).abs().max().item() <= tol, (name, key)
