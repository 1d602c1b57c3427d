"""Shared helpers of the GPU parity tests: seeded inputs and the tolerance rule.

Tolerance (fp32 compare against the CPU oracle run on the same inputs, with
alpha / basis rounded to the compute dtype as verify.py:54-64 does):
  bf16 I/O : |got - ref| <= 1e-2 * rms(ref) + 1.6e-2 * |ref|   elementwise, and
             max |got - ref| <= 2^-7 * max |ref| + 1e-6          per tensor
  fp32 I/O : |got - ref| <= 1e-5 * rms(ref) + 1e-5   * |ref|   elementwise
One further allowance, only where a test passes ``extra``: dz of the module,
formed from bf16 logit gradients on both sides (``ulp_allowance``).
The reference's own bar (verify.py:20-23) is atol = rtol = 1e-1 (bf16) and
5e-3 (fp32); the rules above are tighter at the shapes tested.
"""
from __future__ import annotations

import torch

TOL = {
    torch.bfloat16: (1e-2, 1.6e-2),
    torch.float32: (1e-5, 1e-5),
}
# per-tensor bound of 16-bit results: max |got - ref| <= MAX_REL * max |ref| + MAX_ABS
MAX_REL, MAX_ABS = 2.0 ** -7, 1e-6


def assert_close(name: str, got: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype,
                 extra: torch.Tensor | None = None) -> None:
    """Check ``got`` against the fp32 oracle result ``ref``.  ``dtype`` is the
    compute (x) dtype; a result stored in a 16-bit dtype is held to the bf16 rule.
    ``extra`` adds an elementwise absolute allowance (see ``ulp_allowance``)."""
    if got.dtype in (torch.bfloat16, torch.float16):
        dtype = torch.bfloat16
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    a_rms, r_rel = TOL[dtype]
    rms = ref.pow(2).mean().sqrt().item() if ref.numel() else 0.0
    err = (got - ref).abs()
    bound = a_rms * rms + r_rel * ref.abs() + 1e-30
    if extra is not None:
        bound = bound + extra.detach().float().cpu().reshape(bound.shape)
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err / bound).flatten()))
        raise AssertionError(
            f"{name} ({dtype}): {int(bad.sum())}/{err.numel()} elements out of tolerance; "
            f"worst at flat {i}: got {got.flatten()[i].item():.6g} ref {ref.flatten()[i].item():.6g} "
            f"(max abs err {err.max().item():.3g}, rms(ref) {rms:.3g})")
    if dtype == torch.bfloat16 and extra is None and err.numel():
        mx = ref.abs().max().item()
        if err.max().item() > MAX_REL * mx + MAX_ABS:
            raise AssertionError(
                f"{name} ({dtype}): max abs err {err.max().item():.3g} above the per-tensor bound "
                f"2^-7 * max|ref| + 1e-6 = {MAX_REL * mx + MAX_ABS:.3g}")


def bf16_ulp(t: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |t| (8 significant bits)."""
    _, e = torch.frexp(t.float())
    return torch.where(t == 0, torch.zeros_like(t, dtype=torch.float32),
                       torch.ldexp(torch.ones_like(t, dtype=torch.float32), e - 8))


def ulp_allowance(d_inter: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Allowance for a result formed as (bf16 intermediate) @ weight, where the
    kernel's and the oracle's intermediate may round to neighbouring bf16
    values: one ulp of each intermediate entry, propagated through |weight|.
    d_inter [..., K] (the oracle's fp32 intermediate), weight [K, M]."""
    u = bf16_ulp(d_inter.detach()).reshape(-1, d_inter.shape[-1])
    return (u @ weight.detach().float().abs()).reshape(*d_inter.shape[:-1], weight.shape[-1])


def round_like(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """t rounded to ``dtype`` in value, with the gradient of the identity."""
    return t + (t.detach().to(dtype).to(t.dtype) - t.detach())


class _RoundGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, t, dtype):
        ctx.dtype = dtype
        return t.view_as(t)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dtype).to(g.dtype), None


def round_grad_like(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Identity whose incoming gradient is rounded to ``dtype``: models a tensor
    of that dtype in the graph (e.g. bf16 router logits, whose gradient torch
    holds in bf16 before the router GEMM's backward)."""
    return _RoundGrad.apply(t, dtype)


def gen(seed: int = 0) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, scale=1.0):
    return torch.randn(*shape, generator=g) * scale
