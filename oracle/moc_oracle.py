"""CPU oracle for the Mixture-of-Convolutions (MoC) hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The product path (``moc`` package +
``libmoc_hip.so``) never imports, calls or links anything under ``oracle/``.

This is a restatement of the reference's PyTorch oracle and of the behaviour of
its API layer, written from the mathematics:

    alpha[n, k] = act_k(logits[n, :])            act = softmax | exp
    W[n, s, d]  = sum_k alpha[n, k] * basis[k, s, d]
    P[n, d]     = sum_s W[n, s, d] * x[n - (S-1-s), d]     (zero outside the sequence)
    y           = silu(P)  if activation in ("silu", "swish") else P

Tap ``s = S-1`` multiplies the current token, tap 0 the oldest one
(reference ``moc/reference.py:29-32``, ``moc/kernels.py:99-130``).

Functions and the reference lines they follow:

* ``moc_ref``          - ``moc/reference.py:19-33`` (pad, unfold, einsum, sum, SiLU).
* ``moc_varlen_ref``   - ``moc/reference.py:36-59`` (per-sequence loop over cu_seqlens).
* ``route``            - ``moc/api.py:383-388`` (router softmax / exp; optionally
                         rounded to the logits' dtype with torch's gradient rule).
* ``final_state``      - ``moc/api.py:218-227`` (last S tokens as [B, D, S]).
* ``moc_prefill_ref``  - ``moc/api.py:299-309`` (prepend the cache, drop its rows).
* ``moc_step_ref``     - ``moc/kernels.py:487-550`` (decode: read slots 1..S-1 plus x,
                         then shift the cache left and write x into slot S-1).
* ``reference_inputs`` - ``verify.py:54-64`` (alpha/basis rounded to the x dtype, fp32 copies).
* ``moc_grads_ref``    - autograd of ``moc_ref`` / ``moc_varlen_ref`` (``verify.py:67-81``).

How each function is pinned (see ``tests/test_oracle.py``): explicit fp64 loops on
tiny shapes, ``torch.nn.functional.conv1d(groups=D)`` for one-hot routing, the
closed forms for S=1 and impulse inputs, linearity, ``gradcheck`` in fp64, the
adjoint identity <y(x), dy> = <x, dx>, varlen == per-sequence fixed, decode
steps == full forward, cache == last S tokens bit-exact.  No function here is
left "parity unpinned".
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "moc_ref",
    "moc_varlen_ref",
    "route",
    "final_state",
    "moc_prefill_ref",
    "moc_step_ref",
    "reference_inputs",
    "moc_grads_ref",
    "moc_varlen_grads_ref",
]


def _activate(p: torch.Tensor, activation: str | None) -> torch.Tensor:
    # moc/reference.py:7-16
    if activation is None:
        return p
    if activation not in ("silu", "swish"):
        raise ValueError(f"unsupported activation: {activation}")
    return F.silu(p)


def moc_ref(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor,
            activation: str | None = None) -> torch.Tensor:
    """Fixed-length MoC.  x [B,T,D], alpha [B,T,K], basis [K,S,D] -> [B,T,D].

    Follows moc/reference.py:19-33: left-pad time by S-1, take windows of S
    tokens, form the per-token kernels with an einsum over k and reduce over
    the window.
    """
    S = basis.shape[1]
    padded = F.pad(x, (0, 0, S - 1, 0))                   # [B, T+S-1, D]
    win = padded.unfold(1, S, 1)                           # [B, T, D, S]; win[..., s] = x[t-(S-1-s)]
    w = torch.einsum("btk,ksd->btds", alpha, basis)        # [B, T, D, S]
    return _activate((win * w).sum(-1), activation)


def moc_varlen_ref(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor,
                   cu_seqlens: torch.Tensor, activation: str | None = None) -> torch.Tensor:
    """Packed MoC.  x [N,D] or [1,N,D]; alpha [N,K] or [1,N,K]; cu_seqlens [n+1].

    Follows moc/reference.py:36-59: every sequence is run as its own batch-1
    fixed-length problem and the results are concatenated.
    """
    batched = x.ndim == 3
    if batched:
        x, alpha = x[0], alpha[0]
    bounds = [int(v) for v in cu_seqlens.detach().cpu().tolist()]
    pieces = []
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        if hi <= lo:  # an empty sequence contributes no rows (the unfold needs T >= 1)
            continue
        pieces.append(moc_ref(x[lo:hi][None], alpha[lo:hi][None], basis, activation)[0])
    out = torch.cat(pieces, 0) if pieces else x.new_zeros(0, x.shape[-1])
    return out[None] if batched else out


class _RoundedRoute(torch.autograd.Function):
    """Router activation whose output is rounded to ``dtype`` and whose
    backward uses that rounded output, as torch's softmax / exp backward does
    for a low-precision tensor (they differentiate through the saved result)."""

    @staticmethod
    def forward(ctx, logits, router_activation, dtype):
        a = route(logits, router_activation).to(dtype).to(logits.dtype)
        ctx.save_for_backward(a)
        ctx.softmax = router_activation == "softmax"
        return a

    @staticmethod
    def backward(ctx, g):
        (a,) = ctx.saved_tensors
        if ctx.softmax:
            return a * (g - (a * g).sum(-1, keepdim=True)), None, None
        return a * g, None, None


def route(logits: torch.Tensor, router_activation: str,
          out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Router activation of moc/api.py:383-388 (softmax over K, or exp).

    With ``out_dtype`` the result is rounded to that dtype (the dtype the
    router's logits have in the module) and the gradient is formed from the
    rounded result, like torch's own softmax / exp on such a tensor."""
    if router_activation not in ("softmax", "exp"):
        raise ValueError(f"unsupported router activation: {router_activation}")
    if out_dtype is not None:
        return _RoundedRoute.apply(logits, router_activation, out_dtype)
    if router_activation == "softmax":
        return torch.softmax(logits, dim=-1)
    return torch.exp(logits)


def final_state(x: torch.Tensor, cache: torch.Tensor | None, S: int) -> torch.Tensor:
    """[B,D,S] state after consuming x [B,T,D] (moc/api.py:218-227)."""
    B, T, D = x.shape
    xt = x.transpose(1, 2)                                  # [B, D, T]
    if T >= S:
        return xt[:, :, T - S:].contiguous()
    head = x.new_zeros(B, D, S - T) if cache is None else cache[:, :, T:]
    return torch.cat((head, xt), dim=-1)


def moc_prefill_ref(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor,
                    cache: torch.Tensor, activation: str | None = None) -> torch.Tensor:
    """Fixed-length MoC continuing from a [B,D,S] cache (moc/api.py:299-309).

    The cache rows act as the S tokens that precede x; their own outputs are
    discarded.
    """
    S = basis.shape[1]
    hist = cache.transpose(1, 2).to(x.dtype)                # [B, S, D], slot 0 oldest
    a0 = alpha.new_zeros(alpha.shape[0], S, alpha.shape[2])
    full = moc_ref(torch.cat((hist, x), 1), torch.cat((a0, alpha), 1), basis, activation)
    return full[:, S:]


def moc_step_ref(x_t: torch.Tensor, alpha_t: torch.Tensor, basis: torch.Tensor,
                 cache: torch.Tensor, activation: str | None = None
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """One decode step (moc/kernels.py:487-550), functional form.

    x_t [B,D], alpha_t [B,K], cache [B,D,S] (slot S-1 newest).  Returns
    (y [B,D], new_cache [B,D,S]).  Tap s<S-1 reads cache slot s+1, tap S-1
    reads x_t; the new cache is the old one shifted left by one slot with x_t
    appended, i.e. exactly the last S inputs.
    """
    S = basis.shape[1]
    w = torch.einsum("bk,ksd->bsd", alpha_t, basis)        # [B, S, D]
    hist = torch.cat((cache[:, :, 1:].to(x_t.dtype), x_t[:, :, None]), -1)  # [B, D, S]
    p = (hist * w.transpose(1, 2)).sum(-1)
    y = _activate(p, activation)
    new_cache = torch.cat((cache[:, :, 1:], x_t[:, :, None].to(cache.dtype)), -1)
    return y, new_cache


def reference_inputs(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor,
                     compute_dtype: torch.dtype):
    """fp32 CPU leaf copies the oracle runs on (verify.py:54-64).

    When the kernel computes in bf16, alpha and basis are rounded to bf16
    first, exactly as the reference's kernels do before their dot products.
    """
    return (
        x.detach().float().cpu().requires_grad_(),
        alpha.detach().to(compute_dtype).float().cpu().requires_grad_(),
        basis.detach().to(compute_dtype).float().cpu().requires_grad_(),
    )


def moc_grads_ref(x, alpha, basis, dy, activation=None):
    """(y, dx, dalpha, dbasis) of moc_ref by autograd on fp32/fp64 CPU leaves."""
    x = x.detach().clone().requires_grad_()
    alpha = alpha.detach().clone().requires_grad_()
    basis = basis.detach().clone().requires_grad_()
    y = moc_ref(x, alpha, basis, activation)
    y.backward(dy.to(y.dtype))
    return y.detach(), x.grad, alpha.grad, basis.grad


def moc_varlen_grads_ref(x, alpha, basis, cu_seqlens, dy, activation=None):
    """(y, dx, dalpha, dbasis) of moc_varlen_ref by autograd."""
    x = x.detach().clone().requires_grad_()
    alpha = alpha.detach().clone().requires_grad_()
    basis = basis.detach().clone().requires_grad_()
    y = moc_varlen_ref(x, alpha, basis, cu_seqlens, activation)
    y.backward(dy.to(y.dtype))
    return y.detach(), x.grad, alpha.grad, basis.grad
