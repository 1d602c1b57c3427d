"""Public MoC API, drop-in for the reference's moc/api.py.

Same names, signatures, validation (exception types and messages), return
conventions, parameter names and cache layout as the reference
(moc/api.py:15-425).  What differs is underneath: the autograd functions call
the gfx950 HIP kernels of libmoc_hip.so through ``ops`` and

* the backward recomputes the pre-activation inside the kernel instead of
  re-running the forward (moc/api.py:176-183);
* the router activation and its gradient cost no kernels of their own
  (moc/api.py:383-388): for bf16 layers ``MoC.forward`` is one autograd node
  whose router kernel forms softmax / exp(z . router^T) and whose MoC backward
  returns d(logits) for the router backward; otherwise (and in ``MoC.step``)
  the kernels take the router *logits*, form the weights themselves and
  return d(logits);
* the router GEMM logits = z . router^T and its backward run on the library's
  skinny-GEMM kernels for bf16 layers (``router_linear``), torch's F.linear
  otherwise.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import ops
from ._lib import (ROUTE_ALPHA, ROUTE_EXP, ROUTE_EXP_WEIGHTS, ROUTE_SOFTMAX,
                   ROUTE_SOFTMAX_WEIGHTS)
from .optim import moc_fan_in_std

SUPPORTED_DTYPES = (torch.bfloat16, torch.float32)

_ROUTING_CODES = {"softmax": ROUTE_SOFTMAX, "exp": ROUTE_EXP}
_WEIGHTS_CODES = {"softmax": ROUTE_SOFTMAX_WEIGHTS, "exp": ROUTE_EXP_WEIGHTS}


# ---------------------------------------------------------------------------
# validation (moc/api.py:18-92, 198-215)

def activation_flag(activation: str | None) -> int:
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"unsupported activation: {activation}")
    return 0 if activation is None else 1


def check_router_activation(router_activation: str) -> None:
    if router_activation not in _ROUTING_CODES:
        raise ValueError(
            f"unsupported router activation: {router_activation}; "
            "expected 'softmax' or 'exp'"
        )


def check_common_dtypes(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor) -> None:
    if not all(t.is_cuda for t in (x, alpha, basis)):
        raise ValueError("x, alpha, and basis must all be CUDA tensors")
    if alpha.device != x.device or basis.device != x.device:
        raise ValueError("x, alpha, and basis must be on the same CUDA device")
    if x.dtype not in SUPPORTED_DTYPES:
        raise TypeError(f"unsupported x dtype: {x.dtype}")
    if not alpha.is_floating_point():
        raise TypeError(f"alpha must be floating point, got {alpha.dtype}")
    if not basis.is_floating_point():
        raise TypeError(f"basis must be floating point, got {basis.dtype}")


def check_fixed_inputs(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor
                       ) -> tuple[int, int, int, int, int]:
    check_common_dtypes(x, alpha, basis)
    if (x.ndim, alpha.ndim, basis.ndim) != (3, 3, 3):
        raise ValueError("fixed-length inputs must have x/alpha/basis ranks 3/3/3")
    B, T, D = x.shape
    Ba, Ta, K = alpha.shape
    Kb, KS, Db = basis.shape
    if (Ba, Ta) != (B, T):
        raise ValueError(f"x and alpha batch/time shapes differ: {(B, T)} vs {(Ba, Ta)}")
    if (Kb, Db) != (K, D):
        raise ValueError(f"alpha/basis dimensions disagree: K,D={(K, D)} vs {(Kb, Db)}")
    if min(B, T, D, K, KS) <= 0:
        raise ValueError("B, T, D, K, and KS must all be positive")
    return B, T, D, K, KS


def check_packed_inputs(x: torch.Tensor, alpha: torch.Tensor, basis: torch.Tensor,
                        cu_seqlens: torch.Tensor, max_seqlen: int
                        ) -> tuple[int, int, int, int, int]:
    check_common_dtypes(x, alpha, basis)
    if (x.ndim, alpha.ndim, basis.ndim) != (2, 2, 3):
        raise ValueError("packed inputs must have x/alpha/basis ranks 2/2/3 internally")
    N, D = x.shape
    Na, K = alpha.shape
    Kb, KS, Db = basis.shape
    if Na != N:
        raise ValueError(f"x and alpha token counts differ: {N} vs {Na}")
    if (Kb, Db) != (K, D):
        raise ValueError(f"alpha/basis dimensions disagree: K,D={(K, D)} vs {(Kb, Db)}")
    if min(N, D, K, KS) <= 0:
        raise ValueError("total tokens, D, K, and KS must all be positive")
    if not cu_seqlens.is_cuda or cu_seqlens.device != x.device:
        raise ValueError("cu_seqlens must be a CUDA tensor on the same device as x")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be rank-1 with at least two entries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError("cu_seqlens must have dtype torch.int32 or torch.int64")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive Python int")
    return N, cu_seqlens.numel() - 1, D, K, KS


def _canonicalize_packed_input(x: torch.Tensor, alpha: torch.Tensor
                               ) -> tuple[torch.Tensor, torch.Tensor, bool]:
    if x.ndim == 2 and alpha.ndim == 2:
        return x, alpha, False
    if x.ndim == 3 and alpha.ndim == 3 and x.shape[0] == 1 and alpha.shape[0] == 1:
        return x[0], alpha[0], True
    raise ValueError("varlen x/alpha must be [N,D]/[N,K] or [1,N,D]/[1,N,K]")


def _check_cache(x: torch.Tensor, basis: torch.Tensor, cache: torch.Tensor) -> None:
    B, _, D = x.shape
    KS = basis.shape[1]
    if tuple(cache.shape) != (B, D, KS):
        raise ValueError(f"cache must have shape {(B, D, KS)}, got {tuple(cache.shape)}")
    if cache.device != x.device or cache.dtype != x.dtype:
        raise ValueError("cache must have the same device and dtype as x")


def _final_state(x: torch.Tensor, cache: torch.Tensor | None, kernel_size: int) -> torch.Tensor:
    """The last ``kernel_size`` inputs as [B,D,S] (moc/api.py:218-227)."""
    B, T, D = x.shape
    xt = x.transpose(1, 2)
    if T >= kernel_size:
        return xt[:, :, T - kernel_size:].contiguous()
    head = x.new_zeros(B, D, kernel_size - T) if cache is None else cache[:, :, T:]
    return torch.cat((head, xt), dim=-1)


# ---------------------------------------------------------------------------
# autograd

def _prepare(ctx_like, x, alpha, basis, cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices):
    """Shared argument handling of the two autograd functions
    (moc/api.py:108-134).  Returns contiguous (x, alpha, basis, cu_seqlens)."""
    x = x.contiguous()
    alpha = alpha.contiguous()
    basis = basis.contiguous()
    if cu_seqlens is not None:
        if max_seqlen is None:
            raise ValueError("max_seqlen is required when cu_seqlens is provided")
        cu_seqlens = cu_seqlens.contiguous()
        check_packed_inputs(x, alpha, basis, cu_seqlens, max_seqlen)
        if chunk_indices is not None:
            ops.check_chunk_indices(chunk_indices.contiguous(), cu_seqlens)
        elif cu_seqlens_cpu is not None:
            ops.check_cu_seqlens_cpu(cu_seqlens_cpu, cu_seqlens)
    else:
        if max_seqlen is not None:
            raise ValueError("max_seqlen must be None when cu_seqlens is None")
        if cu_seqlens_cpu is not None or chunk_indices is not None:
            raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
        check_fixed_inputs(x, alpha, basis)
    return x, alpha, basis, cu_seqlens


def _moc_forward(ctx, x, alpha, basis, activation, routing, cu_seqlens, max_seqlen,
                 cu_seqlens_cpu, chunk_indices, extra=()):
    """Forward of the autograd functions; saves x, alpha, basis, then the
    tensors of ``extra``, then cu_seqlens (varlen)."""
    x, alpha, basis, cu_seqlens = _prepare(ctx, x, alpha, basis, cu_seqlens, max_seqlen,
                                           cu_seqlens_cpu, chunk_indices)
    act = activation_flag(activation)
    y = ops.launch_forward(x, alpha, basis, activation_flag=act, cu_seqlens=cu_seqlens,
                           routing=routing)
    tail = () if cu_seqlens is None else (cu_seqlens,)
    ctx.save_for_backward(x, alpha, basis, *extra, *tail)
    ctx.n_extra = len(extra)
    ctx.act = act
    ctx.routing = routing
    ctx.varlen = cu_seqlens is not None
    return y


def _moc_backward(ctx, dy):
    saved = ctx.saved_tensors
    x, alpha, basis = saved[:3]
    cu_seqlens = saved[3 + ctx.n_extra] if ctx.varlen else None
    return ops.launch_backward(x, alpha, basis, dy, activation_flag=ctx.act,
                               need_x=ctx.needs_input_grad[0], cu_seqlens=cu_seqlens,
                               routing=ctx.routing)


class _MoCFunction(torch.autograd.Function):
    """MoC on routing weights ``alpha`` (moc/api.py:95-195)."""

    @staticmethod
    def forward(ctx, x, alpha, basis, activation, cu_seqlens, max_seqlen, cu_seqlens_cpu,
                chunk_indices):
        return _moc_forward(ctx, x, alpha, basis, activation, ROUTE_ALPHA, cu_seqlens,
                            max_seqlen, cu_seqlens_cpu, chunk_indices)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        dx, dalpha, dbasis = _moc_backward(ctx, dy)
        return dx, dalpha, dbasis, None, None, None, None, None


class _MoCRoutedFunction(torch.autograd.Function):
    """MoC on router logits: alpha = softmax(logits) or exp(logits) is formed
    inside the kernels and the backward returns d(logits)."""

    @staticmethod
    def forward(ctx, x, logits, basis, activation, router_activation, cu_seqlens, max_seqlen,
                cu_seqlens_cpu, chunk_indices):
        return _moc_forward(ctx, x, logits, basis, activation, _ROUTING_CODES[router_activation],
                            cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        dx, dlogits, dbasis = _moc_backward(ctx, dy)
        return dx, dlogits, dbasis, None, None, None, None, None, None


class _RouterLinear(torch.autograd.Function):
    """logits = z . router^T on the library's router kernels, with their
    backward (dz = dlogits . router, drouter = dlogits^T . z)."""

    @staticmethod
    def forward(ctx, z, router):
        ctx.save_for_backward(z, router)
        return ops.router_forward(z, router)

    @staticmethod
    @once_differentiable
    def backward(ctx, dlogits):
        z, router = ctx.saved_tensors
        dz, dr = ops.router_backward(z, router, dlogits, ctx.needs_input_grad[0],
                                     ctx.needs_input_grad[1])
        return dz, dr


class _MoCLayerFunction(torch.autograd.Function):
    """The MoC layer (moc/api.py:372-400) on the library's kernels end to end:
    the router kernel forms the routing weights softmax / exp(z . router^T)
    (bf16, once per token), the MoC forward uses them as given, the MoC
    backward (routing *_WEIGHTS) returns the logits gradient, which the router
    backward turns into dz and drouter."""

    @staticmethod
    def forward(ctx, x, z, router, basis, activation, router_activation, cu_seqlens, max_seqlen,
                cu_seqlens_cpu, chunk_indices):
        weights = ops.router_forward(z, router, routing=_ROUTING_CODES[router_activation])
        return _moc_forward(ctx, x, weights, basis, activation,
                            _WEIGHTS_CODES[router_activation], cu_seqlens, max_seqlen,
                            cu_seqlens_cpu, chunk_indices, extra=(z, router))

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        dx, dlogits, dbasis = _moc_backward(ctx, dy)
        z, router = ctx.saved_tensors[3:5]
        dz = dr = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dz, dr = ops.router_backward(z, router, dlogits, ctx.needs_input_grad[1],
                                         ctx.needs_input_grad[2])
        return dx, dz, dr, dbasis, None, None, None, None, None, None


class _MoCGroupFunction(torch.autograd.Function):
    """Several MoC layers on one routing input z as one autograd node: one
    router pass over the concatenated routers forms every layer's weights, each
    layer's MoC forward / backward runs on its weights (routing *_WEIGHTS), and
    one router backward over the layers' logits gradients side by side gives
    dz (their sum) and every drouter."""

    @staticmethod
    def forward(ctx, z, spec, *tensors):
        # spec: (n, activations, router_activations, cu_seqlens, max_seqlen,
        #        cu_seqlens_cpu, chunk_indices); tensors: routers, xs, bases
        n, acts, routes, cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices = spec
        routers, xs, bases = tensors[:n], tensors[n:2 * n], tensors[2 * n:]
        ks = [r.shape[0] for r in routers]
        router_cat = torch.cat([r.contiguous() for r in routers], 0)
        weights = ops.router_forward_grouped(z, router_cat, ks,
                                             [_ROUTING_CODES[r] for r in routes])
        saved_x, saved_b = [], []
        cu = None
        for g in range(n):
            x, w, b, cu = _prepare(None, xs[g], weights[g], bases[g], cu_seqlens, max_seqlen,
                                   cu_seqlens_cpu, chunk_indices)
            saved_x.append(x)
            saved_b.append(b)
        flags = [activation_flag(a) for a in acts]
        codes = [_WEIGHTS_CODES[r] for r in routes]
        # one call for all layers when they share S and the dtype (each its own K
        # and activation)
        together = len({b.shape[1] for b in saved_b}) == 1 and len({x.dtype for x in saved_x}) == 1
        if together:
            ys = ops.launch_forward_layers(saved_x, weights, saved_b, activation_flags=flags,
                                           routings=codes, cu_seqlens=cu)
        else:
            ys = [ops.launch_forward(x, w, b, activation_flag=f, cu_seqlens=cu, routing=c)
                  for x, w, b, f, c in zip(saved_x, weights, saved_b, flags, codes)]
        tail = () if cu is None else (cu,)
        ctx.save_for_backward(z, router_cat, *saved_x, *weights, *saved_b, *tail)
        ctx.spec = (n, flags, codes, ks, cu is not None, together)
        return tuple(ys)

    @staticmethod
    @once_differentiable
    def backward(ctx, *dys):
        n, acts, codes, ks, varlen, together = ctx.spec
        saved = ctx.saved_tensors
        z, router_cat = saved[0], saved[1]
        xs, weights, bases = saved[2:2 + n], saved[2 + n:2 + 2 * n], saved[2 + 2 * n:2 + 3 * n]
        cu = saved[2 + 3 * n] if varlen else None
        dys = [dy if dy is not None else torch.zeros_like(x) for dy, x in zip(dys, xs)]
        need = [ctx.needs_input_grad[2 + n + g] for g in range(n)]
        if together:
            res = ops.launch_backward_layers(xs, weights, bases, dys, activation_flags=acts,
                                             routings=codes, need_xs=need, cu_seqlens=cu)
        else:
            res = [ops.launch_backward(x, w, b, dy, activation_flag=f, need_x=nx, cu_seqlens=cu,
                                       routing=c)
                   for x, w, b, dy, f, nx, c in zip(xs, weights, bases, dys, acts, need, codes)]
        dxs = [r[0] for r in res]
        dls = [r[1] for r in res]
        dbs = [r[2] for r in res]
        need_z = ctx.needs_input_grad[0]
        need_r = any(ctx.needs_input_grad[2:2 + n])
        dz, dr = None, None
        if need_z or need_r:
            dz, dr = ops.router_backward(z, router_cat, torch.cat(dls, -1), need_z, need_r)
        drs = list(dr.split(ks, 0)) if dr is not None else [None] * n
        return (dz, None, *drs, *dxs, *dbs)


def router_linear(z: torch.Tensor, router: torch.Tensor) -> torch.Tensor:
    """``F.linear(z, router)`` of ``MoC.forward`` (moc/api.py:383): the router
    kernels of the HIP library where they apply (bf16, k % 4 == 0, k <= 32,
    z_dim % 64 == 0), torch's GEMM otherwise."""
    if ops.router_supported(z, router):
        if torch.is_grad_enabled() and (z.requires_grad or router.requires_grad):
            return _RouterLinear.apply(z, router)
        return ops.router_forward(z, router)
    return F.linear(z, router)


def _apply(x, a, basis, activation, router_activation, cu_seqlens=None, max_seqlen=None,
           cu_seqlens_cpu=None, chunk_indices=None):
    if router_activation is None:
        return _MoCFunction.apply(x, a, basis, activation, cu_seqlens, max_seqlen,
                                  cu_seqlens_cpu, chunk_indices)
    return _MoCRoutedFunction.apply(x, a, basis, activation, router_activation, cu_seqlens,
                                    max_seqlen, cu_seqlens_cpu, chunk_indices)


def _step(x, a, basis, cache, activation, router_activation):
    """Decode step (moc/api.py:242-259): in place on ``cache``."""
    _, T, _, _, _ = check_fixed_inputs(x, a, basis)
    if T != 1:
        raise ValueError(f"step expects sequence length 1, got {T}")
    _check_cache(x, basis, cache)
    routing = ROUTE_ALPHA if router_activation is None else _ROUTING_CODES[router_activation]
    y = ops.launch_update(x[:, 0], a[:, 0], basis, cache,
                          activation_flag=activation_flag(activation), routing=routing)
    return y[:, None]


class _MoCPrefillFunction(torch.autograd.Function):
    """Prefill continuing from a cache (moc/api.py:299-309) with its final
    state (moc/api.py:218-227) on the library's prefill entries: one forward
    launch whose taps that reach before a sequence's first token read the
    cache, and which writes the final state; one backward call that also forms
    the cache gradient.  Returns (y, final state or None); a gradient of the
    final state (a slice of x and the cache) is added to dx / dcache here."""

    @staticmethod
    def forward(ctx, x, a, basis, cache, activation, routing, want_state):
        x, a, basis = x.contiguous(), a.contiguous(), basis.contiguous()
        act = activation_flag(activation)
        y, fin = ops.launch_forward_prefill(x, a, basis, cache, activation_flag=act,
                                            final_state=want_state, routing=routing)
        ctx.save_for_backward(x, a, basis, cache)
        ctx.act = act
        ctx.routing = routing
        ctx.set_materialize_grads(False)
        return y, fin

    @staticmethod
    @once_differentiable
    def backward(ctx, dy, dfin):
        x, a, basis, cache = ctx.saved_tensors
        dx, da, db, dc = _prefill_backward(ctx, dy, dfin, x, a, basis, cache,
                                           ctx.needs_input_grad[0], ctx.needs_input_grad[3])
        return dx, da, db, dc, None, None, None


def _prefill_backward(ctx, dy, dfin, x, a, basis, cache, need_x, need_cache):
    """(dx or None, dalpha, dbasis, dcache or None) of a prefill launch, with a
    gradient of the final state (the last S inputs, a slice of x and for T < S
    of the cache, moc/api.py:218-227) added to dx / dcache."""
    B, T, _ = x.shape
    S = basis.shape[1]
    if dy is None:
        dy = torch.zeros_like(x)
    dx, da, db, dc = ops.launch_backward_prefill(
        x, a, basis, cache, dy, activation_flag=ctx.act, need_x=need_x or dfin is not None,
        need_cache=need_cache, routing=ctx.routing)
    if dfin is not None:
        n = min(S, T)
        dx[:, T - n:] += dfin[:, :, S - n:].transpose(1, 2).to(dx.dtype)
        if T < S and dc is not None:
            dc[:, :, T:] += dfin[:, :, :S - T].to(dc.dtype)
    return (dx if need_x else None), da, db, dc


class _MoCLayerPrefillFunction(torch.autograd.Function):
    """MoC.forward continuing from a cache (moc/api.py:299-309, 383-388) on the
    library's kernels end to end: the router kernel forms the routing weights
    softmax / exp(z . router^T), the prefill entries run on them (routing
    *_WEIGHTS, so the backward returns the logits gradient), and the router
    backward turns that into dz and drouter.  Returns (y, final state or None)."""

    @staticmethod
    def forward(ctx, x, z, router, basis, cache, activation, router_activation, want_state):
        weights = ops.router_forward(z, router, routing=_ROUTING_CODES[router_activation])
        x, basis = x.contiguous(), basis.contiguous()
        check_fixed_inputs(x, weights, basis)
        _check_cache(x, basis, cache)
        act = activation_flag(activation)
        routing = _WEIGHTS_CODES[router_activation]
        y, fin = ops.launch_forward_prefill(x, weights, basis, cache, activation_flag=act,
                                            final_state=want_state, routing=routing)
        ctx.save_for_backward(x, weights, basis, cache, z, router)
        ctx.act = act
        ctx.routing = routing
        ctx.set_materialize_grads(False)
        return y, fin

    @staticmethod
    @once_differentiable
    def backward(ctx, dy, dfin):
        x, w, basis, cache, z, router = ctx.saved_tensors
        dx, dlogits, db, dc = _prefill_backward(ctx, dy, dfin, x, w, basis, cache,
                                                ctx.needs_input_grad[0], ctx.needs_input_grad[4])
        dz = dr = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dz, dr = ops.router_backward(z, router, dlogits, ctx.needs_input_grad[1],
                                         ctx.needs_input_grad[2])
        return dx, dz, dr, db, dc, None, None, None


def _prefill(x, a, basis, cache, activation, router_activation, output_final_state):
    """Prefill continuing from a cache (moc/api.py:299-309): (y, final state or
    None).  On the library's prefill entries where they take the shape
    (_MoCPrefillFunction), else by _prefill_window."""
    routing = ROUTE_ALPHA if router_activation is None else _ROUTING_CODES[router_activation]
    if ops.prefill_supported(x, basis, with_cache=True):
        return _MoCPrefillFunction.apply(x, a, basis, cache, activation, routing,
                                         output_final_state)
    y = _prefill_window(x, a, basis, cache, activation, router_activation)
    return y, (_final_state(x, cache, basis.shape[1]) if output_final_state else None)


def _prefill_window(x, a, basis, cache, activation, router_activation):
    """Prefill without the prefill entries.  The reference prepends the whole
    cache to x (and zero routing to a) and drops the first S outputs.  Only the
    first S-1 tokens of each sequence have taps that reach into the cache, so
    here the op runs on x as it is, and those tokens are recomputed from a
    short window (the S-1 newest cached tokens, then the tokens themselves) and
    written over the first result.  No copy of x; y is the reference's bit for
    bit (each token's output depends only on its own window), and gradients
    flow to x, a, basis and the cache as there."""
    B, T, _ = x.shape
    KS = basis.shape[1]
    y = _apply(x, a, basis, activation, router_activation)
    h = min(KS - 1, T)
    if h == 0:
        return y
    hist = cache.transpose(1, 2)[:, 1:]
    xh = torch.cat((hist, x[:, :h]), 1)
    ah = torch.cat((a.new_zeros(B, KS - 1, a.shape[-1]), a[:, :h]), 1)
    yh = _apply(xh, ah, basis, activation, router_activation)[:, KS - 1:]
    y[:, :h] = yh
    return y


def _dispatch(x, a, basis, cache, output_final_state, activation, router_activation,
              cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices):
    """Routing of moc/api.py:262-335 for weights (router_activation None) or
    logits."""
    activation_flag(activation)
    if cu_seqlens is None:
        if cu_seqlens_cpu is not None or chunk_indices is not None:
            raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
        B, T, D, K, KS = check_fixed_inputs(x, a, basis)
        if cache is not None:
            _check_cache(x, basis, cache)
            if T == 1:
                y = _step(x, a, basis, cache, activation, router_activation)
                return y, (cache if output_final_state else None)
            return _prefill(x, a, basis, cache, activation, router_activation,
                            output_final_state)
        else:
            y = _apply(x, a, basis, activation, router_activation)
        return y, (_final_state(x, cache, KS) if output_final_state else None)

    if cache is not None or output_final_state:
        raise ValueError("cache and output_final_state are only supported for fixed-length inputs")
    if max_seqlen is None:
        raise ValueError("max_seqlen is required for varlen inputs")
    xp, ap, restore = _canonicalize_packed_input(x, a)
    check_packed_inputs(xp, ap, basis, cu_seqlens, max_seqlen)
    y = _apply(xp, ap, basis, activation, router_activation, cu_seqlens, max_seqlen,
               cu_seqlens_cpu, chunk_indices)
    return (y[None] if restore else y), None


def moc_triton(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    cache: torch.Tensor | None = None,
    output_final_state: bool = False,
    activation: str | None = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    max_seqlen: Optional[int] = None,
    cu_seqlens_cpu: Optional[torch.Tensor] = None,
    chunk_indices: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Functional MoC on routing weights (moc/api.py:262-335), backed by the
    HIP kernels.  The name is kept for drop-in compatibility; ``moc_hip`` is the
    same function."""
    return _dispatch(x, alpha, basis, cache, output_final_state, activation, None,
                     cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices)


moc_hip = moc_triton


class MoC(nn.Module):
    """Mixture-of-Convolutions layer (moc/api.py:338-425).

    Parameters ``conv_bases`` [k, kernel_size, dim] and ``router`` [k, z_dim]
    have the reference's names, shapes and initialisation, so state dicts load
    unchanged.
    """

    def __init__(self, dim: int, z_dim: int, kernel_size: int, k: int,
                 activation: str | None = None, init_std: float | None = None,
                 router_activation: str = "softmax") -> None:
        super().__init__()
        activation_flag(activation)
        check_router_activation(router_activation)
        self.dim = dim
        self.z_dim = z_dim
        self.kernel_size = kernel_size
        self.k = k
        self.activation = activation
        self.router_activation = router_activation
        self.conv_bases = nn.Parameter(torch.empty(k, kernel_size, dim))
        self.router = nn.Parameter(torch.zeros(k, z_dim))
        if init_std is None:
            init_std = moc_fan_in_std(k, kernel_size)
        bound = init_std * math.sqrt(3)
        nn.init.uniform_(self.conv_bases, a=-bound, b=bound)

    def forward(self, x: torch.Tensor, z: torch.Tensor, cache: torch.Tensor | None = None,
                output_final_state: bool = False, cu_seqlens: Optional[torch.Tensor] = None,
                max_seqlen: Optional[int] = None, cu_seqlens_cpu: Optional[torch.Tensor] = None,
                chunk_indices: Optional[torch.Tensor] = None
                ) -> tuple[torch.Tensor, torch.Tensor | None]:
        if cache is not None and cu_seqlens is None:
            # single-token step: router GEMM, router activation and cache update
            # in one launch (the step is not differentiable, as in the reference);
            # the parameters are fetched once (each module attribute lookup costs
            # about as much as a tensor check on this per-token path)
            router, basis = self.router, self.conv_bases
            if ops.decode_step_supported(x, z, router, basis, cache):
                if cu_seqlens_cpu is not None or chunk_indices is not None:
                    raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
                y = ops.launch_decode_step(x, z, router, basis, cache,
                                           activation_flag=activation_flag(self.activation),
                                           routing=_ROUTING_CODES[self.router_activation])
                return y, (cache if output_final_state else None)
        routed = (self.router.shape[0] <= ops.ROUTER_MAX_ROUTED_K
                  and ops.router_supported(z, self.router))
        if cache is None and routed:
            return self._forward_kernels(x, z, output_final_state, cu_seqlens, max_seqlen,
                                         cu_seqlens_cpu, chunk_indices)
        if (routed and cu_seqlens is None and x.dim() == 3 and x.shape[1] > 1
                and ops.prefill_supported(x, self.conv_bases, with_cache=True)):
            # prefill from the cache: router epilogue + prefill entries, one node
            if cu_seqlens_cpu is not None or chunk_indices is not None:
                raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
            return _MoCLayerPrefillFunction.apply(x, z, self.router, self.conv_bases, cache,
                                                  self.activation, self.router_activation,
                                                  output_final_state)
        logits = router_linear(z, self.router)
        return _dispatch(x, logits, self.conv_bases, cache, output_final_state,
                         self.activation, self.router_activation, cu_seqlens, max_seqlen,
                         cu_seqlens_cpu, chunk_indices)

    def _forward_kernels(self, x, z, output_final_state, cu_seqlens, max_seqlen, cu_seqlens_cpu,
                         chunk_indices):
        """forward without a cache, router included, as one autograd node
        (_MoCLayerFunction); same checks and returns as _dispatch."""
        activation_flag(self.activation)
        args = (self.router, self.conv_bases, self.activation, self.router_activation)
        if cu_seqlens is None:
            if cu_seqlens_cpu is not None or chunk_indices is not None:
                raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
            y = _MoCLayerFunction.apply(x, z, *args, None, None, None, None)
            state = _final_state(x, None, self.kernel_size) if output_final_state else None
            return y, state
        if output_final_state:
            raise ValueError("cache and output_final_state are only supported for fixed-length inputs")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required for varlen inputs")
        xp, zp, restore = _canonicalize_packed_input(x, z)
        y = _MoCLayerFunction.apply(xp, zp, *args, cu_seqlens, max_seqlen, cu_seqlens_cpu,
                                    chunk_indices)
        return (y[None] if restore else y), None

    def step(self, x: torch.Tensor, z: torch.Tensor, cache: torch.Tensor | None = None,
             output_final_state: bool = False) -> tuple[torch.Tensor, torch.Tensor | None]:
        if x.ndim != 3 or x.shape[1] != 1:
            raise ValueError(f"step expects x with shape [B, 1, D], got {tuple(x.shape)}")
        if z.ndim != 3 or z.shape[:2] != x.shape[:2]:
            raise ValueError(f"step expects z with shape [B, 1, Z], got {tuple(z.shape)}")
        if cache is None:
            cache = x.new_zeros(x.shape[0], self.dim, self.kernel_size)
        return self.forward(x, z, cache=cache, output_final_state=output_final_state)

    @property
    def state_size(self) -> int:
        return self.dim * self.kernel_size


class MoCGroup(nn.Module):
    """MoC layers that share their routing input ``z``, run together: the QKV
    pattern of the reference README (README.md:80-129), where each of
    ``q_conv(q, x_norm)``, ``k_conv(k, x_norm)``, ``v_conv(v, x_norm)`` runs its
    own router GEMM over ``x_norm`` (moc/api.py:383-388).

    ``MoCGroup(q_conv, k_conv, v_conv)(xs=[q, k, v], z=x_norm)`` returns the
    same ``[(y, state), ...]`` as calling the layers one by one.  For bf16
    layers on the library's router kernels (at most 4 layers, k % 4 == 0,
    k <= 32 each) the routers run as one: z is read once in the forward, and
    once in the backward, which writes dz once instead of once per layer plus
    autograd's sum.  Otherwise, or with a cache, the layers run one by one.
    The layers keep their parameters (held here as submodules).
    """

    def __init__(self, *layers: MoC) -> None:
        super().__init__()
        if not layers:
            raise ValueError("MoCGroup needs at least one MoC layer")
        if any(not isinstance(m, MoC) for m in layers):
            raise TypeError("MoCGroup takes MoC layers")
        if len({m.z_dim for m in layers}) != 1:
            raise ValueError("the layers of a MoCGroup must share z_dim")
        self.layers = nn.ModuleList(layers)

    def _grouped(self, xs, z, cache) -> bool:
        return (cache is None and ops.router_grouped_supported(z, [m.router for m in self.layers])
                and all(isinstance(x, torch.Tensor) and x.device == z.device for x in xs))

    def forward(self, xs, z: torch.Tensor, cache=None, output_final_state: bool = False,
                cu_seqlens: Optional[torch.Tensor] = None, max_seqlen: Optional[int] = None,
                cu_seqlens_cpu: Optional[torch.Tensor] = None,
                chunk_indices: Optional[torch.Tensor] = None
                ) -> list[tuple[torch.Tensor, torch.Tensor | None]]:
        xs = list(xs)
        if len(xs) != len(self.layers):
            raise ValueError(f"MoCGroup of {len(self.layers)} layers got {len(xs)} inputs")
        caches = list(cache) if cache is not None else [None] * len(xs)
        if len(caches) != len(xs):
            raise ValueError(f"MoCGroup of {len(self.layers)} layers got {len(caches)} caches")
        if not self._grouped(xs, z, cache):
            return [m(x, z, cache=c, output_final_state=output_final_state, cu_seqlens=cu_seqlens,
                      max_seqlen=max_seqlen, cu_seqlens_cpu=cu_seqlens_cpu,
                      chunk_indices=chunk_indices)
                    for m, x, c in zip(self.layers, xs, caches)]
        for m in self.layers:
            activation_flag(m.activation)
        n = len(xs)
        routers = [m.router for m in self.layers]
        bases = [m.conv_bases for m in self.layers]
        acts = [m.activation for m in self.layers]
        routes = [m.router_activation for m in self.layers]
        if cu_seqlens is None:
            if cu_seqlens_cpu is not None or chunk_indices is not None:
                raise ValueError("cu_seqlens_cpu and chunk_indices require cu_seqlens")
            spec = (n, acts, routes, None, None, None, None)
            ys = _MoCGroupFunction.apply(z, spec, *routers, *xs, *bases)
            return [(y, _final_state(x, None, m.kernel_size) if output_final_state else None)
                    for y, x, m in zip(ys, xs, self.layers)]
        if output_final_state:
            raise ValueError("cache and output_final_state are only supported for fixed-length inputs")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required for varlen inputs")
        packed = [_canonicalize_packed_input(x, z) for x in xs]
        restore = packed[0][2]
        spec = (n, acts, routes, cu_seqlens, max_seqlen, cu_seqlens_cpu, chunk_indices)
        ys = _MoCGroupFunction.apply(packed[0][1], spec, *routers, *[p[0] for p in packed], *bases)
        return [((y[None] if restore else y), None) for y in ys]


__all__ = ["MoC", "MoCGroup", "moc_triton", "moc_hip", "router_linear"]
