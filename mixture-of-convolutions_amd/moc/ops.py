"""Launch layer: torch tensors in, libmoc_hip.so C-ABI calls out.

Each ``launch_*`` function keeps the name and argument meaning of the
reference's launch function it replaces (moc/ops.py:129-362) and calls one
entry point of the HIP library on the current stream of the tensors' device.
Output tensors and the workspace come from torch's caching allocator; the
library itself never allocates.

``prepare_chunk_indices`` / ``clear_chunk_index_cache`` (moc/ops.py:30-104) are
kept for callers that precompute chunk indices; the HIP kernels locate sequence
boundaries from ``cu_seqlens`` directly and do not need them.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import ROUTE_ALPHA

VARLEN_BLOCK_T = 64
_CHUNK_CACHE_SIZE = 4
_chunk_index_cache: list[tuple] = []

# operand dtypes the kernels read directly; others are cast to fp32 around the call
_KERNEL_OPERAND_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def clear_chunk_index_cache() -> None:
    _chunk_index_cache.clear()


def prepare_chunk_indices(
    cu_seqlens: torch.Tensor,
    chunk_size: int = VARLEN_BLOCK_T,
    cu_seqlens_cpu: torch.Tensor | None = None,
) -> torch.Tensor:
    """[n_chunks, 2] int32 (sequence id, chunk id within the sequence) for
    ``chunk_size``-token chunks; a 4-entry LRU keyed on tensor identity and
    version (same contract as moc/ops.py:47-104)."""
    if not isinstance(chunk_size, int) or chunk_size <= 0:
        raise ValueError("chunk_size must be a positive Python int")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be rank-1 with at least two entries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError("cu_seqlens must have dtype torch.int32 or torch.int64")
    if cu_seqlens_cpu is not None:
        check_cu_seqlens_cpu(cu_seqlens_cpu, cu_seqlens)

    key = (cu_seqlens, cu_seqlens._version, chunk_size, cu_seqlens_cpu,
           None if cu_seqlens_cpu is None else cu_seqlens_cpu._version)
    for i, entry in enumerate(_chunk_index_cache):
        if all(a is b if isinstance(a, torch.Tensor) or a is None else a == b
               for a, b in zip(entry[:5], key)):
            _chunk_index_cache.insert(0, _chunk_index_cache.pop(i))
            return entry[5]

    src = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens
    lengths = (src[1:] - src[:-1]).to(torch.int64)
    counts = torch.div(lengths + chunk_size - 1, chunk_size, rounding_mode="floor")
    seq_ids = torch.repeat_interleave(torch.arange(counts.numel(), device=src.device), counts)
    first = F.pad(counts.cumsum(0), (1, 0))[:-1]
    local = torch.arange(seq_ids.numel(), device=src.device) - first[seq_ids]
    chunks = torch.stack((seq_ids, local), 1).to(device=cu_seqlens.device, dtype=torch.int32)
    chunks = chunks.contiguous()
    _chunk_index_cache.insert(0, (*key, chunks))
    del _chunk_index_cache[_CHUNK_CACHE_SIZE:]
    return chunks


def check_cu_seqlens_cpu(cu_seqlens_cpu: torch.Tensor, cu_seqlens: torch.Tensor) -> None:
    """Same acceptance rules as moc/ops.py:59-65."""
    if cu_seqlens_cpu.device.type != "cpu":
        raise ValueError("cu_seqlens_cpu must be a CPU tensor")
    if cu_seqlens_cpu.ndim != 1 or cu_seqlens_cpu.numel() != cu_seqlens.numel():
        raise ValueError("cu_seqlens_cpu must match cu_seqlens shape")
    if cu_seqlens_cpu.dtype not in (torch.int32, torch.int64):
        raise TypeError("cu_seqlens_cpu must have dtype torch.int32 or torch.int64")


def check_chunk_indices(chunk_indices: torch.Tensor, cu_seqlens: torch.Tensor) -> None:
    """Same acceptance rules as moc/ops.py:118-126."""
    if not chunk_indices.is_cuda or chunk_indices.device != cu_seqlens.device:
        raise ValueError("chunk_indices must be a CUDA tensor on the same device as cu_seqlens")
    if chunk_indices.ndim != 2 or chunk_indices.shape[1] != 2:
        raise ValueError("chunk_indices must have shape [num_chunks, 2]")
    if chunk_indices.dtype not in (torch.int32, torch.int64):
        raise TypeError("chunk_indices must have dtype torch.int32 or torch.int64")
    if not chunk_indices.is_contiguous():
        raise ValueError("chunk_indices must be contiguous")


def _operand(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.dtype in _KERNEL_OPERAND_DTYPES else t.float()


def _seq_args(x: torch.Tensor, cu_seqlens: torch.Tensor | None):
    """(cu_ptr, cu_is_i64, n_seqs, n_tokens, seq_len, dim) of a [B,T,D] or [N,D] x."""
    if cu_seqlens is None:
        B, T, D = x.shape
        return None, 0, 0, B * T, T, D
    N, D = x.shape
    return (cu_seqlens.data_ptr(), int(cu_seqlens.dtype == torch.int64),
            cu_seqlens.numel() - 1, N, 0, D)


def dy_operand(dy: torch.Tensor, dtype: torch.dtype, one: bool = True
               ) -> tuple[torch.Tensor, int]:
    """(dy tensor, row stride in elements) for moc_backward.  A gradient that is
    one element broadcast over every token and channel (all strides 0, as
    autograd hands over the gradient of ``y.sum()``) is passed as that element
    with row stride -1; one row broadcast over every token (stride 0 over the
    token dimensions) as that row with row stride 0.  Either replaces the
    [n_tokens, D] copy that ``dy.contiguous()`` would make (the reference's
    moc/api.py:171) and the small copy of the row; anything else is made
    contiguous, rows D apart.  ``one=False`` (the prefill entry, which takes
    rows only) passes a broadcast element as one row."""
    D = dy.shape[-1]
    if one and dy.numel() > 1 and all(st == 0 for st in dy.stride()):
        one = dy.as_strided((1,), (1,), dy.storage_offset())
        return (one if one.dtype == dtype else one.to(dtype)), -1
    if dy.ndim >= 2 and dy.numel() > D and all(st == 0 for st in dy.stride()[:-1]):
        row = dy[(0,) * (dy.ndim - 1)]
        return row.to(dtype).contiguous(), 0
    dy = dy.contiguous()
    if dy.dtype != dtype:
        dy = dy.to(dtype)
    return dy, D


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def launch_forward(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    *,
    activation_flag: int,
    cu_seqlens: torch.Tensor | None = None,
    cu_seqlens_cpu: torch.Tensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    routing: int = ROUTE_ALPHA,
) -> torch.Tensor:
    """y = MoC(x, alpha, basis) (moc/ops.py:129-194).  ``alpha`` holds routing
    weights (routing 0, 3, 4) or router logits whose softmax (1) / exp (2) is
    fused."""
    del cu_seqlens_cpu, chunk_indices  # boundaries come from cu_seqlens on device
    L = _lib.lib()
    x = x.contiguous()
    a = _operand(alpha)
    b = _operand(basis)
    K, S, _ = b.shape
    cu_ptr, cu64, n_seqs, n_tokens, seq_len, D = _seq_args(x, cu_seqlens)
    out = torch.empty_like(x)
    x_dt = _lib.dtype_code(x.dtype)
    with _lib.device_guard(x.device):
        # the size depends on the launch device (its CU count): queried there
        nbytes = L.moc_forward_workspace_bytes(n_tokens, D, K, S, x_dt, routing)
        ws = _workspace(nbytes, x.device)
        rc = L.moc_forward(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), out.data_ptr(),
            cu_ptr, cu64, n_seqs, n_tokens, seq_len, D, K, S,
            x_dt, _lib.dtype_code(a.dtype), _lib.dtype_code(b.dtype),
            int(activation_flag), int(routing),
            ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device),
        )
    _lib.check(rc, "moc_forward")
    return out


def launch_preact(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    *,
    cu_seqlens: torch.Tensor | None = None,
    cu_seqlens_cpu: torch.Tensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    routing: int = ROUTE_ALPHA,
) -> torch.Tensor:
    """Pre-activation P (moc/ops.py:197-213).  The fused backward recomputes P
    itself; this stays for callers that want P explicitly."""
    return launch_forward(x, alpha, basis, activation_flag=0, cu_seqlens=cu_seqlens,
                          cu_seqlens_cpu=cu_seqlens_cpu, chunk_indices=chunk_indices,
                          routing=routing)


def launch_backward(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    moc_dy: torch.Tensor,
    preact: torch.Tensor | None = None,
    *,
    activation_flag: int,
    need_x: bool,
    cu_seqlens: torch.Tensor | None = None,
    cu_seqlens_cpu: torch.Tensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    routing: int = ROUTE_ALPHA,
) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor]:
    """(dx or None, dalpha, dbasis) (moc/ops.py:216-338).  ``preact`` is
    accepted for signature compatibility and ignored: the kernel recomputes the
    pre-activation in registers.  With routing != 0, ``dalpha`` is the
    gradient with respect to the logits (routing 3 / 4: the softmax / exp
    gradient formed from the weights ``alpha``)."""
    del preact, cu_seqlens_cpu, chunk_indices
    L = _lib.lib()
    x = x.contiguous()
    dy, dy_stride = dy_operand(moc_dy, x.dtype)
    a = _operand(alpha)
    b = _operand(basis)
    K, S, _ = b.shape
    cu_ptr, cu64, n_seqs, n_tokens, seq_len, D = _seq_args(x, cu_seqlens)
    dx = torch.empty_like(x) if need_x else None
    dalpha = torch.empty_like(a)
    dbasis = torch.empty_like(b)
    x_dt = _lib.dtype_code(x.dtype)
    with _lib.device_guard(x.device):
        # the size depends on the launch device (its CU count): queried there
        nbytes = L.moc_backward_workspace_bytes(n_tokens, D, K, S, x_dt, routing)
        ws = _workspace(nbytes, x.device)
        rc = L.moc_backward(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), dy.data_ptr(), dy_stride,
            None if dx is None else dx.data_ptr(), dalpha.data_ptr(), dbasis.data_ptr(),
            cu_ptr, cu64, n_seqs, n_tokens, seq_len, D, K, S,
            x_dt, _lib.dtype_code(a.dtype), _lib.dtype_code(b.dtype),
            int(activation_flag), int(routing),
            ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device),
        )
    _lib.check(rc, "moc_backward")
    if dalpha.dtype != alpha.dtype:
        dalpha = dalpha.to(alpha.dtype)
    if dbasis.dtype != basis.dtype:
        dbasis = dbasis.to(basis.dtype)
    return dx, dalpha, dbasis


def prefill_supported(x: torch.Tensor, basis: torch.Tensor, with_cache: bool) -> bool:
    """Whether moc_forward_prefill / moc_backward_prefill take a [B, T, D] x
    with this basis (matrix-core shapes; T >= kernel_size - 1 with a cache)."""
    B, T, D = x.shape
    K, S, _ = basis.shape
    if x.dtype not in (torch.bfloat16, torch.float32):
        return False
    return bool(_lib.lib().moc_prefill_supported(B, T, D, K, S, _lib.dtype_code(x.dtype),
                                                 int(with_cache)))


def launch_forward_prefill(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    cache: torch.Tensor | None,
    *,
    activation_flag: int,
    final_state: bool,
    routing: int = ROUTE_ALPHA,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """(y, final state or None) of a fixed-length [B, T, D] x continuing from
    ``cache`` [B, D, S] (moc/api.py:299-309, 218-227) in one launch: the taps
    that reach before a sequence's first token read the cache, and the kernel
    writes the final state (the last S inputs, [B, D, S])."""
    L = _lib.lib()
    x = x.contiguous()
    a = _operand(alpha)
    b = _operand(basis)
    K, S, _ = b.shape
    B, T, D = x.shape
    c = None if cache is None else cache.to(x.dtype).contiguous()
    out = torch.empty_like(x)
    fin = x.new_empty(B, D, S) if final_state else None
    x_dt = _lib.dtype_code(x.dtype)
    with _lib.device_guard(x.device):
        nbytes = L.moc_forward_workspace_bytes(B * T, D, K, S, x_dt, routing)
        ws = _workspace(nbytes, x.device)
        rc = L.moc_forward_prefill(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), out.data_ptr(),
            None if c is None else c.data_ptr(), None if fin is None else fin.data_ptr(),
            B, T, D, K, S, x_dt, _lib.dtype_code(a.dtype), _lib.dtype_code(b.dtype),
            int(activation_flag), int(routing),
            ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device),
        )
    _lib.check(rc, "moc_forward_prefill")
    return out, fin


def launch_backward_prefill(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    cache: torch.Tensor,
    moc_dy: torch.Tensor,
    *,
    activation_flag: int,
    need_x: bool,
    need_cache: bool,
    routing: int = ROUTE_ALPHA,
) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """(dx or None, dalpha, dbasis, dcache or None) of launch_forward_prefill's
    y in one moc_backward_prefill call."""
    L = _lib.lib()
    x = x.contiguous()
    dy, dy_stride = dy_operand(moc_dy, x.dtype, one=False)
    a = _operand(alpha)
    b = _operand(basis)
    K, S, _ = b.shape
    B, T, D = x.shape
    c = cache.to(x.dtype).contiguous()
    dx = torch.empty_like(x) if need_x else None
    dalpha = torch.empty_like(a)
    dbasis = torch.empty_like(b)
    dcache = torch.empty_like(c) if need_cache else None
    x_dt = _lib.dtype_code(x.dtype)
    with _lib.device_guard(x.device):
        nbytes = L.moc_backward_workspace_bytes(B * T, D, K, S, x_dt, routing)
        ws = _workspace(nbytes, x.device)
        rc = L.moc_backward_prefill(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), dy.data_ptr(), dy_stride, c.data_ptr(),
            None if dx is None else dx.data_ptr(), dalpha.data_ptr(), dbasis.data_ptr(),
            None if dcache is None else dcache.data_ptr(),
            B, T, D, K, S, x_dt, _lib.dtype_code(a.dtype), _lib.dtype_code(b.dtype),
            int(activation_flag), int(routing),
            ws.data_ptr(), ws.numel(), _lib.stream_ptr(x.device),
        )
    _lib.check(rc, "moc_backward_prefill")
    if dalpha.dtype != alpha.dtype:
        dalpha = dalpha.to(alpha.dtype)
    if dbasis.dtype != basis.dtype:
        dbasis = dbasis.to(basis.dtype)
    if dcache is not None and dcache.dtype != cache.dtype:
        dcache = dcache.to(cache.dtype)
    return dx, dalpha, dbasis, dcache


def _layer_table(entries):
    """ctypes array of MocLayer from dicts of field values."""
    arr = (_lib.MocLayer * len(entries))()
    for i, e in enumerate(entries):
        for k, v in e.items():
            setattr(arr[i], k, v)
    return arr


def launch_forward_layers(xs, alphas, bases, *, activation_flags, routings,
                          cu_seqlens: torch.Tensor | None = None) -> list[torch.Tensor]:
    """y of several MoC layers on one token axis (same S and dtype; each its own
    K and activation) in one call: one forward launch over every layer's
    channels where the library can (bf16 matrix-core layers), the layers one
    by one otherwise."""
    L = _lib.lib()
    xs = [x.contiguous() for x in xs]
    aa = [_operand(a) for a in alphas]
    bb = [_operand(b) for b in bases]
    S = bb[0].shape[1]
    cu_ptr, cu64, n_seqs, n_tokens, seq_len, _ = _seq_args(xs[0], cu_seqlens)
    ys = [torch.empty_like(x) for x in xs]
    table = _layer_table([dict(x=x.data_ptr(), alpha=a.data_ptr(), basis=b.data_ptr(),
                               y=y.data_ptr(), dim=x.shape[-1], routing=int(r),
                               alpha_dtype=_lib.dtype_code(a.dtype),
                               basis_dtype=_lib.dtype_code(b.dtype), activation=int(f),
                               k=b.shape[0])
                          for x, a, b, y, r, f in zip(xs, aa, bb, ys, routings, activation_flags)])
    x_dt = _lib.dtype_code(xs[0].dtype)
    dev = xs[0].device
    with _lib.device_guard(dev):
        nbytes = L.moc_forward_layers_workspace_bytes(table, len(xs), n_tokens, S, x_dt)
        ws = _workspace(nbytes, dev)
        rc = L.moc_forward_layers(table, len(xs), cu_ptr, cu64, n_seqs, n_tokens, seq_len, S,
                                  x_dt, ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "moc_forward_layers")
    return ys


def launch_backward_layers(xs, alphas, bases, dys, *, activation_flags, routings, need_xs,
                           cu_seqlens: torch.Tensor | None = None):
    """[(dx or None, dalpha, dbasis)] of several MoC layers on one token axis in
    one call (see launch_forward_layers); per layer the results of
    launch_backward."""
    L = _lib.lib()
    xs = [x.contiguous() for x in xs]
    aa = [_operand(a) for a in alphas]
    bb = [_operand(b) for b in bases]
    S = bb[0].shape[1]
    cu_ptr, cu64, n_seqs, n_tokens, seq_len, _ = _seq_args(xs[0], cu_seqlens)
    dyo = [dy_operand(dy, x.dtype) for dy, x in zip(dys, xs)]
    dxs = [torch.empty_like(x) if nx else None for x, nx in zip(xs, need_xs)]
    das = [torch.empty_like(a) for a in aa]
    dbs = [torch.empty_like(b) for b in bb]
    table = _layer_table([dict(x=x.data_ptr(), alpha=a.data_ptr(), basis=b.data_ptr(),
                               dy=d[0].data_ptr(), dy_row_stride=d[1],
                               dx=None if dx is None else dx.data_ptr(), dalpha=da.data_ptr(),
                               dbasis=db.data_ptr(), dim=x.shape[-1], routing=int(r),
                               alpha_dtype=_lib.dtype_code(a.dtype),
                               basis_dtype=_lib.dtype_code(b.dtype), activation=int(f),
                               k=b.shape[0])
                          for x, a, b, d, dx, da, db, r, f in zip(xs, aa, bb, dyo, dxs, das, dbs,
                                                                  routings, activation_flags)])
    x_dt = _lib.dtype_code(xs[0].dtype)
    dev = xs[0].device
    with _lib.device_guard(dev):
        nbytes = L.moc_backward_layers_workspace_bytes(table, len(xs), n_tokens, S, x_dt)
        ws = _workspace(nbytes, dev)
        rc = L.moc_backward_layers(table, len(xs), cu_ptr, cu64, n_seqs, n_tokens, seq_len, S,
                                   x_dt, ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "moc_backward_layers")
    out = []
    for dx, da, db, a, b in zip(dxs, das, dbs, alphas, bases):
        out.append((dx, da if da.dtype == a.dtype else da.to(a.dtype),
                    db if db.dtype == b.dtype else db.to(b.dtype)))
    return out


def launch_update(
    x: torch.Tensor,
    alpha: torch.Tensor,
    basis: torch.Tensor,
    cache: torch.Tensor,
    *,
    activation_flag: int,
    routing: int = ROUTE_ALPHA,
) -> torch.Tensor:
    """One decode step, cache updated in place (moc/ops.py:341-362).
    x [B,D], alpha [B,K] (weights or logits), cache [B,D,S] (any strides)."""
    L = _lib.lib()
    x = x.contiguous()
    a = _operand(alpha)
    b = _operand(basis)
    B, D = x.shape
    K, S, _ = b.shape
    out = torch.empty_like(x)
    with _lib.device_guard(x.device):
        rc = L.moc_update(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), cache.data_ptr(),
            *cache.stride(), out.data_ptr(), B, D, K, S,
            _lib.dtype_code(x.dtype), _lib.dtype_code(a.dtype), _lib.dtype_code(b.dtype),
            int(activation_flag), int(routing), _lib.stream_ptr(x.device),
        )
    _lib.check(rc, "moc_update")
    return out


_router_support_cache: dict[tuple, bool] = {}
ROUTER_MAX_TOKENS = 65535 * 64   # grid bound of the router kernels (include/moc_hip.h)


def router_supported(z: torch.Tensor, router: torch.Tensor) -> bool:
    """Whether the router GEMM of ``MoC.forward`` runs on the library's kernels
    (bf16 z and router on a GPU, k % 4 == 0, k <= 96, z_dim % 64 == 0; the
    fused router activation further needs k <= 32)."""
    if not (z.is_cuda and router.is_cuda) or z.dtype != torch.bfloat16 or router.dtype != z.dtype:
        return False
    K, Z = router.shape
    return _router_shape_supported(z, K, Z)


def _router_shape_supported(z: torch.Tensor, K: int, Z: int) -> bool:
    if z.shape[-1] != Z or z.numel() == 0:
        return False
    N = z.numel() // Z
    # the answer depends on N only through the 2^31-byte buffer bound and the
    # grid bound of the kernels (N <= 65535 * 64)
    key = (Z, K, N * Z * 2 < (1 << 31), N <= ROUTER_MAX_TOKENS)
    hit = _router_support_cache.get(key)
    if hit is None:
        hit = bool(_lib.lib().moc_router_supported(N, Z, K, _lib.DT_BF16))
        _router_support_cache[key] = hit
    return hit


def router_forward(z: torch.Tensor, router: torch.Tensor, routing: int = ROUTE_ALPHA
                   ) -> torch.Tensor:
    """logits = z . router^T (the F.linear(z, router) of moc/api.py:383-388);
    with routing 1 / 2 the router activation of moc/api.py:385-388 too:
    softmax / exp of the bf16 logits, rounded to bf16 (the routing weights)."""
    L = _lib.lib()
    z = z.contiguous()
    r = router.contiguous()
    K, Z = r.shape
    N = z.numel() // Z
    out = torch.empty(*z.shape[:-1], K, dtype=z.dtype, device=z.device)
    with _lib.device_guard(z.device):
        if routing == ROUTE_ALPHA:
            rc = L.moc_router_forward(z.data_ptr(), r.data_ptr(), out.data_ptr(), N, Z, K,
                                      _lib.DT_BF16, _lib.stream_ptr(z.device))
        else:
            rc = L.moc_router_forward_routed(z.data_ptr(), r.data_ptr(), out.data_ptr(), N, Z,
                                             K, _lib.DT_BF16, int(routing),
                                             _lib.stream_ptr(z.device))
    _lib.check(rc, "moc_router_forward")
    return out


ROUTER_MAX_ROUTED_K = 32   # the fused router activation
ROUTER_MAX_GROUPS = 4


def router_grouped_supported(z: torch.Tensor, routers: list[torch.Tensor]) -> bool:
    """Whether ``router_forward_grouped`` applies: bf16 z and routers on one
    GPU, at most 4 groups of k % 4 == 0, k <= 32 routes, 96 in all."""
    if not routers or len(routers) > ROUTER_MAX_GROUPS:
        return False
    if not z.is_cuda or z.dtype != torch.bfloat16:
        return False
    if any(r.dtype != torch.bfloat16 or r.device != z.device or r.ndim != 2 for r in routers):
        return False
    ks = [r.shape[0] for r in routers]
    if any(k % 4 or k > ROUTER_MAX_ROUTED_K for k in ks):
        return False
    Z = routers[0].shape[1]
    if any(r.shape[1] != Z for r in routers):
        return False
    return _router_shape_supported(z, sum(ks), Z)


def router_forward_grouped(z: torch.Tensor, router_cat: torch.Tensor, ks: list[int],
                           routings: list[int]) -> list[torch.Tensor]:
    """One pass over z against the concatenated routers [sum(ks), Z]: group g's
    weights routings[g] (softmax / exp, or 0 for the logits) of its logits,
    each [..., ks[g]] bf16 (the F.linear + activation of several MoC.forward
    calls on one z, moc/api.py:383-388)."""
    import ctypes
    L = _lib.lib()
    z = z.contiguous()
    r = router_cat.contiguous()
    Z = r.shape[1]
    N = z.numel() // Z
    outs = [torch.empty(*z.shape[:-1], k, dtype=z.dtype, device=z.device) for k in ks]
    n = len(ks)
    ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    karr = (ctypes.c_int64 * n)(*ks)
    rarr = (ctypes.c_int * n)(*routings)
    with _lib.device_guard(z.device):
        rc = L.moc_router_forward_grouped(z.data_ptr(), r.data_ptr(), ctypes.addressof(ptrs),
                                          ctypes.addressof(karr), ctypes.addressof(rarr), n, N,
                                          Z, _lib.DT_BF16, _lib.stream_ptr(z.device))
    _lib.check(rc, "moc_router_forward_grouped")
    return outs


def router_backward(z: torch.Tensor, router: torch.Tensor, dlogits: torch.Tensor,
                    need_z: bool, need_router: bool
                    ) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """(dz, drouter) = (dlogits . router, dlogits^T . z); either may be skipped."""
    L = _lib.lib()
    z = z.contiguous()
    r = router.contiguous()
    dl = dlogits.contiguous()
    if dl.dtype != z.dtype:
        dl = dl.to(z.dtype)
    K, Z = r.shape
    N = z.numel() // Z
    dz = torch.empty_like(z) if need_z else None
    dr = torch.empty_like(r) if need_router else None
    with _lib.device_guard(z.device):
        nbytes = L.moc_router_backward_workspace_bytes(N, Z, K, _lib.DT_BF16) if need_router else 0
        ws = _workspace(nbytes, z.device)
        rc = L.moc_router_backward(
            z.data_ptr(), r.data_ptr(), dl.data_ptr(),
            None if dz is None else dz.data_ptr(), None if dr is None else dr.data_ptr(),
            N, Z, K, _lib.DT_BF16, ws.data_ptr() if nbytes else None, nbytes,
            _lib.stream_ptr(z.device))
    _lib.check(rc, "moc_router_backward")
    return dz, dr


_step_support_cache: dict[tuple, bool] = {}


def decode_step_supported(x: torch.Tensor, z: torch.Tensor, router: torch.Tensor,
                          basis: torch.Tensor, cache: torch.Tensor) -> bool:
    """Whether ``launch_decode_step`` applies: bf16 tensors on one GPU, x [B,1,D],
    z [B,1,Z], contiguous cache [B,D,S], and a shape the kernel is built for."""
    bf = torch.bfloat16
    if not (x.is_cuda and x.dtype == bf and z.dtype == bf and router.dtype == bf
            and basis.dtype == bf and cache.dtype == bf):
        return False
    if x.ndim != 3 or z.ndim != 3 or x.shape[1] != 1 or z.shape[:2] != x.shape[:2]:
        return False
    B, _, D = x.shape
    K, S, Db = basis.shape
    Z = z.shape[2]
    if Db != D or tuple(router.shape) != (K, Z) or tuple(cache.shape) != (B, D, S):
        return False
    if not cache.is_contiguous():
        return False
    dev = x.device
    if z.device != dev or router.device != dev or basis.device != dev or cache.device != dev:
        return False
    key = (B, Z, D, K, S)
    hit = _step_support_cache.get(key)
    if hit is None:
        hit = bool(_lib.lib().moc_decode_step_supported(B, Z, D, K, S))
        _step_support_cache[key] = hit
    return hit


def launch_decode_step(x: torch.Tensor, z: torch.Tensor, router: torch.Tensor,
                       basis: torch.Tensor, cache: torch.Tensor, *, activation_flag: int,
                       routing: int) -> torch.Tensor:
    """One decode step of the MoC layer in one launch: router GEMM, softmax / exp
    and the cache update (MoC.step, moc/api.py:403-425).  x [B,D] or [B,1,D],
    z [B,Z] or [B,1,Z]; ``cache`` [B,D,S] contiguous, updated in place; returns
    y shaped as x."""
    L = _lib.lib()
    x = x.contiguous()
    z = z.contiguous()
    r = router.contiguous()
    b = basis.contiguous()
    B, D = x.shape[0], x.shape[-1]
    K, S, _ = b.shape
    out = torch.empty_like(x)
    with _lib.device_guard(x.device):
        rc = L.moc_decode_step(z.data_ptr(), r.data_ptr(), x.data_ptr(), b.data_ptr(),
                               cache.data_ptr(), out.data_ptr(), B, z.shape[-1], D, K, S,
                               int(activation_flag), int(routing), _lib.stream_ptr(x.device))
    _lib.check(rc, "moc_decode_step")
    return out
