"""ctypes binding of libmoc_hip.so (C ABI declared in include/moc_hip.h).

The library is loaded on first use from this package's directory.  There is no
fallback: if it is missing or fails to load, every MoC op raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmoc_hip.so"
ABI_VERSION = 5

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
ROUTE_ALPHA, ROUTE_SOFTMAX, ROUTE_EXP = 0, 1, 2
# alpha holds softmax / exp weights already; the backward returns d/dlogits
ROUTE_SOFTMAX_WEIGHTS, ROUTE_EXP_WEIGHTS = 3, 4
# kernel families (moc_set_kernel_path)
PATH_AUTO, PATH_GENERIC, PATH_MFMA_PREP = 0, 1, 2
# device scratch of moc_backward_noalloc
NOALLOC_SCRATCH_BYTES = 64 << 20

_DTYPE_CODES = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float16: DT_F16}

EXPORTED_SYMBOLS = (
    "moc_abi_version",
    "moc_last_error",
    "moc_set_kernel_path",
    "moc_matrix_core_supported",
    "moc_forward_workspace_bytes",
    "moc_forward",
    "moc_backward_workspace_bytes",
    "moc_backward",
    "moc_backward_noalloc",
    "moc_forward_layers_workspace_bytes",
    "moc_forward_layers",
    "moc_backward_layers_workspace_bytes",
    "moc_backward_layers",
    "moc_prefill_supported",
    "moc_forward_prefill",
    "moc_backward_prefill",
    "moc_update",
    "moc_profile_events",
    "moc_decode_step_supported",
    "moc_decode_step",
    "moc_router_supported",
    "moc_router_forward",
    "moc_router_forward_routed",
    "moc_router_forward_grouped",
    "moc_router_backward_workspace_bytes",
    "moc_router_backward",
)

MAX_LAYERS = 4


class MocLayer(ctypes.Structure):
    """struct MocLayer of include/moc_hip.h: one layer of a grouped launch."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("alpha", ctypes.c_void_p), ("basis", ctypes.c_void_p),
        ("y", ctypes.c_void_p), ("dy", ctypes.c_void_p), ("dy_row_stride", ctypes.c_int64),
        ("dx", ctypes.c_void_p), ("dalpha", ctypes.c_void_p), ("dbasis", ctypes.c_void_p),
        ("dim", ctypes.c_int64), ("routing", ctypes.c_int), ("alpha_dtype", ctypes.c_int),
        ("basis_dtype", ctypes.c_int), ("activation", ctypes.c_int), ("k", ctypes.c_int64),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_z = ctypes.c_size_t


def _declare(lib: ctypes.CDLL) -> None:
    lib.moc_abi_version.argtypes = []
    lib.moc_abi_version.restype = _i
    lib.moc_last_error.argtypes = []
    lib.moc_last_error.restype = ctypes.c_char_p
    lib.moc_forward_workspace_bytes.argtypes = [_l, _l, _l, _l, _i, _i]
    lib.moc_forward_workspace_bytes.restype = _z
    lib.moc_backward_workspace_bytes.argtypes = [_l, _l, _l, _l, _i, _i]
    lib.moc_backward_workspace_bytes.restype = _z
    lib.moc_forward.argtypes = [
        _p, _p, _p, _p,            # x, alpha, basis, y
        _p, _i, _l,                # cu_seqlens, cu_seqlens_i64, n_seqs
        _l, _l,                    # n_tokens, seq_len
        _l, _l, _l,                # dim, k, kernel_size
        _i, _i, _i,                # dtypes
        _i, _i,                    # activation, routing
        _p, _z, _p,                # workspace, bytes, stream
    ]
    lib.moc_forward.restype = _i
    bwd = [
        _p, _p, _p, _p, _l,        # x, alpha, basis, dy, dy_row_stride
        _p, _p, _p,                # dx, dalpha, dbasis
        _p, _i, _l,
        _l, _l,
        _l, _l, _l,
        _i, _i, _i,
        _i, _i,
    ]
    lib.moc_backward.argtypes = bwd + [_p, _z, _p]   # workspace, bytes, stream
    lib.moc_backward.restype = _i
    lib.moc_backward_noalloc.argtypes = bwd + [_p]   # stream
    lib.moc_backward_noalloc.restype = _i
    lib.moc_matrix_core_supported.argtypes = [_l, _l, _l, _l, _i, _i]
    lib.moc_matrix_core_supported.restype = _i
    lib.moc_prefill_supported.argtypes = [_l, _l, _l, _l, _l, _i, _i]
    lib.moc_prefill_supported.restype = _i
    lib.moc_forward_prefill.argtypes = [
        _p, _p, _p, _p,            # x, alpha, basis, y
        _p, _p,                    # cache, final_state
        _l, _l,                    # n_seqs, seq_len
        _l, _l, _l,                # dim, k, kernel_size
        _i, _i, _i,                # dtypes
        _i, _i,                    # activation, routing
        _p, _z, _p,                # workspace, bytes, stream
    ]
    lib.moc_forward_prefill.restype = _i
    lib.moc_backward_prefill.argtypes = [
        _p, _p, _p, _p, _l,        # x, alpha, basis, dy, dy_row_stride
        _p,                        # cache
        _p, _p, _p, _p,            # dx, dalpha, dbasis, dcache
        _l, _l,                    # n_seqs, seq_len
        _l, _l, _l,                # dim, k, kernel_size
        _i, _i, _i,                # dtypes
        _i, _i,                    # activation, routing
        _p, _z, _p,                # workspace, bytes, stream
    ]
    lib.moc_backward_prefill.restype = _i
    lib.moc_set_kernel_path.argtypes = [_i]
    lib.moc_set_kernel_path.restype = _i
    for name in ("moc_forward_layers", "moc_backward_layers"):
        fn = getattr(lib, name)
        # layers, n_layers, cu_seqlens, cu_seqlens_i64, n_seqs, n_tokens, seq_len,
        # kernel_size, x_dtype, workspace, bytes, stream
        fn.argtypes = [_p, _i, _p, _i, _l, _l, _l, _l, _i, _p, _z, _p]
        fn.restype = _i
        q = getattr(lib, name + "_workspace_bytes")
        q.argtypes = [_p, _i, _l, _l, _i]   # layers, n_layers, n_tokens, kernel_size, x_dtype
        q.restype = _z
    lib.moc_update.argtypes = [
        _p, _p, _p, _p,            # x, alpha, basis, cache
        _l, _l, _l,                # cache strides (elements)
        _p,                        # y
        _l, _l, _l, _l,            # batch, dim, k, kernel_size
        _i, _i, _i,                # dtypes
        _i, _i, _p,                # activation, routing, stream
    ]
    lib.moc_update.restype = _i
    lib.moc_profile_events.argtypes = [_p, _p]
    lib.moc_profile_events.restype = _i
    lib.moc_decode_step_supported.argtypes = [_l, _l, _l, _l, _l]
    lib.moc_decode_step_supported.restype = _i
    lib.moc_decode_step.argtypes = [_p, _p, _p, _p, _p, _p, _l, _l, _l, _l, _l, _i, _i, _p]
    lib.moc_decode_step.restype = _i
    lib.moc_router_supported.argtypes = [_l, _l, _l, _i]
    lib.moc_router_supported.restype = _i
    lib.moc_router_forward.argtypes = [_p, _p, _p, _l, _l, _l, _i, _p]
    lib.moc_router_forward.restype = _i
    lib.moc_router_forward_routed.argtypes = [_p, _p, _p, _l, _l, _l, _i, _i, _p]
    lib.moc_router_forward_routed.restype = _i
    lib.moc_router_forward_grouped.argtypes = [_p, _p, _p, _p, _p, _i, _l, _l, _i, _p]
    lib.moc_router_forward_grouped.restype = _i
    lib.moc_router_backward_workspace_bytes.argtypes = [_l, _l, _l, _i]
    lib.moc_router_backward_workspace_bytes.restype = _z
    lib.moc_router_backward.argtypes = [_p, _p, _p, _p, _p, _l, _l, _l, _i, _p, _z, _p]
    lib.moc_router_backward.restype = _i


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is not built; run "
                        "`python mixture-of-convolutions_amd/build_lib.py` "
                        "(or __graft_entry__.build()) first"
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                _declare(handle)
                if handle.moc_abi_version() != ABI_VERSION:
                    raise RuntimeError(
                        f"{LIB_PATH} has ABI version {handle.moc_abi_version()}, this package "
                        f"binds version {ABI_VERSION}; rebuild it with "
                        "`python mixture-of-convolutions_amd/build_lib.py`")
                _lib = handle
    return _lib


@contextlib.contextmanager
def kernel_path(path: int):
    """Run the enclosed calls on kernel family ``path`` (PATH_GENERIC to
    cross-check the generic kernels against the matrix-core ones), then restore
    the previous family.  Process-wide."""
    L = lib()
    old = L.moc_set_kernel_path(int(path))
    if old < 0:
        check(old, "moc_set_kernel_path")
    try:
        yield
    finally:
        L.moc_set_kernel_path(old)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().moc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise TypeError(f"libmoc_hip has no kernel operand of dtype {dt}") from None


# torch's direct bindings for the current device and stream (a few hundred ns
# instead of several microseconds per launch); the public calls otherwise
_get_device = getattr(torch._C, "_cuda_getDevice", None)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def device_guard(device: torch.device):
    """``torch.cuda.device(device)``, or a no-op when it is already current."""
    if _get_device is not None and (device.index is None or device.index == _get_device()):
        return contextlib.nullcontext()
    return torch.cuda.device(device)
