"""The C ABI library without a GPU: it loads, exports every symbol
include/moc_hip.h declares, sizes workspaces, and rejects bad arguments with the
documented status codes before touching the device."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from moc import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "moc_hip.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(moc_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _declared()
    assert set(names) == set(_lib.EXPORTED_SYMBOLS)
    for name in names:
        assert hasattr(L, name), name
    assert L.moc_abi_version() == _lib.ABI_VERSION == 5


def test_header_constants_match_binding():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (MOC_\w+)\s+(-?\d+)", text))
    assert int(consts["MOC_DT_F32"]) == _lib.DT_F32
    assert int(consts["MOC_DT_BF16"]) == _lib.DT_BF16
    assert int(consts["MOC_DT_F16"]) == _lib.DT_F16
    assert int(consts["MOC_ROUTE_ALPHA"]) == _lib.ROUTE_ALPHA
    assert int(consts["MOC_ROUTE_SOFTMAX"]) == _lib.ROUTE_SOFTMAX
    assert int(consts["MOC_ROUTE_EXP"]) == _lib.ROUTE_EXP


def test_workspace_queries():
    L = _lib.lib()
    for x_dt in (_lib.DT_BF16, _lib.DT_F32):
        f = L.moc_forward_workspace_bytes(16384, 2048, 16, 4, x_dt, 1)
        b = L.moc_backward_workspace_bytes(16384, 2048, 16, 4, x_dt, 1)
        assert f % 256 == 0 and b % 256 == 0 and b >= f
    assert L.moc_forward_workspace_bytes(0, 2048, 16, 4, 1, 0) == 0
    assert L.moc_backward_workspace_bytes(16, -1, 16, 4, 1, 0) == 0


FAKE = 0x1000  # never dereferenced: every call below fails validation first
ERR_ARG, ERR_DTYPE, ERR_WORKSPACE = -1, -2, -3  # MOC_ERR_* of include/moc_hip.h


def _fwd(**kw):
    args = dict(x=FAKE, alpha=FAKE, basis=FAKE, y=FAKE, cu=None, cu64=0, n_seqs=0,
                n_tokens=8, seq_len=8, dim=16, k=4, ks=4, x_dt=1, a_dt=1, b_dt=1,
                act=0, route=0, ws=FAKE, ws_bytes=1 << 30, stream=None)
    args.update(kw)
    return _lib.lib().moc_forward(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(x_dt=2), -2),          # fp16 x is not a supported compute dtype
    (dict(a_dt=7), -2),
    (dict(b_dt=-1), -2),
    (dict(dim=0), -1),
    (dict(k=-3), -1),
    (dict(act=2), -1),
    (dict(route=5), -1),
    (dict(route=-1), -1),
    (dict(x=None), -1),
    (dict(seq_len=0), -1),
    (dict(cu=FAKE, n_seqs=0), -1),
    (dict(ws_bytes=16), -3),
])
def test_forward_rejects_bad_arguments(kw, code):
    assert _fwd(**kw) == code
    assert _lib.lib().moc_last_error().decode()


def test_status_maps_to_runtime_error():
    rc = _fwd(x_dt=5)
    with pytest.raises(RuntimeError, match="unsupported x dtype code 5"):
        _lib.check(rc, "moc_forward")


def test_backward_and_update_reject_bad_arguments():
    L = _lib.lib()
    rc = L.moc_backward(FAKE, FAKE, FAKE, FAKE, 16, None, None, FAKE, None, 0, 0, 8, 8, 16, 4, 4,
                        1, 1, 1, 0, 0, FAKE, 1 << 30, None)
    assert rc == -1 and b"null" in L.moc_last_error()
    rc = L.moc_backward(FAKE, FAKE, FAKE, FAKE, 16, None, FAKE, FAKE, None, 0, 0, 8, 8, 16, 4, 4,
                        1, 1, 1, 0, 0, FAKE, 8, None)
    assert rc == -3
    # dy rows are dim (contiguous) or 0 (one broadcast row) elements apart, or
    # -1 (one element for every token and channel)
    for bad in (7, -2):
        rc = L.moc_backward(FAKE, FAKE, FAKE, FAKE, bad, None, FAKE, FAKE, None, 0, 0, 8, 8, 16, 4,
                            4, 1, 1, 1, 0, 0, FAKE, 1 << 30, None)
        assert rc == -1 and b"dy_row_stride" in L.moc_last_error()
    # -1 passes the argument checks (the call then stops at the workspace size)
    rc = L.moc_backward(FAKE, FAKE, FAKE, FAKE, -1, None, FAKE, FAKE, None, 0, 0, 8, 8, 16, 4, 4,
                        1, 1, 1, 0, 0, FAKE, 8, None)
    assert rc == -3
    rc = L.moc_update(FAKE, FAKE, FAKE, FAKE, 64, 4, 1, FAKE, 70000, 16, 4, 4, 1, 1, 1, 0, 0, None)
    assert rc == -1
    rc = L.moc_update(FAKE, FAKE, FAKE, FAKE, 64, 4, 1, FAKE, 2, 16, 4, 4, 1, 9, 1, 0, 0, None)
    assert rc == -2


def test_dtype_codes():
    import torch
    assert _lib.dtype_code(torch.bfloat16) == 1
    with pytest.raises(TypeError):
        _lib.dtype_code(torch.int8)
    assert isinstance(_lib.lib(), ctypes.CDLL)


def test_router_grouped_rejects_bad_groups():
    """moc_router_forward_grouped validates its group arrays before any launch."""
    L = _lib.lib()

    def call(ks, routes, outs=None, n=None, Z=64):
        n = len(ks) if n is None else n
        m = max(n, 1)
        karr = (ctypes.c_int64 * m)(*ks)
        rarr = (ctypes.c_int * m)(*routes)
        ptrs = (ctypes.c_void_p * m)(*(outs if outs is not None else [FAKE] * m))
        return L.moc_router_forward_grouped(FAKE, FAKE, ctypes.addressof(ptrs),
                                            ctypes.addressof(karr), ctypes.addressof(rarr), n,
                                            100, Z, 1, None)

    assert call([16], [1], n=0) == -1
    assert call([16] * 5, [1] * 5) == -1            # more than 4 groups
    assert call([18], [1]) == -1                    # k % 4 != 0
    assert call([36], [1]) == -1                    # k > 32
    assert call([32, 32, 32, 4], [1, 1, 1, 1]) == -1  # 100 routes in all
    assert call([16], [3]) == -1                    # routing code
    assert call([16], [1], outs=[FAKE + 2]) == -1   # misaligned output
    assert call([16], [1], Z=48) == -1              # z_dim % 64 != 0
    assert b"group" in L.moc_last_error() or b"z_dim" in L.moc_last_error()


def test_kernel_path_switch():
    """moc_set_kernel_path returns the previous family and rejects unknown ones;
    the workspace size follows the family (generic kernels: fp32 scratch)."""
    L = _lib.lib()
    auto = L.moc_backward_workspace_bytes(4096, 256, 16, 4, _lib.DT_BF16, 1)
    assert L.moc_set_kernel_path(7) == -1 and b"kernel path" in L.moc_last_error()
    with _lib.kernel_path(_lib.PATH_GENERIC):
        assert L.moc_set_kernel_path(_lib.PATH_GENERIC) == _lib.PATH_GENERIC
        generic = L.moc_backward_workspace_bytes(4096, 256, 16, 4, _lib.DT_BF16, 1)
    assert L.moc_set_kernel_path(_lib.PATH_AUTO) == _lib.PATH_AUTO
    assert generic != auto and generic >= 4096 * 256 * 4


def test_backward_noalloc_rejects_before_touching_the_device():
    """The no-allocation backward validates like moc_backward and rejects a
    problem whose workspace exceeds its device scratch, before any device call."""
    L = _lib.lib()
    args = [FAKE, FAKE, FAKE, FAKE, 2048, FAKE, FAKE, FAKE, None, 0, 0]
    rc = L.moc_backward_noalloc(*args, 8, 8, 2048, 4, 4, 9, 1, 1, 0, 0, None)
    assert rc == -2 and b"x dtype" in L.moc_last_error()
    big = 1 << 20   # 1 M tokens x 2048 channels: partial sums far above the scratch
    need = L.moc_backward_workspace_bytes(big, 2048, 16, 4, _lib.DT_BF16, 3)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    rc = L.moc_backward_noalloc(*args, big, 4096, 2048, 16, 4, 1, 1, 1, 1, 3, None)
    assert rc == -3 and b"moc_backward_noalloc holds" in L.moc_last_error()
    small = L.moc_backward_workspace_bytes(16384, 2048, 16, 4, _lib.DT_BF16, 3)
    assert small <= _lib.NOALLOC_SCRATCH_BYTES    # the headline shape fits


def _layers(dims, k=32, activation=0, **kw):
    arr = (_lib.MocLayer * max(len(dims), 1))()
    for i, d in enumerate(dims):
        arr[i].x = arr[i].alpha = arr[i].basis = arr[i].y = FAKE
        arr[i].dy = arr[i].dx = arr[i].dalpha = arr[i].dbasis = FAKE
        arr[i].dy_row_stride = d
        arr[i].dim = d
        arr[i].routing = 3
        arr[i].alpha_dtype = arr[i].basis_dtype = _lib.DT_BF16
        arr[i].k = k[i] if isinstance(k, list) else k
        arr[i].activation = activation[i] if isinstance(activation, list) else activation
        for name, v in kw.items():
            setattr(arr[i], name, v)
    return arr


def test_layer_entries_validate_and_size():
    """moc_*_layers: argument checks before any launch; grouped bf16 layers need
    the per-layer workspaces side by side, each sized for its own k."""
    L = _lib.lib()
    dims = [4096, 1024, 1024]
    N, K, S = 16384, 32, 8
    for which in ("forward", "backward"):
        q = getattr(L, f"moc_{which}_layers_workspace_bytes")
        single = getattr(L, f"moc_{which}_workspace_bytes")
        # the single-layer queries cover either activation (no argument there);
        # with SiLU a single backward of these shapes also holds g for its
        # taps pass, which the grouped backward (the fused pass) does not
        total = sum(single(N, d, K, S, _lib.DT_BF16, 3) for d in dims)
        if which == "forward":
            assert q(_layers(dims, activation=1), 3, N, S, _lib.DT_BF16) == total
        else:
            assert 0 < q(_layers(dims, activation=1), 3, N, S, _lib.DT_BF16) <= total
        assert q(_layers(dims), 3, N, S, _lib.DT_BF16) <= total
        assert q(_layers(dims), 0, N, S, _lib.DT_BF16) == 0
        ks = [16, 32, 64]
        mixed = sum(single(N, d, k, S, _lib.DT_BF16, 3) for d, k in zip(dims, ks))
        if which == "forward":
            assert q(_layers(dims, k=ks, activation=[1, 0, 1]), 3, N, S, _lib.DT_BF16) == mixed
        arr = _layers(dims)
        fn = getattr(L, f"moc_{which}_layers")
        assert fn(arr, 5, None, 0, 0, N, N, S, 1, FAKE, 1 << 40, None) == -1
        assert b"n_layers" in L.moc_last_error()
        assert fn(arr, 3, None, 0, 0, N, N, S, 1, FAKE, 16, None) == -3
        assert fn(_layers(dims, k=0), 3, None, 0, 0, N, N, S, 1, FAKE, 1 << 40, None) == -1
        assert fn(_layers(dims, activation=2), 3, None, 0, 0, N, N, S, 1, FAKE, 1 << 40, None) == -1
    bad = _layers([64, 64], k=16, dy_row_stride=7)
    assert L.moc_backward_layers(bad, 2, None, 0, 0, 8, 8, 4, 1, FAKE, 1 << 30, None) == -1
    assert b"dy_row_stride" in L.moc_last_error()
    nul = _layers([64], k=16, dalpha=None)
    assert L.moc_backward_layers(nul, 1, None, 0, 0, 8, 8, 4, 1, FAKE, 1 << 30, None) == -1
    assert b"null" in L.moc_last_error()


def _pre_fwd(**kw):
    args = dict(x=FAKE, alpha=FAKE, basis=FAKE, y=FAKE, cache=FAKE, fin=None, n_seqs=2,
                seq_len=8, dim=16, k=4, ks=4, x_dt=1, a_dt=1, b_dt=1, act=0, route=0,
                ws=FAKE, ws_bytes=0, stream=None)
    args.update(kw)
    return _lib.lib().moc_forward_prefill(*args.values())


def _pre_bwd(**kw):
    args = dict(x=FAKE, alpha=FAKE, basis=FAKE, dy=FAKE, dys=16, cache=FAKE, dx=FAKE,
                dalpha=FAKE, dbasis=FAKE, dcache=FAKE, n_seqs=2, seq_len=8, dim=16, k=4, ks=4,
                x_dt=1, a_dt=1, b_dt=1, act=0, route=0, ws=FAKE, ws_bytes=0, stream=None)
    args.update(kw)
    return _lib.lib().moc_backward_prefill(*args.values())


def test_matrix_core_supported_names_the_kernel_family():
    """moc_matrix_core_supported: 1 for the shapes the matrix-core kernels are
    built for (forward: 2-16 taps, up to 32 routes or 64 with bf16 x, an even
    channel count; backward: the same up to 8 taps, and bf16 with up to 16
    routes up to 16 taps), 0 elsewhere and while the generic family is forced."""
    L = _lib.lib()
    bf, f32 = _lib.DT_BF16, _lib.DT_F32
    for bwd in (0, 1):
        assert L.moc_matrix_core_supported(1024, 2048, 16, 4, bf, bwd) == 1
        assert L.moc_matrix_core_supported(1024, 198, 16, 4, bf, bwd) == 1    # D % 4 == 2
        assert L.moc_matrix_core_supported(1024, 2050, 32, 8, f32, bwd) == 1
        assert L.moc_matrix_core_supported(1024, 197, 16, 4, bf, bwd) == 1    # D odd: padded copy
        assert L.moc_matrix_core_supported(1024, 197, 48, 12, f32, bwd) == 1  # padded, route parts
        assert L.moc_matrix_core_supported(1024, 197, 80, 4, bf, bwd) == 0     # past 64 routes
        assert L.moc_matrix_core_supported(1024, 2048, 64, 2, bf, bwd) == 1
        assert L.moc_matrix_core_supported(1024, 2048, 48, 12, f32, bwd) == 1  # fp32, route parts
        assert L.moc_matrix_core_supported(1024, 2048, 80, 12, f32, bwd) == 0  # past 64 routes
        assert L.moc_matrix_core_supported(1024, 2048, 16, 12, bf, bwd) == 1  # 9-16 taps, 16 routes
        assert L.moc_matrix_core_supported(1024, 2048, 16, 17, bf, bwd) == 0
        assert L.moc_matrix_core_supported(1024, 2048, 16, 1, bf, bwd) == 0
        assert L.moc_matrix_core_supported(1024, 2048, 16, 4, _lib.DT_F16, bwd) == 0
        assert L.moc_matrix_core_supported(0, 2048, 16, 4, bf, bwd) == 0
    # 9-16 taps: the forward for every route count (fp32 past 32 routes in
    # route halves), the backward for bf16 (past 16 routes per 16-route chunk)
    # and for fp32 (past 16 routes in parts of 16)
    assert L.moc_matrix_core_supported(1024, 2048, 32, 16, bf, 0) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 32, 16, bf, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 64, 9, bf, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 16, 9, f32, 0) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 16, 9, f32, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 16, 16, f32, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 32, 9, f32, 0) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 32, 9, f32, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 64, 16, f32, 0) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 64, 16, f32, 1) == 1
    # fp32 with 33-64 routes up to 8 taps: the forward, and the backward in two
    # route halves
    assert L.moc_matrix_core_supported(1024, 2048, 48, 4, f32, 0) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 48, 4, f32, 1) == 1
    assert L.moc_matrix_core_supported(1024, 2048, 64, 8, f32, 1) == 1
    with _lib.kernel_path(_lib.PATH_GENERIC):
        assert L.moc_matrix_core_supported(1024, 2048, 16, 4, bf, 0) == 0
        assert L.moc_matrix_core_supported(1024, 2048, 16, 4, bf, 1) == 0


def test_prefill_entries_validate_before_touching_the_device():
    """moc_prefill_supported's answer, and the prefill entries' status codes for
    bad arguments (every call below fails before a launch: the valid-shape ones
    with a zero-byte workspace)."""
    L = _lib.lib()
    assert L.moc_prefill_supported(2, 8, 16, 4, 4, _lib.DT_BF16, 1) == 1
    assert L.moc_prefill_supported(2, 3, 16, 4, 4, _lib.DT_BF16, 1) == 1   # T = S-1
    assert L.moc_prefill_supported(2, 2, 16, 4, 4, _lib.DT_BF16, 1) == 0   # T < S-1 with a cache
    assert L.moc_prefill_supported(2, 2, 16, 4, 4, _lib.DT_BF16, 0) == 1   # no cache: any T
    assert L.moc_prefill_supported(2, 8, 16, 4, 5, _lib.DT_BF16, 1) == 1   # S = 5
    assert L.moc_prefill_supported(2, 8, 16, 4, 9, _lib.DT_BF16, 1) == 0   # no prefill kernels at S = 9
    assert L.moc_prefill_supported(2, 8, 18, 4, 4, _lib.DT_BF16, 1) == 1   # D even
    assert L.moc_prefill_supported(2, 8, 17, 4, 4, _lib.DT_BF16, 1) == 0   # D odd
    assert L.moc_prefill_supported(2, 8, 16, 33, 4, _lib.DT_F32, 1) == 0   # K > 32 with fp32 x
    assert L.moc_prefill_supported(0, 8, 16, 4, 4, _lib.DT_BF16, 1) == 0
    fwd_need = L.moc_forward_workspace_bytes(16, 16, 4, 4, _lib.DT_BF16, 0)
    assert fwd_need > 0
    assert _pre_fwd() == ERR_WORKSPACE
    assert _pre_fwd(n_seqs=0) == ERR_ARG
    assert _pre_fwd(seq_len=2) == ERR_ARG
    assert b"kernel_size - 1" in L.moc_last_error()
    assert _pre_fwd(seq_len=2, cache=None) == ERR_WORKSPACE  # no cache: T = 2 is fine
    assert _pre_fwd(x_dt=_lib.DT_F16) == ERR_DTYPE
    assert _pre_fwd(ks=9, seq_len=9) == ERR_ARG
    assert _pre_fwd(x=None, ws_bytes=fwd_need) == ERR_ARG
    assert _pre_fwd(act=2) == ERR_ARG
    assert _pre_bwd() == ERR_WORKSPACE
    assert _pre_bwd(cache=None) == ERR_ARG
    assert _pre_bwd(dys=3) == ERR_ARG
    assert _pre_bwd(dalpha=None) == ERR_ARG
    assert _pre_bwd(seq_len=1) == ERR_ARG
    assert _pre_bwd(route=7) == ERR_ARG


def test_backward_workspace_query_covers_the_activation():
    """moc_backward_workspace_bytes has no activation argument: at 8 taps,
    32 routes, bf16 (two passes without SiLU, the fused pass with it) it gives
    at least what either plan needs, so it is no smaller than the 4-tap figure
    scaled by the taps (partials grow with S)."""
    L = _lib.lib()
    n = L.moc_backward_workspace_bytes(16384, 2048, 32, 8, _lib.DT_BF16, 0)
    assert n > 0 and n % 256 == 0
    assert n >= L.moc_backward_workspace_bytes(16384, 2048, 32, 4, _lib.DT_BF16, 0)
