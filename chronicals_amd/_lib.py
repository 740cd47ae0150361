"""ctypes binding of libchronicals_cce.so (declared in include/chronicals_cce.h).

Loading fails loudly: there is no CPU or PyTorch fallback for this path.
"""
from __future__ import annotations

import ctypes
import os
import threading

from . import build as _build

# constants mirrored from include/chronicals_cce.h
CCE_ABI_VERSION = 7
CCE_OK = 0
CCE_ERR_INVALID_ARG = 1
CCE_ERR_WORKSPACE = 2
CCE_ERR_HIP = 3
CCE_REDUCTION_NONE = 0
CCE_REDUCTION_MEAN = 1
CCE_REDUCTION_SUM = 2
CCE_DTYPE_BF16 = 0
CCE_DTYPE_F32 = 1
CCE_DTYPE_F16 = 2
CCE_SMOOTH_LOGV = 0
CCE_SMOOTH_UNIFORM = 1
CCE_LSE_ALL_ROWS = 0
CCE_LSE_LABELLED_ROWS = 1
CCE_NOALLOC_SCRATCH_BYTES = 64 << 20

CCE_KERNEL_FWD_LSE = 0
CCE_KERNEL_BWD_GRAD = 1
CCE_KERNEL_BWD_DH = 2
CCE_KERNEL_BWD_DW = 3
CCE_KERNEL_BWD_DHDW = 4
CCE_KERNEL_BWD_BAND = 5
CCE_KERNEL_LOGITS_FWD = 6
CCE_KERNEL_LOGITS_BWD = 7
CCE_KERNEL_LOGITS_FUSED = 8
CCE_KERNEL_KINDS = 9
KERNEL_KIND_NAMES = {CCE_KERNEL_FWD_LSE: "fwd_lse", CCE_KERNEL_BWD_GRAD: "bwd_grad", CCE_KERNEL_BWD_DH: "bwd_dh",
                     CCE_KERNEL_BWD_DW: "bwd_dw", CCE_KERNEL_BWD_DHDW: "bwd_dhdw", CCE_KERNEL_BWD_BAND: "bwd_band",
                     CCE_KERNEL_LOGITS_FWD: "logits_fwd", CCE_KERNEL_LOGITS_BWD: "logits_bwd",
                     CCE_KERNEL_LOGITS_FUSED: "logits_fused"}

REDUCTIONS = {"none": CCE_REDUCTION_NONE, "mean": CCE_REDUCTION_MEAN, "sum": CCE_REDUCTION_SUM}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "cce_abi_version": (_i32, []),
    "cce_source_hash": (ctypes.c_char_p, []),
    "cce_last_error": (ctypes.c_char_p, []),
    "cce_forward_workspace_bytes": (_i32, [_i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_sz)]),
    "cce_backward_workspace_bytes": (_i32, [_i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, ctypes.POINTER(_sz)]),
    "cce_forward": (_i32, [
        _vp, _vp, _vp, _i32, _vp,            # hidden, weight, labels, labels_int64, bias
        _i64, _i64, _i64, _i64,              # N, d, V, ignore_index
        _f32, _f32, _i32, _i32, _i32,        # label_smoothing, z_loss_weight, smoothing_form, reduction, lse_rows
        _vp, _vp, _vp, _vp,                  # loss_out, lse_out, target_out, n_valid_out
        _vp, _sz, _vp,                       # workspace, workspace_bytes, stream
    ]),
    "cce_forward_noalloc": (_i32, [
        _vp, _vp, _vp, _i32, _vp,            # hidden, weight, labels, labels_int64, bias
        _i64, _i64, _i64, _i64,              # N, d, V, ignore_index
        _f32, _f32, _i32, _i32, _i32,        # label_smoothing, z_loss_weight, smoothing_form, reduction, lse_rows
        _vp, _vp, _vp, _vp,                  # loss_out, lse_out, target_out, n_valid_out
        _vp,                                 # stream
    ]),
    "cce_backward": (_i32, [
        _vp, _vp, _vp, _vp, _i32, _vp,       # grad_out, hidden, weight, labels, labels_int64, bias
        _vp, _vp,                            # lse, n_valid
        _i64, _i64, _i64, _i64,              # N, d, V, ignore_index
        _f32, _f32, _i32, _i64,              # label_smoothing, z_loss_weight, reduction, chunk_size
        _vp, _i32, _vp, _i32, _vp,           # grad_hidden, dtype, grad_weight, dtype, grad_bias
        _vp, _sz, _vp,                       # workspace, workspace_bytes, stream
    ]),
    "cce_logits_forward_workspace_bytes": (_i32, [_i64, _i64, _i32, ctypes.POINTER(_sz)]),
    "cce_logits_forward": (_i32, [
        _vp, _i32, _i64, _vp, _i32,          # logits, dtype, ld, labels, labels_int64
        _i64, _i64, _i64,                    # N, V, ignore_index
        _f32, _f32, _i32, _i32,              # label_smoothing, z_loss_weight, smoothing_form, reduction
        _vp, _vp, _vp,                       # loss_out, lse_out, n_valid_out
        _vp, _sz, _vp,                       # workspace, workspace_bytes, stream
    ]),
    "cce_logits_backward": (_i32, [
        _vp, _vp, _i32, _i64, _vp, _i32,     # grad_out, logits, dtype, ld, labels, labels_int64
        _vp, _vp, _i64, _i64, _i64,          # lse, n_valid, N, V, ignore_index
        _f32, _f32, _i32, _i32,              # label_smoothing, z_loss_weight, smoothing_form, reduction
        _vp, _i32, _i64, _vp,                # grad_logits, grad_dtype, ld_grad, stream
    ]),
    "cce_logits_forward_backward": (_i32, [
        _vp, _i32, _i64, _vp, _i32,          # logits, dtype, ld, labels, labels_int64
        _i64, _i64, _i64,                    # N, V, ignore_index
        _f32, _f32, _i32, _i32, _i32,        # label_smoothing, z_loss_weight, smoothing_form, reduction, grad_mean
        _vp, _vp, _vp,                       # loss_out, lse_out, n_valid_out
        _vp, _i32, _i64,                     # grad_logits, grad_dtype, ld_grad
        _vp, _sz, _vp,                       # workspace, workspace_bytes, stream
    ]),
    "cce_kernel_timing_enable": (_i32, [_i32]),
    "cce_kernel_timing_read": (_i32, [_i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64),
                                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
}

_lock = threading.Lock()
_lib = None


class CCEError(RuntimeError):
    """A non-zero return from libchronicals_cce."""


def lib_path() -> str:
    """The library to load: CHRONICALS_CCE_LIB when set and non-empty, else the in-tree build."""
    return os.environ.get("CHRONICALS_CCE_LIB") or _build.LIB_PATH


def check_fresh(lib: ctypes.CDLL, path: str) -> None:
    """Refuse an in-tree library that was built from other sources than the
    tree's (a stale build).  A library named by CHRONICALS_CCE_LIB is the
    caller's explicit choice and is not checked; neither is a tree without
    its sources."""
    if os.path.abspath(path) != os.path.abspath(_build.LIB_PATH):
        return
    if not (os.path.exists(_build.SRC) and os.path.exists(_build.HEADER)):
        return
    built = (lib.cce_source_hash() or b"").decode()
    want = _build.source_hash()
    if built != want:
        raise ImportError(
            f"{path} was built from other sources (library {built[:16]}, tree {want[:16]}): "
            f"rebuild it with `python -m chronicals_amd.build` (or __graft_entry__.build())"
        )


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built or
    was built from other sources than the tree's."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise ImportError(
                f"libchronicals_cce.so not found at {path}: build it with "
                f"`python -m chronicals_amd.build` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                raise ImportError(f"{path} does not export {name} (an older build?): rebuild it with "
                                  f"`python -m chronicals_amd.build` (or __graft_entry__.build())") from None
            fn.restype = res
            fn.argtypes = args
        ver = lib.cce_abi_version()
        if ver != CCE_ABI_VERSION:
            raise ImportError(f"libchronicals_cce ABI version {ver}, expected {CCE_ABI_VERSION}")
        check_fresh(lib, path)
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != CCE_OK:
        msg = load().cce_last_error()
        raise CCEError(f"libchronicals_cce error {rc}: {msg.decode() if msg else ''}")


def forward_workspace_bytes(N: int, d: int, V: int, reduction: int, lse_rows: int = CCE_LSE_ALL_ROWS) -> int:
    out = _sz(0)
    check(load().cce_forward_workspace_bytes(N, d, V, reduction, lse_rows, ctypes.byref(out)))
    return out.value


def backward_workspace_bytes(N: int, d: int, V: int, chunk_size: int, need_dh: bool, need_dw: bool,
                             dh_f32: bool = False, dw_f32: bool = False) -> int:
    out = _sz(0)
    check(load().cce_backward_workspace_bytes(N, d, V, chunk_size, int(need_dh),
                                              CCE_DTYPE_F32 if dh_f32 else CCE_DTYPE_BF16, int(need_dw),
                                              CCE_DTYPE_F32 if dw_f32 else CCE_DTYPE_BF16, ctypes.byref(out)))
    return out.value


def logits_forward_workspace_bytes(N: int, V: int, reduction: int) -> int:
    out = _sz(0)
    check(load().cce_logits_forward_workspace_bytes(N, V, reduction, ctypes.byref(out)))
    return out.value


def kernel_timing_enable(enable: bool) -> None:
    check(load().cce_kernel_timing_enable(int(enable)))


def kernel_timing_read(kind: int):
    """(total milliseconds, launches, credited FLOPs, executed FLOPs) recorded for one
    kernel kind since the last read."""
    ms = ctypes.c_double(0.0)
    n = _i64(0)
    cr = ctypes.c_double(0.0)
    ex = ctypes.c_double(0.0)
    check(load().cce_kernel_timing_read(kind, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(cr), ctypes.byref(ex)))
    return ms.value, n.value, cr.value, ex.value
