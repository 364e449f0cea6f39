"""Loader and ctypes signatures for libjlust_hip.so (include/jlust_hip.h).

torch is imported before the library is opened: torch ships its own
libamdhip64.so.7 (same SONAME as ROCm's), so the library then binds to the HIP
runtime torch already loaded and device pointers are shared with torch's
allocator.  There is no fallback: if the library is missing the import of the
compute path fails loudly.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import torch  # noqa: F401  (must precede the HIP library, see module docstring)

from . import errors

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libjlust_hip.so")

ABI_VERSION = 2          # JLUST_HIP_ABI_VERSION of include/jlust_hip.h

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_D = ctypes.c_double
_F = ctypes.c_float

# Every symbol include/jlust_hip.h declares, with (restype, argtypes).
SIGNATURES = {
    "jlust_hip_version": (_INT, []),
    "jlust_hip_last_error": (ctypes.c_char_p, []),
    "jlust_hip_device_arch": (_INT, [ctypes.c_char_p, ctypes.c_size_t]),
    "jlust_hip_preload": (_INT, [_P]),
    "jlust_hip_check_csr": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _INT]),
    "jlust_hip_check_pos_i32": (_INT, [_I64, _I64, _I32, _P, _P]),
    "jlust_hip_check_crd_i32": (_INT, [_I64, _I64, _I32, _INT, _P, _P]),
    "jlust_hip_expand_pos_i32": (_INT, [_I64, _I64, _I32, _P, _P, _P, _P]),
    "jlust_hip_row_order_i32": (_INT, [_I32, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P,
                                       ctypes.POINTER(_I32), _P]),
    "jlust_hip_gather_f64": (_INT, [_I64, _P, _P, _P, _P]),
    "jlust_hip_gather_f32": (_INT, [_I64, _P, _P, _P, _P]),
    "jlust_hip_csr_spmv_f64_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _D, _P, _P]),
    "jlust_hip_csr_spmv_f32_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _F, _P, _P]),
    "jlust_hip_csr_spmv_f64_i32_noalloc": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _D, _P,
                                                  _P]),
    "jlust_hip_csr_spmv_plan_create": (_INT, [_I64, _I64, _I64, _I32, _INT, _P, _P, _P, _P,
                                              ctypes.POINTER(_P)]),
    "jlust_hip_csr_spmv_plan_update_values": (_INT, [_P, _P, _P]),
    "jlust_hip_csr_spmv_plan_execute_f64": (_INT, [_P, _D, _P, _D, _P, _P]),
    "jlust_hip_csr_spmv_plan_execute_f32": (_INT, [_P, _F, _P, _F, _P, _P]),
    "jlust_hip_csr_spmv_plan_destroy": (_INT, [_P]),
    "jlust_hip_csr_spmv_plan_execute_values_f64": (_INT, [_P, _P, _D, _P, _D, _P, _P]),
    "jlust_hip_csr_spmv_plan_execute_values_f32": (_INT, [_P, _P, _F, _P, _F, _P, _P]),
    "jlust_hip_csr_spmv_plan_capture_f64": (_INT, [_P, _D, _P, _D, _P, ctypes.POINTER(_P)]),
    "jlust_hip_csr_spmv_plan_capture_f32": (_INT, [_P, _F, _P, _F, _P, ctypes.POINTER(_P)]),
    "jlust_hip_spmv_graph_launch": (_INT, [_P, _P]),
    "jlust_hip_spmv_graph_destroy": (_INT, [_P]),
    "jlust_hip_csr_spmv_plan_info": (_INT, [_P, ctypes.POINTER(_I32), ctypes.POINTER(_I32),
                                            ctypes.POINTER(_I64)]),
    "jlust_hip_coo_spmv_plan_create": (_INT, [_I64, _I64, _I64, _I32, _INT, _P, _P, _P, _P,
                                              ctypes.POINTER(_P)]),
    "jlust_hip_coo_spmv_f64_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _D, _P, _P]),
    "jlust_hip_coo_spmv_f32_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _F, _P, _P]),
    "jlust_hip_csr_spmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _I64,
                                          _D, _P, _I64, _INT, _P]),
    "jlust_hip_csr_spmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _I64,
                                          _F, _P, _I64, _INT, _P]),
    "jlust_hip_csr_sddmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _D, _P, _I64, _P,
                                           _I64, _D, _P, _P, _P]),
    "jlust_hip_csr_sddmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _F, _P, _I64, _P,
                                           _I64, _F, _P, _P, _P]),
    "jlust_hip_csr_spmm_plan_create": (_INT, [_I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _P, _P,
                                              ctypes.POINTER(_P)]),
    "jlust_hip_csr_spmm_plan_update_values": (_INT, [_P, _P, _P]),
    "jlust_hip_csr_spmm_plan_execute_f64": (_INT, [_P, _D, _P, _I64, _D, _P, _I64, _INT, _P]),
    "jlust_hip_csr_spmm_plan_execute_f32": (_INT, [_P, _F, _P, _I64, _F, _P, _I64, _INT, _P]),
    "jlust_hip_csr_spmm_plan_info": (_INT, [_P, ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                                            ctypes.POINTER(_I64), ctypes.POINTER(_I32)]),
    "jlust_hip_csr_spmm_plan_destroy": (_INT, [_P]),
    "jlust_hip_coo_spmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _I64, _D,
                                          _P, _I64, _P]),
    "jlust_hip_coo_spmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _I64, _F,
                                          _P, _I64, _P]),
    "jlust_hip_csc_spmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _I64, _D,
                                          _P, _I64, _P]),
    "jlust_hip_csc_spmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _I64, _F,
                                          _P, _I64, _P]),
    "jlust_hip_coo_spmm_plan_create": (_INT, [_I32, _I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _P, _P,
                                              ctypes.POINTER(_P)]),
    "jlust_hip_coo_sddmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _D, _P, _I64, _P,
                                           _I64, _D, _P, _P, _P]),
    "jlust_hip_coo_sddmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _F, _P, _I64, _P,
                                           _I64, _F, _P, _P, _P]),
    "jlust_hip_dcsr_sddmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _D, _P,
                                            _I64, _P, _I64, _D, _P, _P, _P]),
    "jlust_hip_dcsr_sddmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _F, _P,
                                            _I64, _P, _I64, _F, _P, _P, _P]),
    "jlust_hip_csc_sddmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _D, _P, _I64, _P,
                                           _I64, _D, _P, _P, _P]),
    "jlust_hip_csc_sddmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _F, _P, _I64, _P,
                                           _I64, _F, _P, _P, _P]),
    "jlust_hip_sddmm_plan_create": (_INT, [_I32, _I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _P,
                                           ctypes.POINTER(_P)]),
    "jlust_hip_dcsr_sddmm_plan_create": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _P,
                                                _P, ctypes.POINTER(_P)]),
    "jlust_hip_sddmm_plan_execute_f64": (_INT, [_P, _D, _P, _I64, _P, _I64, _D, _P, _P, _P]),
    "jlust_hip_sddmm_plan_execute_f32": (_INT, [_P, _F, _P, _I64, _P, _I64, _F, _P, _P, _P]),
    "jlust_hip_sddmm_plan_info": (_INT, [_P, ctypes.POINTER(_I64), ctypes.POINTER(_I32)]),
    "jlust_hip_sddmm_plan_destroy": (_INT, [_P]),
    "jlust_hip_csc_spmv_f64_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _D, _P, _D, _P, _P]),
    "jlust_hip_csc_spmv_f32_i32": (_INT, [_I64, _I64, _I64, _I32, _P, _P, _P, _F, _P, _F, _P, _P]),
    "jlust_hip_bsr_spmm_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _INT, _I64, _F,
                                          _P, _I64, _F, _P, _I64, _P]),
    "jlust_hip_bsr_spmm_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _INT, _I64, _D,
                                          _P, _I64, _D, _P, _I64, _P]),
    "jlust_hip_bsr_spmv_f64_i32": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _INT, _D, _P, _D,
                                          _P, _P]),
    "jlust_hip_bsr_spmv_f32_i32": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _INT, _F, _P, _F,
                                          _P, _P]),
    "jlust_hip_bsr_expand_csr_i32": (_INT, [_I64, _I64, _I64, _I64, _I32, _P, _P, _P, _INT, _INT, _P, _P,
                                            _P, _P]),
    "jlust_hip_bsr_spmm_plan_create": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _INT, _INT, _P, _P, _P, _I64,
                                              _P, ctypes.POINTER(_P)]),
    "jlust_hip_bsr_spmm_plan_update_values": (_INT, [_P, _P, _P]),
    "jlust_hip_bsr_spmm_plan_execute_f32": (_INT, [_P, _F, _P, _I64, _F, _P, _I64, _P]),
    "jlust_hip_bsr_spmm_plan_execute_f64": (_INT, [_P, _D, _P, _I64, _D, _P, _I64, _P]),
    "jlust_hip_bsr_spmm_plan_info": (_INT, [_P, ctypes.POINTER(_I32)]),
    "jlust_hip_bsr_spmm_plan_destroy": (_INT, [_P]),
    "jlust_hip_bsr_spmv_plan_create": (_INT, [_I64, _I64, _I64, _I64, _I64, _I32, _INT, _INT, _P, _P, _P, _P,
                                              ctypes.POINTER(_P)]),
    "jlust_hip_bsr_spmv_plan_update_values": (_INT, [_P, _P, _P]),
    "jlust_hip_bsr_spmv_plan_execute_f64": (_INT, [_P, _D, _P, _D, _P, _P]),
    "jlust_hip_bsr_spmv_plan_execute_f32": (_INT, [_P, _F, _P, _F, _P, _P]),
    "jlust_hip_bsr_spmv_plan_destroy": (_INT, [_P]),
    "jlust_hip_narrow_index_i64": (_INT, [_I64, _P, _P, _P]),
    "jlust_hip_convert_analyze": (_INT, [_P, _I32, _I32, _I32, _I32, _INT, _P, ctypes.POINTER(_P),
                                         ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "jlust_hip_convert_fill": (_INT, [_P, _P, _P]),
    "jlust_hip_convert_destroy": (_INT, [_P]),
    "jlust_hip_sparse_to_dense": (_INT, [_P, _INT, _P, _I64, _P]),
    "jlust_hip_shift_index": (_INT, [_P, _P, _I64, _I32, _P]),
    "jlust_hip_csr_assemble": (_INT, [_I64, _I64, _I32, _P, _INT, _P, _P, _P, _I64, _P]),
    "jlust_hip_scatter_values": (_INT, [_P, _I64, _P, _P, _I64, _INT, _P]),
    "jlust_hip_bbm_periodic_spmv_f64": (_INT, [_I64, _I64, _I64, _I64, _P, _P, _P, _D, _P, _D, _P, _P]),
    "jlust_hip_bbm_periodic_spmv_f32": (_INT, [_I64, _I64, _I64, _I64, _P, _P, _P, _F, _P, _F, _P, _P]),
    "jlust_hip_shifted_diag_spmv_f64": (_INT, [_I64, _I64, _I64, _D, _D, _P, _D, _P, _P]),
    "jlust_hip_shifted_diag_spmv_f32": (_INT, [_I64, _I64, _I64, _F, _F, _P, _F, _P, _P]),
    "jlust_hip_shifted_diag_spmm_f64": (_INT, [_I64, _I64, _I64, _I64, _D, _D, _P, _I64, _D, _P, _I64,
                                               _P]),
    "jlust_hip_shifted_diag_spmm_f32": (_INT, [_I64, _I64, _I64, _I64, _F, _F, _P, _I64, _F, _P, _I64,
                                               _P]),
    "jlust_hip_apply_fn_f64": (_INT, [_I64, _I32, _D, _D, _P, _D, _D, _P, _P]),
    "jlust_hip_apply_fn_f32": (_INT, [_I64, _I32, _F, _F, _P, _F, _F, _P, _P]),
    "jlust_hip_gather_rows_f64": (_INT, [_I64, _I64, _I32, _P, _I64, _P, _I64, _P, _I64, _P]),
    "jlust_hip_gather_rows_f32": (_INT, [_I64, _I64, _I32, _P, _I64, _P, _I64, _P, _I64, _P]),
    "jlust_hip_scatter_rows_f64": (_INT, [_I64, _I64, _I32, _P, _I64, _P, _I64, _P, _I64, _P]),
    "jlust_hip_scatter_rows_f32": (_INT, [_I64, _I64, _I32, _P, _I64, _P, _I64, _P, _I64, _P]),
}

STATUS = {
    0: "SUCCESS", 1: "INVALID_ARGUMENT", 2: "UNSUPPORTED_VALUE_TYPE", 3: "UNSUPPORTED_FORMAT",
    4: "NONCANONICAL_STORAGE", 5: "INDEX_ORIGIN", 6: "HIP_ERROR", 7: "NO_DEVICE",
    8: "OUT_OF_MEMORY", 9: "STREAM_CAPTURING", 10: "UNSUPPORTED_INDEX_TYPE",
}
STREAM_CAPTURING = 9

_lib = None

# Per-call device plumbing, kept cheap for microsecond-scale products: torch's
# raw current-stream handle and current-device index where this torch build
# exposes them (the public Stream / device-guard objects cost several
# microseconds per call), else the public API.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_CUR_DEVICE = getattr(torch._C, "_cuda_getDevice", None)
_NO_GUARD = contextlib.nullcontext()


def stream_handle(dev: torch.device) -> ctypes.c_void_p:
    """The current stream of `dev` as a hipStream_t."""
    if _RAW_STREAM is not None and dev.index is not None:
        return ctypes.c_void_p(_RAW_STREAM(dev.index))
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def on_device(dev: torch.device):
    """torch.cuda.device(dev), or no guard when dev is already current."""
    if _CUR_DEVICE is not None and dev.index is not None and _CUR_DEVICE() == dev.index:
        return _NO_GUARD
    return torch.cuda.device(dev)


def lib():
    """Open libjlust_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m jlust_amd.build` "
                "(the sparse operators have no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.jlust_hip_version() != ABI_VERSION:
            raise RuntimeError("libjlust_hip.so ABI version mismatch")
        _lib = L
    return _lib


def last_error() -> str:
    return lib().jlust_hip_last_error().decode(errors="replace")


def check(status: int, what: str, fmt=None, backend=None, T=None):
    """Raise the JLUST exception that corresponds to a C ABI status code."""
    if status == 0:
        return
    msg = f"{what}: {last_error()}"
    if status == 1:
        raise errors.IncompatibleExtents(msg)
    if status == 2:
        raise errors.UnsupportedValueType(T, backend, msg)
    if status == 3:
        raise errors.UnsupportedFormat(fmt, backend, msg)
    if status == 4:
        raise errors.NonCanonicalStorage(msg)
    if status == 5:
        raise errors.IndexOriginMismatch("origin", msg)
    if status == 7:
        raise errors.NoDevice(msg)
    if status == 8:
        raise MemoryError(msg)
    if status == 10:
        raise errors.UnsupportedIndexType(T, backend, msg)
    raise errors.HIPError(f"{STATUS.get(status, status)}: {msg}")


def preload(device=None) -> None:
    """Load the library's device code on `device` (default: the current one)
    now rather than at the first call that needs each part
    (jlust_hip_preload): a server pays the runtime's one-time code-object
    loading at start-up instead of in its first prepared plan."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    with on_device(dev):
        check(lib().jlust_hip_preload(stream_handle(dev)), "preload")
