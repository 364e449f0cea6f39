"""Format conversions of device tensors through the C ABI (include/jlust_hip.h).

Mirrors the reference's conversion API: ``convert_format(u, fmt)``
(src/convert.jl:302-388), ``convert_index_type`` / ``convert_value_type``
(:392-396), ``sparse_to_dense`` (ext/KernelAbstractionsExt/ops/conversion.jl:
47-65), ``csc_tensor`` / ``dcsr_tensor`` (src/interop.jl:220-314) and the
origin shift of ``materialize`` (ext/CUDAExt/CUDAExt.jl:199-220).  Results are
the reference's bit for bit: explicit zeros dropped, stable lexicographic
order on the target's levels, adjacent duplicates on unique levels reduced to
their first value, the source's index origin kept.

Everything runs on the HIP device; host-resident tensors raise
UnsupportedFormat (the product has no CPU path).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .errors import UnsupportedFormat, UnsupportedValueType
from .formats import Formats, TensorFormat, bsr_blocksize, is_bsr
from .tensor import AbstractIndexOrigin, OneBased, USTensor, _as_torch

FMT_CSR, FMT_CSC, FMT_COO, FMT_DCSR, FMT_BSR = 0, 1, 2, 3, 4
_VT = {torch.float64: 0, torch.float32: 1}


class Sparse(ctypes.Structure):
    """struct jlust_sparse."""
    _fields_ = [("format", ctypes.c_int32), ("origin", ctypes.c_int32),
                ("m", ctypes.c_int64), ("n", ctypes.c_int64),
                ("b1", ctypes.c_int32), ("b2", ctypes.c_int32),
                ("row_major_blocks", ctypes.c_int32),
                ("nnz", ctypes.c_int64), ("nouter", ctypes.c_int64),
                ("pos1", ctypes.c_void_p), ("crd1", ctypes.c_void_p),
                ("pos2", ctypes.c_void_p), ("crd2", ctypes.c_void_p),
                ("val", ctypes.c_void_p)]


def _format_id(fmt: TensorFormat):
    """(format id, b1, b2, row_major) of a supported format."""
    if is_bsr(fmt):
        b1, b2, rm = bsr_blocksize(fmt)
        return FMT_BSR, b1, b2, rm
    for fid, f in ((FMT_CSR, Formats.CSR), (FMT_CSC, Formats.CSC), (FMT_COO, Formats.COO),
                   (FMT_DCSR, Formats.DCSR)):
        if fmt == f:
            return fid, 0, 0, True
    raise UnsupportedFormat(fmt.name, "HIPBackend",
                            "format conversion supports CSR, CSC, COO, DCSR and BSR")


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _descriptor(u: USTensor) -> Sparse:
    fid, b1, b2, rm = _format_id(u.format)
    m, n = u.extents
    d = Sparse(format=fid, origin=u.origin.offset, m=m, n=n, b1=b1, b2=b2,
               row_major_blocks=int(rm), nnz=u.val.numel())
    pos, crd = u.pos_buffers, u.crd_buffers
    if fid in (FMT_CSR, FMT_CSC):
        d.pos2, d.crd2 = _ptr(pos[1]), _ptr(crd[1])
    elif fid == FMT_COO:
        d.crd1, d.crd2 = _ptr(crd[0]), _ptr(crd[1])
    elif fid == FMT_DCSR:
        d.nouter = crd[0].numel()
        d.crd1, d.pos2, d.crd2 = _ptr(crd[0]), _ptr(pos[1]), _ptr(crd[1])
    else:
        d.nouter = crd[1].numel()
        d.pos2, d.crd2 = _ptr(pos[1]), _ptr(crd[1])
    d.val = _ptr(u.val)
    return d


def _device_of(u: USTensor) -> torch.device:
    dev = u.val.device
    if dev.type != "cuda":
        raise UnsupportedFormat(u.format.name, "HIPBackend",
                                "format conversion runs on the HIP device; materialize the tensor "
                                "to HIPDevice first")
    for b in (*u.pos_buffers, *u.crd_buffers):
        if b is not None and b.device != dev:
            raise UnsupportedFormat(u.format.name, "HIPBackend", "buffers on several devices")
        if b is not None and b.dtype != torch.int32:
            raise UnsupportedFormat(u.format.name, "HIPBackend", "index buffers must be Int32")
    return dev


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def convert_format(u: USTensor, fmt: TensorFormat, index_type=None, value_type=None) -> USTensor:
    """src/convert.jl:302-388 on the device: a new tensor in `fmt` with u's origin."""
    if index_type not in (None, torch.int32):
        raise UnsupportedFormat(u.format.name, "HIPBackend", "conversions produce Int32 indices only")
    if value_type not in (None, u.val.dtype):
        raise UnsupportedValueType(value_type, "HIPBackend", "conversion keeps the value type")
    if u.val.dtype not in _VT:
        raise UnsupportedValueType(u.val.dtype, "HIPBackend", "conversion moves Float64 or Float32 values")
    dev = _device_of(u)
    src = _descriptor(u)
    fid, b1, b2, rm = _format_id(fmt)
    L = _lib.lib()
    h = ctypes.c_void_p()
    nnz_out, nouter = ctypes.c_int64(), ctypes.c_int64()
    with torch.cuda.device(dev):
        st = L.jlust_hip_convert_analyze(ctypes.byref(src), fid, b1, b2, int(rm), _VT[u.val.dtype],
                                         _stream(dev), ctypes.byref(h), ctypes.byref(nnz_out),
                                         ctypes.byref(nouter))
        _lib.check(st, "convert_analyze", fmt)
        try:
            m, n = u.extents
            o = u.origin.offset
            nz, no = nnz_out.value, nouter.value
            i32 = dict(dtype=torch.int32, device=dev)
            val = torch.empty(nz, dtype=u.val.dtype, device=dev)
            dst = Sparse(format=fid, origin=o, m=m, n=n, b1=b1, b2=b2, row_major_blocks=int(rm),
                         nnz=nz, nouter=no)
            dst.val = _ptr(val)
            if fid in (FMT_CSR, FMT_CSC):
                ptr = torch.empty((m if fid == FMT_CSR else n) + 1, **i32)
                crd = torch.empty(nz, **i32)
                dst.pos2, dst.crd2 = ptr.data_ptr(), _ptr(crd)
                pos_b, crd_b = (None, ptr), (None, crd)
            elif fid == FMT_COO:
                pos1 = torch.empty(2, **i32)
                rows, cols = torch.empty(nz, **i32), torch.empty(nz, **i32)
                dst.pos1, dst.crd1, dst.crd2 = pos1.data_ptr(), _ptr(rows), _ptr(cols)
                pos_b, crd_b = (pos1, None), (rows, cols)
            elif fid == FMT_DCSR:
                pos1 = torch.empty(2, **i32)
                outer, inner_pos = torch.empty(no, **i32), torch.empty(no + 1, **i32)
                inner = torch.empty(nz, **i32)
                dst.pos1, dst.crd1 = pos1.data_ptr(), _ptr(outer)
                dst.pos2, dst.crd2 = inner_pos.data_ptr(), _ptr(inner)
                pos_b, crd_b = (pos1, inner_pos), (outer, inner)
            else:
                browptr, bcol = torch.empty(m // b1 + 1, **i32), torch.empty(no, **i32)
                dst.pos2, dst.crd2 = browptr.data_ptr(), _ptr(bcol)
                pos_b, crd_b = (None, browptr, None, None), (None, bcol, None, None)
            st = L.jlust_hip_convert_fill(h, ctypes.byref(dst), _stream(dev))
            _lib.check(st, "convert_fill", fmt)
            torch.cuda.current_stream(dev).synchronize()
        finally:
            L.jlust_hip_convert_destroy(h)
    return USTensor((m, n), fmt, pos_b, crd_b, val, None, u.origin)


def convert_index_type(u: USTensor, index_type) -> USTensor:
    """src/convert.jl:392-393."""
    return convert_format(u, u.format, index_type=index_type)


def convert_value_type(u: USTensor, value_type) -> USTensor:
    """src/convert.jl:395-396."""
    return convert_format(u, u.format, value_type=value_type)


def sparse_to_dense(u: USTensor) -> torch.Tensor:
    """ext/KernelAbstractionsExt/ops/conversion.jl:47-65: an m x n column-major
    matrix with every stored entry scattered into zeros."""
    if u.val.dtype not in _VT:
        raise UnsupportedValueType(u.val.dtype, "HIPBackend", "sparse_to_dense moves Float64 or Float32 values")
    dev = _device_of(u)
    m, n = u.extents
    out = torch.empty((n, m), dtype=u.val.dtype, device=dev).t()
    src = _descriptor(u)
    with torch.cuda.device(dev):
        st = _lib.lib().jlust_hip_sparse_to_dense(ctypes.byref(src), _VT[u.val.dtype], _ptr(out),
                                                  max(m, 1), _stream(dev))
    _lib.check(st, "sparse_to_dense", u.format)
    return out


def shift_index(t: torch.Tensor, delta: int) -> torch.Tensor:
    """A new Int32 device buffer t + delta (materialize's origin change)."""
    if t.dtype != torch.int32 or t.device.type != "cuda":
        raise UnsupportedFormat(None, "HIPBackend", "shift_index takes Int32 device buffers only")
    t = t.contiguous()
    out = torch.empty_like(t)
    with torch.cuda.device(t.device):
        st = _lib.lib().jlust_hip_shift_index(_ptr(out), _ptr(t), t.numel(), int(delta),
                                              _stream(t.device))
    _lib.check(st, "shift_index", None)
    return out


def csc_tensor(colptr, rowind, nzval, dims, origin: AbstractIndexOrigin = OneBased()) -> USTensor:
    """src/interop.jl:220-230."""
    m, n = dims
    return USTensor((int(m), int(n)), Formats.CSC, (None, _as_torch(colptr)),
                    (None, _as_torch(rowind)), _as_torch(nzval), None, origin)


def dcsr_tensor(outer_crd, inner_pos, inner_crd, nzval, dims,
                origin: AbstractIndexOrigin = OneBased()) -> USTensor:
    """src/interop.jl:304-314: stored rows, their segments, columns, values."""
    m, n = dims
    return USTensor((int(m), int(n)), Formats.DCSR, (None, _as_torch(inner_pos)),
                    (_as_torch(outer_crd), _as_torch(inner_crd)), _as_torch(nzval), None, origin)
