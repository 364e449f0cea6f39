"""HIPBackend: execute/prepare for SpMV, SpMM and SDDMM over libjlust_hip.so.

The checks mirror what the reference raises before it launches
(validate_storage, src/backends.jl:309-316; the error types of
src/errors.jl): value type, index type, device, extents, buffer lengths.
Every compute call goes to the C ABI on torch's current stream; there is no
CPU path here.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from collections import OrderedDict

import torch

from . import _lib
from .errors import (DeviceMismatch, IncompatibleExtents, NonCanonicalStorage,
                     UnsupportedFormat, UnsupportedIndexType, UnsupportedValueType)
from .formats import (Formats, bsr_blocksize, is_bsr, is_coo_shaped, is_csc_shaped, is_csr_shaped,
                      is_periodic_csr, is_shifted_diag)
from .ops import AbstractKernelHandle, HIPBackend, Op, SDDMMOp, SpMMOp, SpMVOp
from .tensor import USTensor, dense_matrix, leading_dim, nnz, nonzeros, ust

_BE = HIPBackend()
_VALUE_TYPES = {torch.float64: "f64", torch.float32: "f32"}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


_stream = _lib.stream_handle
_on = _lib.on_device


def _dense_fmt(fmt) -> bool:
    return fmt.is_dense


# ---------------------------------------------------------------- capability

_SUPPORTS = {}


def supports(op: Op) -> bool:
    """Capability table (the counterpart of KernelAbstractionsExt.jl:31-41),
    memoised per (op, operand formats)."""
    key = (op.tag, op.formats)
    r = _SUPPORTS.get(key)
    if r is None:
        r = _SUPPORTS[key] = _supports(op)
    return r


def _supports(op: Op) -> bool:
    f = op.formats
    if op.tag == "SpMV" and len(f) == 3:
        return (is_csr_shaped(f[0]) or is_coo_shaped(f[0]) or is_csc_shaped(f[0]) or
                is_shifted_diag(f[0]) or f[0] == Formats.DCSR or is_periodic_csr(f[0]) or
                is_bsr(f[0])) and \
            _dense_fmt(f[1]) and \
            _dense_fmt(f[2]) and f[1].ndims == 1 and f[2].ndims == 1
    if op.tag == "SpMM" and len(f) == 3:
        a_ok = (is_csr_shaped(f[0]) or is_coo_shaped(f[0]) or is_csc_shaped(f[0]) or
                f[0] == Formats.DCSR or is_bsr(f[0]) or is_shifted_diag(f[0]) or is_periodic_csr(f[0]))
        return a_ok and _dense_fmt(f[1]) and _dense_fmt(f[2]) and f[1].ndims == 2 and \
            f[2].ndims == 2
    if op.tag == "SDDMM" and len(f) == 3:
        return _dense_fmt(f[0]) and _dense_fmt(f[1]) and \
            (is_csr_shaped(f[2]) or is_coo_shaped(f[2]) or is_csc_shaped(f[2]) or f[2] == Formats.DCSR)
    return False


# --------------------------------------------------------------------- checks

def _value_suffix(u: USTensor) -> str:
    s = _VALUE_TYPES.get(nonzeros(u).dtype)
    if s is None:
        raise UnsupportedValueType(nonzeros(u).dtype, _BE)
    return s


def _check_index(u: USTensor, *bufs):
    for b in bufs:
        if b.dtype != torch.int32:
            raise UnsupportedIndexType(b.dtype, _BE)
        if not b.is_contiguous():
            raise NonCanonicalStorage(f"{u.format} index buffers must be contiguous")


def _narrow_buffer(u: USTensor, b):
    """An Int64 index buffer narrowed to Int32 on the device
    (jlust_hip_narrow_index_i64), once per torch version of it: the copy is
    kept on the buffer object, so it lives as long as the buffer does."""
    if b is None or b.dtype != torch.int64:
        return b
    c = b.__dict__.get("_jlust_i32")
    if c is not None and c[0] == b._version:
        return c[1]
    if not b.is_contiguous():
        raise NonCanonicalStorage(f"{u.format} index buffers must be contiguous")
    dev = _check_same_device(b)
    out = torch.empty(b.shape, dtype=torch.int32, device=dev)
    with _on(dev):
        st = _lib.lib().jlust_hip_narrow_index_i64(b.numel(), _ptr(b), _ptr(out), _stream(dev))
    _lib.check(st, "narrow_index", u.format, _BE, b.dtype)
    b.__dict__["_jlust_i32"] = (b._version, out)
    return out


def _narrowed(u):
    """u itself, or, when it holds Int64 index buffers, the same tensor over
    their Int32 narrowing (the walker keeps the index type as stored,
    ext/KernelAbstractionsExt/ops/_walker.jl:105-110; the kernels take
    Int32).  The values are shared, so results written into them are the
    caller's.  The wrapper is kept on u while its Int64 buffers are unchanged
    (plans and checks cached on it keep applying); an index beyond Int32
    raises UnsupportedIndexType."""
    if not isinstance(u, USTensor):
        return u
    bufs = [b for b in (*u.pos_buffers, *u.crd_buffers) if b is not None and b.dtype == torch.int64]
    if not bufs:
        return u
    key = tuple((id(b), b._version) for b in bufs) + (id(u.val),)
    c = u.__dict__.get("_jlust_narrowed")
    if c is not None and c[0] == key:
        return c[1]
    n = USTensor(u.extents, u.format, tuple(_narrow_buffer(u, b) for b in u.pos_buffers),
                 tuple(_narrow_buffer(u, b) for b in u.crd_buffers), u.val, u.owner, u.origin)
    u.__dict__["_jlust_narrowed"] = (key, n)
    return n


def _check_same_device(*ts):
    devs = {t.device for t in ts if t is not None}
    if len(devs) != 1:
        raise DeviceMismatch(f"operands on several devices: {sorted(map(str, devs))}")
    dev = devs.pop()
    if dev.type != "cuda":
        raise DeviceMismatch(f"HIPBackend needs GPU buffers, got {dev}")
    return dev


def _check_values(u: USTensor, T):
    v = nonzeros(u)
    if v.dtype != T:
        raise UnsupportedValueType(v.dtype, _BE, f"operands must share the value type {T}")
    if not v.is_contiguous():
        raise NonCanonicalStorage("value buffers must be contiguous")


def _checked_once(t: torch.Tensor, key, check):
    """Run check() (a device-side structural check that raises on bad
    storage) once per (tensor, key) and torch version of the tensor: an index
    buffer written in place through torch is checked again, one that is not is
    checked once.  The record lives on the tensor object."""
    done = t.__dict__.get("_jlust_checked")
    if done is not None and done.get(key) == t._version:
        return
    check()
    if done is None:
        done = t.__dict__["_jlust_checked"] = {}
    done[key] = t._version


def _check_pos_once(u: USTensor, pos: torch.Tensor, nouter: int, nnz_: int, dev):
    """pos[nouter+1] from the origin to nnz + origin, never decreasing
    (jlust_hip_check_pos_i32), checked once per version of pos."""
    def run():
        with _on(dev):
            st = _lib.lib().jlust_hip_check_pos_i32(nouter, nnz_, u.origin.offset, _ptr(pos), _stream(dev))
        _lib.check(st, "check_pos", u.format, _BE)
    _checked_once(pos, ("pos", nouter, nnz_, u.origin.offset), run)


def _check_crd_once(u: USTensor, crd: torch.Tensor, extent: int, strict: bool, dev):
    """Coordinates within [origin, extent + origin) (strictly increasing when
    `strict`; jlust_hip_check_crd_i32), checked once per version of crd."""
    def run():
        with _on(dev):
            st = _lib.lib().jlust_hip_check_crd_i32(crd.numel(), extent, u.origin.offset, int(strict),
                                                     _ptr(crd), _stream(dev))
        _lib.check(st, "check_crd", u.format, _BE)
    _checked_once(crd, ("crd", extent, bool(strict), u.origin.offset), run)


def _csr_parts(u: USTensor):
    rowptr, colind = u.pos_buffers[1], u.crd_buffers[1]
    if rowptr is None or colind is None:
        raise NonCanonicalStorage(f"{u.format}: missing level-2 pos/crd buffer")
    _check_index(u, rowptr, colind)
    m, n = u.extents
    if rowptr.numel() != m + 1:
        raise NonCanonicalStorage(f"rowptr has {rowptr.numel()} entries, expected m+1 = {m + 1}")
    if colind.numel() != nnz(u):
        raise NonCanonicalStorage(
            f"val buffer length {nnz(u)} != nnz {colind.numel()} (backend=HIPBackend)")
    return rowptr, colind


# -------------------------------------------------------------------- execute

def execute(op: Op, *ts, alpha=1.0, beta=0.0, input_fn=None, output_fn=None,
            skip_empty_rows=False, mask=None):
    from .elementwise import is_identity
    if not supports(op):
        raise UnsupportedFormat(op.formats, _BE)
    nts = tuple(_narrowed(t) for t in ts)
    if any(a is not b for a, b in zip(nts, ts)):
        # Int64 index buffers: the product runs on their Int32 narrowing; an
        # operand returned is the caller's own tensor.
        r = execute(op, *nts, alpha=alpha, beta=beta, input_fn=input_fn, output_fn=output_fn,
                    skip_empty_rows=skip_empty_rows, mask=_narrowed(mask))
        for a, b in zip(nts, ts):
            if r is a:
                return b
        return r
    if mask is not None and _narrowed(mask) is not mask:
        return execute(op, *ts, alpha=alpha, beta=beta, input_fn=input_fn, output_fn=output_fn,
                       skip_empty_rows=skip_empty_rows, mask=_narrowed(mask))
    if op.tag == "SpMV":
        return spmv_with_fns(_spmv, *ts, alpha=alpha, beta=beta, input_fn=input_fn,
                             output_fn=output_fn)
    if not (is_identity(input_fn) and is_identity(output_fn)):
        raise UnsupportedFormat(op.formats, _BE, "input_fn/output_fn belong to SpMV")
    if op.tag == "SpMM":
        return _spmm(*ts, alpha=alpha, beta=beta, skip_empty_rows=skip_empty_rows)
    return _sddmm(*ts, alpha=alpha, beta=beta, mask=mask)


def spmv_with_fns(spmv, u_A, u_x, u_y, alpha=1.0, beta=0.0, input_fn=None, output_fn=None):
    """y = alpha*output_fn(A*input_fn.(x)) + beta*y (spmv.jl:371-374) around a
    plain SpMV `spmv(u_A, u_x, u_y, alpha, beta)`: in_fn.(x) into a new
    vector, the product into a row-sum vector when output_fn is given, then
    the row write on the device (jlust_amd/elementwise.py).  Strided
    vectors (a row of a column-major matrix, a stepped slice), which the
    reference's ust takes as any AbstractVector (src/interop.jl:36-46), pass
    through contiguous device copies, and y is copied back into its view."""
    x0, y0 = nonzeros(u_x), nonzeros(u_y)
    if (x0.dim() == 1 and not x0.is_contiguous()) or (y0.dim() == 1 and not y0.is_contiguous()):
        yc = y0.contiguous()
        spmv_with_fns(spmv, u_A, ust(x0.contiguous()), ust(yc), alpha, beta, input_fn, output_fn)
        if yc is not y0:
            y0.copy_(yc)
        return u_y
    if input_fn is None and output_fn is None:
        return spmv(u_A, u_x, u_y, alpha, beta)
    from .elementwise import apply_fn, is_identity
    if is_identity(input_fn) and is_identity(output_fn):
        return spmv(u_A, u_x, u_y, alpha, beta)
    x, y = _vec_checks(u_A, u_x, u_y)
    if not is_identity(output_fn) and (is_coo_shaped(u_A.format) or is_csc_shaped(u_A.format)):
        # The reference rejects output_fn where rows are accumulated by atomics
        # (scatter mode, spmv.jl:394-399); COO's and CSC's row sums are such
        # atomics here.
        raise UnsupportedFormat(u_A.format, _BE,
                                f"output_fn is unsupported for {u_A.format.name} SpMV; convert A to CSR first")
    if not is_identity(input_fn):
        x2 = torch.empty_like(x)
        apply_fn(input_fn, x, x2)
        u_x = ust(x2)
    if is_identity(output_fn):
        return spmv(u_A, u_x, u_y, alpha, beta)
    t = torch.empty_like(y)
    spmv(u_A, u_x, ust(t), 1.0, 0.0)
    apply_fn(output_fn, t, y, alpha, beta)
    return u_y


def _vec_checks(u_A, u_x, u_y):
    T = nonzeros(u_A).dtype
    x, y = nonzeros(u_x), nonzeros(u_y)
    _check_values(u_x, T)
    _check_values(u_y, T)
    m, n = u_A.extents
    if x.numel() != n or y.numel() != m:
        raise IncompatibleExtents(
            f"SpMV: A is {m}x{n}, x has {x.numel()} entries, y has {y.numel()}")
    return x, y


def _spmv(u_A: USTensor, u_x: USTensor, u_y: USTensor, alpha, beta):
    suf = _value_suffix(u_A)
    x, y = _vec_checks(u_A, u_x, u_y)
    m, n = u_A.extents
    L = _lib.lib()
    if u_A.format == Formats.DCSR:
        return _dcsr_product(u_A, u_x, u_y, alpha, beta)
    if is_periodic_csr(u_A.format):
        _periodic_spmv(u_A, x, y, alpha, beta)
        return u_y
    if is_bsr(u_A.format):
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u_A)
        _check_values(u_A, nonzeros(u_A).dtype)
        dev = _check_same_device(browptr, bcolind, nonzeros(u_A), x, y)
        # The kernel clamps malformed block pointers into range; they are
        # rejected here instead, once per version of the index buffers.
        _check_pos_once(u_A, browptr, mb, bcolind.numel(), dev)
        _check_crd_once(u_A, bcolind, nb, False, dev)
        if PLAN_CACHE.enabled and PLAN_CACHE.run(u_A, browptr, bcolind, dev, alpha, x, beta, y):
            return u_y
        with _on(dev):
            st = getattr(L, f"jlust_hip_bsr_spmv_{suf}_i32")(
                mb, nb, b1, b2, bcolind.numel(), u_A.origin.offset, _ptr(browptr), _ptr(bcolind),
                _ptr(nonzeros(u_A)), int(row_major), float(alpha), _ptr(x), float(beta), _ptr(y),
                _stream(dev))
        _lib.check(st, "bsr_spmv", u_A.format, _BE, nonzeros(u_A).dtype)
        return u_y
    if is_shifted_diag(u_A.format):
        lv = u_A.format.levels[1]
        dev = _check_same_device(x, y)
        with _on(dev):
            st = getattr(L, f"jlust_hip_shifted_diag_spmv_{suf}")(
                m, n, lv.shift, lv.val, float(alpha), _ptr(x), float(beta), _ptr(y), _stream(dev))
        _lib.check(st, "shifted_diag_spmv", u_A.format, _BE, nonzeros(u_A).dtype)
        return u_y
    if is_csr_shaped(u_A.format):
        rowptr, colind = _csr_parts(u_A)
        dev = _check_same_device(rowptr, colind, nonzeros(u_A), x, y)
        if PLAN_CACHE.enabled and PLAN_CACHE.run(u_A, rowptr, colind, dev, alpha, x, beta, y):
            return u_y
        with _on(dev):
            st = getattr(L, f"jlust_hip_csr_spmv_{suf}_i32")(
                m, n, nnz(u_A), u_A.origin.offset, _ptr(rowptr), _ptr(colind),
                _ptr(nonzeros(u_A)), float(alpha), _ptr(x), float(beta), _ptr(y), _stream(dev))
        _lib.check(st, "csr_spmv", u_A.format, _BE, nonzeros(u_A).dtype)
        return u_y
    if is_csc_shaped(u_A.format):
        colptr, rowind = _csc_parts(u_A)
        dev = _check_same_device(colptr, rowind, nonzeros(u_A), x, y)
        _check_pos_once(u_A, colptr, n, nnz(u_A), dev)
        if PLAN_CACHE.enabled and PLAN_CACHE.run(u_A, colptr, rowind, dev, alpha, x, beta, y):
            return u_y
        with _on(dev):
            st = getattr(L, f"jlust_hip_csc_spmv_{suf}_i32")(
                m, n, nnz(u_A), u_A.origin.offset, _ptr(colptr), _ptr(rowind), _ptr(nonzeros(u_A)),
                float(alpha), _ptr(x), float(beta), _ptr(y), _stream(dev))
        _lib.check(st, "csc_spmv", u_A.format, _BE, nonzeros(u_A).dtype)
        return u_y
    rows, cols = _coo_parts(u_A)
    dev = _check_same_device(rows, cols, nonzeros(u_A), x, y)
    if PLAN_CACHE.enabled and PLAN_CACHE.run(u_A, rows, cols, dev, alpha, x, beta, y):
        return u_y
    with _on(dev):
        st = getattr(L, f"jlust_hip_coo_spmv_{suf}_i32")(
            m, n, nnz(u_A), u_A.origin.offset, _ptr(rows), _ptr(cols), _ptr(nonzeros(u_A)),
            float(alpha), _ptr(x), float(beta), _ptr(y), _stream(dev))
    _lib.check(st, "coo_spmv", u_A.format, _BE, nonzeros(u_A).dtype)
    return u_y


def _csc_parts(u: USTensor):
    colptr, rowind = u.pos_buffers[1], u.crd_buffers[1]
    if colptr is None or rowind is None:
        raise NonCanonicalStorage("CSC: missing level-2 pos/crd buffer")
    _check_index(u, colptr, rowind)
    n = u.extents[1]
    if colptr.numel() != n + 1 or rowind.numel() != nnz(u):
        raise NonCanonicalStorage(f"CSC: colptr needs n+1 = {n + 1} entries (got {colptr.numel()}) "
                                  f"and rowind nnz = {nnz(u)} (got {rowind.numel()})")
    return colptr, rowind


def _dcsr_parts(u: USTensor):
    rows, pos, cols = u.crd_buffers[0], u.pos_buffers[1], u.crd_buffers[1]
    if rows is None or pos is None or cols is None:
        raise NonCanonicalStorage("DCSR: missing level buffers")
    _check_index(u, rows, pos, cols)
    nout = rows.numel()
    if pos.numel() != nout + 1 or cols.numel() != nnz(u):
        raise NonCanonicalStorage(
            f"DCSR: {nout} stored rows need {nout + 1} segment pointers (got {pos.numel()}) and "
            f"{nnz(u)} columns (got {cols.numel()})")
    return rows, pos, cols


def _coo_parts(u: USTensor):
    rows, cols = u.crd_buffers[0], u.crd_buffers[1]
    if rows is None or cols is None:
        raise NonCanonicalStorage("COO: missing coordinate buffers")
    _check_index(u, rows, cols)
    if rows.numel() != nnz(u) or cols.numel() != nnz(u):
        raise NonCanonicalStorage("COO coordinate buffers must have nnz entries")
    return rows, cols


def _periodic_spmv(u_A: USTensor, x: torch.Tensor, y: torch.Tensor, alpha, beta):
    """PeriodicCSR SpMV (kron(I(T), block) * x, src/named_formats.jl:63-88)
    as one CSR SpMM of the block with the T column blocks of x as the
    columns of a column-major n_cols x T matrix and y as an m_b x T one:
    every row of the block is read once for all T periods."""
    lv = u_A.format.levels[0]
    T, nc = lv.periods, lv.n_cols
    br = u_A.format.levels[1].size
    block = USTensor((br, nc), Formats.CSR, (None, u_A.pos_buffers[2]), (None, u_A.crd_buffers[2]),
                     nonzeros(u_A), u_A.owner, u_A.origin)
    X = x.view(T, nc).t()                 # column t = x[t*nc : (t+1)*nc]
    Y = y.view(T, br).t()
    _spmm(block, ust(X), ust(Y), alpha, beta)
    return y


def _dcsr_product(u_A: USTensor, u_X: USTensor, u_Y: USTensor, alpha, beta):
    """DCSR SpMV/SpMM: the CSR product over the stored rows into a compact
    result, with y[rows] gathered first when beta != 0 and scattered back
    after, so rows that are not stored stay untouched (the walker writes
    stored rows only, spmv.jl:449-502; dcsr.hip)."""
    rows, pos, cols = _dcsr_parts(u_A)
    nout = rows.numel()
    m, n = u_A.extents
    Y = nonzeros(u_Y)
    dev = _check_same_device(rows, pos, cols, nonzeros(u_A), nonzeros(u_X), Y)
    if nout == 0:
        return u_Y
    compact = USTensor((nout, n), Formats.CSR, (None, pos), (None, cols), nonzeros(u_A),
                       u_A.owner, u_A.origin)
    vec = Y.dim() == 1
    k = 1 if vec else Y.shape[1]
    suf = _value_suffix(u_A)
    t = torch.empty(nout, dtype=Y.dtype, device=dev) if vec else \
        dense_matrix(nout, k, dtype=Y.dtype, device=dev)
    ldy = 1 if vec else leading_dim(Y)
    ldt = 1 if vec else leading_dim(t)
    L = _lib.lib()
    o = u_A.origin.offset
    if beta != 0:
        with _on(dev):
            st = getattr(L, f"jlust_hip_gather_rows_{suf}")(nout, k, o, _ptr(rows), m, _ptr(Y), ldy,
                                                            _ptr(t), ldt, _stream(dev))
        _lib.check(st, "gather_rows", u_A.format, _BE, Y.dtype)
    if vec:
        _spmv(compact, u_X, ust(t), alpha, beta)
    else:
        _spmm(compact, u_X, ust(t), alpha, beta)
    with _on(dev):
        st = getattr(L, f"jlust_hip_scatter_rows_{suf}")(nout, k, o, _ptr(rows), m, _ptr(t), ldt,
                                                         _ptr(Y), ldy, _stream(dev))
    _lib.check(st, "scatter_rows", u_A.format, _BE, Y.dtype)
    return u_Y


def _bsr_parts(u: USTensor):
    """(b1, b2, row_major, browptr, bcolind, mb, nb) of a BSR tensor, checked."""
    b1, b2, row_major = bsr_blocksize(u.format)
    browptr, bcolind = u.pos_buffers[1], u.crd_buffers[1]
    if browptr is None or bcolind is None:
        raise NonCanonicalStorage(f"{u.format}: missing level-2 pos/crd buffer")
    _check_index(u, browptr, bcolind)
    m, n = u.extents
    if m % b1 or n % b2:
        raise IncompatibleExtents(f"BSR extents {m}x{n} are not multiples of {b1}x{b2}")
    mb, nb = m // b1, n // b2
    if browptr.numel() != mb + 1 or nnz(u) != bcolind.numel() * b1 * b2:
        raise NonCanonicalStorage("BSR: browptr must have mb+1 entries and val nnzb*b1*b2")
    return b1, b2, row_major, browptr, bcolind, mb, nb


def _bsr_as_csr(u: USTensor) -> USTensor:
    """The BSR tensor expanded to CSR on the device (jlust_hip_bsr_expand_csr_i32):
    scalar rows in block order, every stored entry kept, the same origin."""
    suf = _value_suffix(u)
    b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u)
    v = nonzeros(u)
    if not v.is_contiguous():
        raise NonCanonicalStorage("value buffers must be contiguous")
    dev = _check_same_device(browptr, bcolind, v)
    total = bcolind.numel() * b1 * b2
    rowptr = torch.empty(mb * b1 + 1, dtype=torch.int32, device=dev)
    colind = torch.empty(total, dtype=torch.int32, device=dev)
    val = torch.empty(total, dtype=v.dtype, device=dev)
    with _on(dev):
        st = _lib.lib().jlust_hip_bsr_expand_csr_i32(
            mb, b1, b2, bcolind.numel(), u.origin.offset, _ptr(browptr), _ptr(bcolind), _ptr(v),
            0 if suf == "f64" else 1, int(row_major), _ptr(rowptr), _ptr(colind), _ptr(val),
            _stream(dev))
    _lib.check(st, "bsr_expand_csr", u.format, _BE, v.dtype)
    return USTensor(u.extents, Formats.CSR, (None, rowptr), (None, colind), val, None, u.origin)


def _spmm(u_A: USTensor, u_B: USTensor, u_C: USTensor, alpha, beta, skip_empty_rows=False):
    suf = _value_suffix(u_A)
    T = nonzeros(u_A).dtype
    B, C = nonzeros(u_B), nonzeros(u_C)
    if B.dtype != T or C.dtype != T:
        raise UnsupportedValueType(B.dtype if B.dtype != T else C.dtype, _BE)
    m, n = u_A.extents
    if B.shape[0] != n or C.shape[0] != m or B.shape[1] != C.shape[1]:
        raise IncompatibleExtents(
            f"SpMM: A is {m}x{n}, B is {tuple(B.shape)}, C is {tuple(C.shape)}")
    for t, nm in ((B, "B"), (C, "C")):
        if t.shape[0] > 1 and t.shape[1] > 0 and t.stride(0) != 1:
            raise NonCanonicalStorage(f"SpMM: {nm} must be column-major (stride(0) == 1)")
    k = B.shape[1]
    L = _lib.lib()
    if u_A.format == Formats.DCSR:
        return _dcsr_product(u_A, u_B, u_C, alpha, beta)
    if is_coo_shaped(u_A.format) or is_csc_shaped(u_A.format):
        # COO (ColFirst) and CSC (scatter) in the reference, spmm.jl:331-335,
        # 412-416: here in row order through the CSR kernels.
        coo = is_coo_shaped(u_A.format)
        idx1, idx2 = _coo_parts(u_A) if coo else _csc_parts(u_A)
        dev = _check_same_device(idx1, idx2, nonzeros(u_A), B, C)
        if PLAN_CACHE.enabled and k > 0 and PLAN_CACHE.run_spmm(u_A, idx1, idx2, dev, alpha, B, beta, C):
            return u_C
        entry = f"jlust_hip_{'coo' if coo else 'csc'}_spmm_{suf}_i32"
        with _on(dev):
            st = getattr(L, entry)(m, n, k, nnz(u_A), u_A.origin.offset, _ptr(idx1), _ptr(idx2),
                                   _ptr(nonzeros(u_A)), float(alpha), _ptr(B), leading_dim(B), float(beta),
                                   _ptr(C), leading_dim(C), _stream(dev))
        _lib.check(st, entry[10:], u_A.format, _BE, T)
        return u_C
    if is_shifted_diag(u_A.format):
        lv = u_A.format.levels[1]
        dev = _check_same_device(B, C)
        with _on(dev):
            st = getattr(L, f"jlust_hip_shifted_diag_spmm_{suf}")(
                m, n, k, lv.shift, lv.val, float(alpha), _ptr(B), leading_dim(B), float(beta), _ptr(C),
                leading_dim(C), _stream(dev))
        _lib.check(st, "shifted_diag_spmm", u_A.format, _BE, T)
        return u_C
    if is_periodic_csr(u_A.format):
        # kron(I(T), block) * B: the block's CSR SpMM on each period's rows of B and C.
        lv = u_A.format.levels[0]
        nper, nc = lv.periods, lv.n_cols
        br = u_A.format.levels[1].size
        block = USTensor((br, nc), Formats.CSR, (None, u_A.pos_buffers[2]), (None, u_A.crd_buffers[2]),
                         nonzeros(u_A), u_A.owner, u_A.origin)
        for t in range(nper):
            _spmm(block, ust(B[t * nc:(t + 1) * nc, :]), ust(C[t * br:(t + 1) * br, :]), alpha, beta)
        return u_C
    if is_bsr(u_A.format):
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u_A)
        if (b1, b2) != (16, 16) or (suf == "f32" and row_major and nonzeros(u_A).data_ptr() % 16):
            # Blocks other than 16 x 16 (the MFMA kernels serve 16 x 16 blocks
            # only), and fp32 row-major blocks whose values are not 16-byte
            # aligned (the fp32 MFMA kernels load a block row as one float4):
            # the CSR expansion and the CSR SpMM, as the prepared BSR plan does.
            return _spmm(_bsr_as_csr(u_A), u_B, u_C, alpha, beta, skip_empty_rows)
        dev = _check_same_device(browptr, bcolind, nonzeros(u_A), B, C)
        with _on(dev):
            st = getattr(L, f"jlust_hip_bsr_spmm_{suf}_i32")(
                mb, nb, b1, bcolind.numel(), u_A.origin.offset, _ptr(browptr), _ptr(bcolind),
                _ptr(nonzeros(u_A)), int(row_major), k, float(alpha), _ptr(B), leading_dim(B),
                float(beta), _ptr(C), leading_dim(C), _stream(dev))
        _lib.check(st, "bsr_spmm", u_A.format, _BE, T)
        return u_C
    rowptr, colind = _csr_parts(u_A)
    dev = _check_same_device(rowptr, colind, nonzeros(u_A), B, C)
    with _on(dev):
        st = getattr(L, f"jlust_hip_csr_spmm_{suf}_i32")(
            m, n, k, nnz(u_A), u_A.origin.offset, _ptr(rowptr), _ptr(colind),
            _ptr(nonzeros(u_A)), float(alpha), _ptr(B), leading_dim(B), float(beta), _ptr(C),
            leading_dim(C), int(bool(skip_empty_rows)), _stream(dev))
    _lib.check(st, "csr_spmm", u_A.format, _BE, T)
    return u_C


def _sddmm(u_A: USTensor, u_B: USTensor, u_C: USTensor, alpha, beta, mask=None):
    suf = _value_suffix(u_C)
    T = nonzeros(u_C).dtype
    A, B = _sddmm_dense_checks(u_A, u_B, u_C)
    m, n = u_C.extents
    K = A.shape[1]
    mk = _sddmm_mask(mask, u_C, T)
    if u_C.format == Formats.DCSR:
        # The walker's compressed outer level binds the stored row
        # (sddmm.jl:49-65 with _walker.jl:323-392).
        rows, pos, cols = _dcsr_parts(u_C)
        dev = _check_same_device(rows, pos, cols, nonzeros(u_C), A, B, mk)
        _check_crd_once(u_C, rows, m, True, dev)
        _check_pos_once(u_C, pos, rows.numel(), nnz(u_C), dev)
        entry = f"jlust_hip_dcsr_sddmm_{suf}_i32"
        with _on(dev):
            st = getattr(_lib.lib(), entry)(
                m, n, K, rows.numel(), nnz(u_C), u_C.origin.offset, _ptr(rows), _ptr(pos), _ptr(cols),
                float(alpha), _ptr(A), leading_dim(A), _ptr(B), leading_dim(B), float(beta),
                _ptr(nonzeros(u_C)), _ptr(mk), _stream(dev))
        _lib.check(st, entry[10:], u_C.format, _BE, T)
        return u_C
    coo, csc = is_coo_shaped(u_C.format), is_csc_shaped(u_C.format)
    idx1, idx2 = _coo_parts(u_C) if coo else _csc_parts(u_C) if csc else _csr_parts(u_C)
    dev = _check_same_device(idx1, idx2, nonzeros(u_C), A, B, mk)
    entry = f"jlust_hip_{'coo' if coo else 'csc' if csc else 'csr'}_sddmm_{suf}_i32"
    with _on(dev):
        st = getattr(_lib.lib(), entry)(
            m, n, K, nnz(u_C), u_C.origin.offset, _ptr(idx1), _ptr(idx2), float(alpha),
            _ptr(A), leading_dim(A), _ptr(B), leading_dim(B), float(beta), _ptr(nonzeros(u_C)),
            _ptr(mk), _stream(dev))
    _lib.check(st, entry[10:], u_C.format, _BE, T)
    return u_C


def _sddmm_mask(mask, u_C: USTensor, T):
    """The optional S_ij factor: nnz(C) contiguous values of C's type, in
    C's storage order (a USTensor's values or a plain tensor)."""
    if mask is None:
        return None
    mk = nonzeros(mask) if isinstance(mask, USTensor) else mask
    if mk.dtype != T or mk.numel() != nnz(u_C) or not mk.is_contiguous():
        raise IncompatibleExtents("SDDMM: mask must hold nnz(C) contiguous values of C's type")
    return mk


def _sddmm_dense_checks(u_A: USTensor, u_B: USTensor, u_C: USTensor):
    T = nonzeros(u_C).dtype
    A, B = nonzeros(u_A), nonzeros(u_B)
    if A.dtype != T or B.dtype != T:
        raise UnsupportedValueType(A.dtype if A.dtype != T else B.dtype, _BE)
    m, n = u_C.extents
    if A.dim() != 2 or B.dim() != 2 or A.shape[0] != m or B.shape[1] != n or \
            A.shape[1] != B.shape[0]:
        raise IncompatibleExtents(
            f"SDDMM: C is {m}x{n}, A is {tuple(A.shape)}, B is {tuple(B.shape)}")
    for t, nm in ((A, "A"), (B, "B")):
        if t.shape[0] > 1 and t.shape[1] > 0 and t.stride(0) != 1:
            raise NonCanonicalStorage(f"SDDMM: {nm} must be column-major (stride(0) == 1)")
    return A, B


# ------------------------------------------------------------- plan cache

class _CachedPlan:
    """A prepared SpMV plan built for repeated plain calls on one matrix.  It
    holds weak references to the matrix's buffers only, so the caller's
    tensors are freed as usual; the plan is dropped when any of them is."""

    __slots__ = ("plan", "suf", "copies", "refs", "pat_ver", "val_ver", "bytes", "dev", "kind", "what",
                 "keep", "_exec", "_exec_values", "__weakref__")

    def __init__(self, u_A: USTensor, idx1, idx2, dev):
        vals = nonzeros(u_A)
        csc = is_csc_shaped(u_A.format)
        coo = is_coo_shaped(u_A.format) or csc
        self.suf = _value_suffix(u_A)
        self.dev = dev
        self.plan = ctypes.c_void_p(0)
        m, n = u_A.extents
        rows, cols = idx1, idx2
        self.keep = None
        if csc:
            # A CSC matrix is planned as COO: its row indices, and each entry's
            # column expanded from colptr (kept: a plan whose rows need no
            # reordering reads its columns in place).
            rows = idx2
            cols = torch.empty(nnz(u_A), dtype=torch.int32, device=vals.device)
            with _on(dev):
                st = _lib.lib().jlust_hip_expand_pos_i32(n, nnz(u_A), u_A.origin.offset, _ptr(idx1), None,
                                                         _ptr(cols), _stream(dev))
            _lib.check(st, "expand_pos", u_A.format, _BE, vals.dtype)
            self.keep = cols
        create = "jlust_hip_coo_spmv_plan_create" if coo else "jlust_hip_csr_spmv_plan_create"
        with _on(dev):
            st = getattr(_lib.lib(), create)(
                m, n, nnz(u_A), u_A.origin.offset, 0 if self.suf == "f64" else 1, _ptr(rows), _ptr(cols),
                _ptr(vals), _stream(dev), ctypes.byref(self.plan))
        _lib.check(st, create[10:], u_A.format, _BE, vals.dtype)
        k, lpr, nb = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
        _lib.check(_lib.lib().jlust_hip_csr_spmv_plan_info(self.plan, ctypes.byref(k), ctypes.byref(lpr),
                                                            ctypes.byref(nb)), "csr_spmv_plan_info")
        self.kind = ("merge", "vector", "sliced", "binned")[k.value]
        self.what = "csr_spmv_plan_execute"
        self.bytes = nb.value
        # Sliced and binned layouts, and COO plans, run on a copy of the values.
        self.copies = coo or self.kind in ("sliced", "binned")
        self.refs = (weakref.ref(idx1), weakref.ref(idx2), weakref.ref(vals))
        self.pat_ver = (idx1._version, idx2._version)
        self.val_ver = vals._version
        L = _lib.lib()
        self._exec = getattr(L, f"jlust_hip_csr_spmv_plan_execute_{self.suf}")
        self._exec_values = getattr(L, f"jlust_hip_csr_spmv_plan_execute_values_{self.suf}")

    def valid(self, idx1, idx2, vals) -> bool:
        r1, r2, r3 = self.refs
        return (r1() is idx1 and r2() is idx2 and r3() is vals and
                (idx1._version, idx2._version) == self.pat_ver)

    def launch(self, alpha, x, beta, y, stream) -> int:
        vals = self.refs[2]()
        if vals._version != self.val_ver:
            # Written in place (or its storage replaced): a copying plan gathers
            # the values again, the others take the address again.
            st = self._exec_values(self.plan, vals.data_ptr() if vals.numel() else None, alpha, x, beta, y,
                                   stream)
            if st == 0:
                self.val_ver = vals._version
            return st
        return self._exec(self.plan, alpha, x, beta, y, stream)

    def destroy(self):
        plan, self.plan = self.plan, ctypes.c_void_p(0)
        if plan.value:
            try:
                _lib.lib().jlust_hip_csr_spmv_plan_destroy(plan)
            except Exception:
                pass


class _CachedBSRPlan:
    """A BSR SpMV plan (jlust_hip_bsr_spmv_plan_*: the block-rows' segment
    table, built once) for repeated plain calls on one matrix, with
    _CachedPlan's interface and weak references only.  The plan reads the
    values in place at every call."""

    __slots__ = ("plan", "refs", "pat_ver", "bytes", "dev", "kind", "what", "_exec", "__weakref__")

    def __init__(self, u_A: USTensor, idx1, idx2, dev):
        vals = nonzeros(u_A)
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u_A)
        suf = _value_suffix(u_A)
        self.dev = dev
        self.plan = ctypes.c_void_p(0)
        with _on(dev):
            st = _lib.lib().jlust_hip_bsr_spmv_plan_create(
                mb, nb, b1, b2, bcolind.numel(), u_A.origin.offset, 0 if suf == "f64" else 1, int(row_major),
                _ptr(browptr), _ptr(bcolind), _ptr(vals), _stream(dev), ctypes.byref(self.plan))
        _lib.check(st, "bsr_spmv_plan_create", u_A.format, _BE, vals.dtype)
        nseg = mb + (bcolind.numel() + 31) // 32         # segments of at most 32 blocks
        self.bytes = 4 * (mb + 1) + 4 * nseg + nseg * b1 * vals.element_size()
        self.kind = "bsr_segments"
        self.what = "bsr_spmv_plan_execute"
        self.refs = (weakref.ref(idx1), weakref.ref(idx2), weakref.ref(vals))
        self.pat_ver = (idx1._version, idx2._version)
        self._exec = getattr(_lib.lib(), f"jlust_hip_bsr_spmv_plan_execute_{suf}")

    def valid(self, idx1, idx2, vals) -> bool:
        r1, r2, r3 = self.refs
        return (r1() is idx1 and r2() is idx2 and r3() is vals and
                (idx1._version, idx2._version) == self.pat_ver)

    def launch(self, alpha, x, beta, y, stream) -> int:
        return self._exec(self.plan, alpha, x, beta, y, stream)

    def destroy(self):
        plan, self.plan = self.plan, ctypes.c_void_p(0)
        if plan.value:
            try:
                _lib.lib().jlust_hip_bsr_spmv_plan_destroy(plan)
            except Exception:
                pass


class _CachedSpMMPlan:
    """A COO or CSC SpMM plan (jlust_hip_coo_spmm_plan_create: the entries put
    in row order once, the column chunking chosen for k) for repeated plain
    SpMM calls on one matrix and column count, with _CachedPlan's interface
    and weak references only.  A reordered plan holds the values in its row
    order and gathers them again when A's value tensor was written since."""

    __slots__ = ("plan", "suf", "refs", "pat_ver", "val_ver", "copies", "bytes", "dev", "kind", "what",
                 "_exec", "__weakref__")

    def __init__(self, u_A: USTensor, idx1, idx2, dev, k: int):
        vals = nonzeros(u_A)
        coo = is_coo_shaped(u_A.format)
        m, n = u_A.extents
        self.suf = _value_suffix(u_A)
        self.dev = dev
        self.plan = ctypes.c_void_p(0)
        with _on(dev):
            st = _lib.lib().jlust_hip_coo_spmm_plan_create(
                2 if coo else 1, m, n, k, nnz(u_A), u_A.origin.offset, 0 if self.suf == "f64" else 1,
                _ptr(idx1), _ptr(idx2), _ptr(vals), _stream(dev), ctypes.byref(self.plan))
        _lib.check(st, "coo_spmm_plan_create", u_A.format, _BE, vals.dtype)
        a, b, c, r = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        _lib.check(_lib.lib().jlust_hip_csr_spmm_plan_info(self.plan, ctypes.byref(a), ctypes.byref(b),
                                                            ctypes.byref(c), ctypes.byref(r)), "csr_spmm_plan_info")
        self.copies = bool(r.value)
        t = vals.element_size()
        # its device memory, within padding: B's column chunk in row order, the
        # entries in row order (and their values), the split rows' partial rows
        self.bytes = n * c.value * t + 4 * (m + 1) + nnz(u_A) * (8 + t) + m + b.value * c.value * t
        self.kind = "coo_spmm" if coo else "csc_spmm"
        self.what = "csr_spmm_plan_execute"
        self.refs = (weakref.ref(idx1), weakref.ref(idx2), weakref.ref(vals))
        self.pat_ver = (idx1._version, idx2._version)
        self.val_ver = vals._version
        self._exec = getattr(_lib.lib(), f"jlust_hip_csr_spmm_plan_execute_{self.suf}")

    def valid(self, idx1, idx2, vals) -> bool:
        r1, r2, r3 = self.refs
        return (r1() is idx1 and r2() is idx2 and r3() is vals and
                (idx1._version, idx2._version) == self.pat_ver)

    def launch(self, alpha, B, ldb, beta, C, ldc, stream) -> int:
        vals = self.refs[2]()
        if self.copies and vals._version != self.val_ver:
            st = _lib.lib().jlust_hip_csr_spmm_plan_update_values(self.plan, vals.data_ptr(), stream)
            if st:
                return st
            self.val_ver = vals._version
        return self._exec(self.plan, alpha, B, ldb, beta, C, ldc, 0, stream)

    def destroy(self):
        plan, self.plan = self.plan, ctypes.c_void_p(0)
        if plan.value:
            try:
                _lib.lib().jlust_hip_csr_spmm_plan_destroy(plan)
            except Exception:
                pass


class PlanCache:
    """Prepared plans for repeated plain SpMV calls, execute(SpMVOp, A, x, y)
    with a CSR, COO, CSC or BSR A (CSC planned as COO; for BSR, the
    block-rows' segment table), and for
    repeated plain SpMM calls with a COO or CSC A (one plan per column count)
    -- the counterpart of the reference's per-matrix cache of compiled views
    in its GPU mul! (ext/CUDAExt/ops/block_mul.jl:53,227,327-357).  A matrix is recognised by its index and value tensors (the same
    objects and device addresses, index tensors not written since: torch's
    version counters).  Its first `after` plain calls run the plain kernels;
    the next one builds a plan (the analysis a prepare would do) and every
    later call runs it.  Values written in place into the value tensor are
    read again as a prepared handle does; an index tensor written in place, a
    new tensor, or a freed one drops the plan.  At most `max_plans` plans and
    `max_bytes` bytes of plan memory are kept (least recently used first out).
    A plan's kernel may sum a row in another order than the plain call's, so
    results can change in their last bits, within the parity bar, at the call
    that switches.  Environment: JLUST_HIP_PLAN_CACHE=0 turns it off;
    JLUST_HIP_PLAN_CACHE_AFTER (default 2), JLUST_HIP_PLAN_CACHE_PLANS (8),
    JLUST_HIP_PLAN_CACHE_BYTES (8 GiB)."""

    def __init__(self):
        env = os.environ.get
        self.enabled = env("JLUST_HIP_PLAN_CACHE", "1") != "0"
        self.after = int(env("JLUST_HIP_PLAN_CACHE_AFTER", "2"))
        self.max_plans = int(env("JLUST_HIP_PLAN_CACHE_PLANS", "8"))
        self.max_bytes = int(env("JLUST_HIP_PLAN_CACHE_BYTES", str(8 << 30)))
        self._seen = OrderedDict()     # key -> (plain calls so far, weak refs of the buffers)
        self._plans = OrderedDict()    # key -> _CachedPlan, least recently used first
        self._bytes = 0

    @staticmethod
    def _key(u_A, idx1, idx2, vals, dev, stream):
        # The stream is part of the key: a plan's partial sums are not shared
        # between streams, as the plain call's scratch is not.
        # The format: a CSC matrix and a CSR one on the same buffers are each
        # other's transposes.
        f = u_A.format
        kind = ("bsr",) + tuple(_bsr_parts(u_A)[:3]) if is_bsr(f) else \
            "coo" if is_coo_shaped(f) else "csc" if is_csc_shaped(f) else "csr"
        return (idx1.data_ptr(), idx2.data_ptr(), vals.data_ptr(), u_A.extents, nnz(u_A),
                u_A.origin.offset, vals.dtype, dev.index, kind, stream.value)

    def _entry(self, u_A: USTensor, idx1, idx2, dev, extra, make):
        """(key, the cached plan of this matrix and `extra`), built by `make`
        at the call after the first `after` plain ones; the plan is None while
        the caller should make the plain call."""
        vals = nonzeros(u_A)
        stream = _stream(dev)
        base = self._key(u_A, idx1, idx2, vals, dev, stream)
        key = base[:-1] + (extra,) + base[-1:]         # the stream stays last (the fast path reads it)
        ent = self._plans.get(key)
        if ent is not None:
            if not ent.valid(idx1, idx2, vals):
                self._drop(key)
                ent = None
            else:
                self._plans.move_to_end(key)
        if ent is None:
            seen = self._seen.get(key)
            refs = (weakref.ref(idx1), weakref.ref(idx2), weakref.ref(vals))
            if seen is None or not all(r() is t for r, t in zip(seen[1], (idx1, idx2, vals))) or \
                    seen[2] != (idx1._version, idx2._version):
                self._seen[key] = (1, refs, (idx1._version, idx2._version))
                self._trim_seen()
                return key, None
            count = seen[0] + 1
            if count <= self.after or torch.cuda.is_current_stream_capturing():
                # (no plan is built while the stream is captured: a build allocates and synchronises)
                self._seen[key] = (count, refs, seen[2])
                return key, None
            del self._seen[key]
            ent = make()
            self._plans[key] = ent
            self._bytes += ent.bytes
            for t in (idx1, idx2, vals):
                fin = weakref.finalize(t, _plan_cache_forget, weakref.ref(self), key, weakref.ref(ent))
                fin.atexit = False             # nothing to give back at interpreter exit
            self._trim()
            if key not in self._plans:         # larger than the whole budget
                return key, None
        return key, ent

    def run(self, u_A: USTensor, idx1, idx2, dev, alpha, x, beta, y, fast=None) -> bool:
        """Run the product through a cached plan and return True, or return
        False (the caller makes the plain call).  `fast`: the fast path's
        record of this matrix, which keeps the plan it runs."""
        kind = _CachedBSRPlan if is_bsr(u_A.format) else _CachedPlan
        key, ent = self._entry(u_A, idx1, idx2, dev, None, lambda: kind(u_A, idx1, idx2, dev))
        if ent is None:
            return False
        if fast is not None:
            fast.key, fast.ent = key, ent
        with _on(dev):
            st = ent.launch(float(alpha), x.data_ptr(), float(beta), y.data_ptr(), _stream(dev))
        _lib.check(st, ent.what, u_A.format, _BE, nonzeros(u_A).dtype)
        return True

    def run_spmm(self, u_A: USTensor, idx1, idx2, dev, alpha, B, beta, C) -> bool:
        """The same for a plain COO or CSC SpMM C = alpha A B + beta C, one plan
        per matrix and column count k."""
        k = B.shape[1]
        key, ent = self._entry(u_A, idx1, idx2, dev, ("spmm", k),
                               lambda: _CachedSpMMPlan(u_A, idx1, idx2, dev, k))
        if ent is None:
            return False
        with _on(dev):
            st = ent.launch(float(alpha), B.data_ptr(), leading_dim(B), float(beta), C.data_ptr(),
                            leading_dim(C), _stream(dev))
        _lib.check(st, ent.what, u_A.format, _BE, nonzeros(u_A).dtype)
        return True

    def _trim_seen(self):
        while len(self._seen) > 64:
            self._seen.popitem(last=False)

    def _trim(self):
        while self._plans and (len(self._plans) > self.max_plans or self._bytes > self.max_bytes):
            self._drop(next(iter(self._plans)))

    def _drop(self, key):
        ent = self._plans.pop(key, None)
        if ent is not None:
            self._bytes -= ent.bytes
            ent.destroy()

    def forget(self, key, ent):
        if self._plans.get(key) is ent:
            self._drop(key)

    def clear(self):
        """Destroy every cached plan (their device memory is given back)."""
        for key in list(self._plans):
            self._drop(key)
        self._seen.clear()

    def info(self) -> list:
        """One dict per cached plan: its kernel, device bytes and extents."""
        return [{"kernel": e.kind, "device_bytes": e.bytes, "extents": k[3], "nnz": k[4]}
                for k, e in self._plans.items()]


class _SpMVFast:
    """What the plain SpMV fast path keeps about one CSR/COO USTensor: its
    buffers as checked once (identity-compared at every call), the device,
    value type and entry point, and the cached plan it last ran."""

    __slots__ = ("pos", "crd", "val", "fmt", "origin", "extents", "idx1", "idx2", "dev", "di", "T", "m",
                 "n", "coo", "plain", "key", "ent")

    def matches(self, u: USTensor) -> bool:
        return (u.val is self.val and u.pos_buffers is self.pos and u.crd_buffers is self.crd and
                u.format is self.fmt and u.origin is self.origin and u.extents is self.extents)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_DENSE1 = Formats.DensedRight(1)


def spmv_fast(u_A: USTensor, x: torch.Tensor, y: torch.Tensor, alpha, beta):
    """execute(SpMVOp, A, x, y; alpha, beta) for a CSR or COO A on the GPU and
    plain contiguous device vectors of its value type: the checks of the
    general path done once per matrix and then reduced to identity and
    attribute compares, the plan cache consulted directly.  Returns the
    output USTensor, or None when the call needs the general path (which then
    raises or handles what this one does not)."""
    u_A = _narrowed(u_A)
    st = u_A.__dict__.get("_hip_spmv")
    if st is None or not st.matches(u_A):
        st = _spmv_fast_state(u_A)
        if st is None:
            return None
    di = st.di
    if (x.dtype is not st.T or y.dtype is not st.T or x.get_device() != di or y.get_device() != di or
            x.numel() != st.n or y.numel() != st.m or not x.is_contiguous() or not y.is_contiguous() or
            _RAW_STREAM is None):
        return None
    if st.m == 0:
        return None
    stream = _RAW_STREAM(di)
    with _on(st.dev):
        ent = st.ent
        if (ent is not None and ent.plan.value and (st.key[-1] or 0) == stream and PLAN_CACHE.enabled and
                PLAN_CACHE._plans.get(st.key) is ent and ent.valid(st.idx1, st.idx2, st.val)):
            PLAN_CACHE._plans.move_to_end(st.key)
            status = ent.launch(float(alpha), x.data_ptr(), float(beta), y.data_ptr(), stream)
            if status:
                _lib.check(status, "csr_spmv_plan_execute", u_A.format, _BE, st.T)
        elif not (PLAN_CACHE.enabled and
                  PLAN_CACHE.run(u_A, st.idx1, st.idx2, st.dev, alpha, x, beta, y, fast=st)):
            status = st.plain(st.m, st.n, st.val.numel(), st.origin.offset, st.idx1.data_ptr(),
                              st.idx2.data_ptr(), st.val.data_ptr(), alpha, x.data_ptr(), beta,
                              y.data_ptr(), stream)
            if status:
                _lib.check(status, "coo_spmv" if st.coo else "csr_spmv", u_A.format, _BE, st.T)
    return USTensor((st.m,), _DENSE1, (None,), (None,), y, y)     # ust(y), built directly


def _spmv_fast_state(u_A: USTensor):
    """Check a matrix once for the fast path (the general path's checks) and
    record it on the USTensor; None when the fast path does not apply."""
    f = u_A.format
    coo = is_coo_shaped(f)
    if not (is_csr_shaped(f) or coo):
        return None
    try:
        suf = _value_suffix(u_A)
        idx1, idx2 = _coo_parts(u_A) if coo else _csr_parts(u_A)
        _check_values(u_A, nonzeros(u_A).dtype)
        dev = _check_same_device(idx1, idx2, nonzeros(u_A))
    except Exception:
        return None                           # the general path raises it
    st = _SpMVFast()
    st.pos, st.crd, st.val, st.fmt = u_A.pos_buffers, u_A.crd_buffers, u_A.val, u_A.format
    st.origin, st.extents = u_A.origin, u_A.extents
    st.idx1, st.idx2, st.dev, st.di = idx1, idx2, dev, dev.index
    st.T = nonzeros(u_A).dtype
    st.m, st.n = u_A.extents
    st.coo = coo
    st.plain = getattr(_lib.lib(), f"jlust_hip_{'coo' if coo else 'csr'}_spmv_{suf}_i32")
    st.key, st.ent = None, None
    u_A.__dict__["_hip_spmv"] = st
    return st


def _plan_cache_forget(cache_ref, key, ent_ref):
    """A buffer of a cached matrix was freed: drop its plan (weakref.finalize
    callback; the cache and the entry are weakly held)."""
    cache, ent = cache_ref(), ent_ref()
    if cache is not None and ent is not None:
        cache.forget(key, ent)


PLAN_CACHE = PlanCache()


# -------------------------------------------------------------------- handles

class HIPSpMVHandle(AbstractKernelHandle):
    """Prepared CSR SpMV: the merge-path partition is computed once
    (prepare(::EmitterBackend, SpMVOp, A), ext/KernelAbstractionsExt/ops/
    spmv.jl:518-544; the cuSPARSE handle contract, ext/CUDAExt/ops/spmv.jl:7-83)."""

    def __init__(self, u_A: USTensor, input_fn=None, output_fn=None):
        coo = is_coo_shaped(u_A.format)
        if not (is_csr_shaped(u_A.format) or coo):
            raise UnsupportedFormat(u_A.format, _BE, "prepared SpMV plans take CSR or COO")
        if coo and output_fn is not None:
            raise UnsupportedFormat(u_A.format, _BE,
                                    "output_fn is unsupported for COO SpMV; convert A to CSR first")
        self.input_fn, self.output_fn = input_fn, output_fn
        suf = _value_suffix(u_A)
        if coo:
            rows, cols = u_A.crd_buffers[0], u_A.crd_buffers[1]
            _check_index(u_A, rows, cols)
            if rows.numel() != nnz(u_A) or cols.numel() != nnz(u_A):
                raise NonCanonicalStorage("COO coordinate buffers must have nnz entries")
            first, second = rows, cols
        else:
            first, second = _csr_parts(u_A)
        self.dev = _check_same_device(first, second, nonzeros(u_A))
        self.u_A = u_A                      # keeps the buffers alive (GC anchor)
        self.T = nonzeros(u_A).dtype
        self.suf = suf
        self._exec = None
        self._plan = ctypes.c_void_p(0)
        m, n = u_A.extents
        create = "jlust_hip_coo_spmv_plan_create" if coo else "jlust_hip_csr_spmv_plan_create"
        with _on(self.dev):
            st = getattr(_lib.lib(), create)(
                m, n, nnz(u_A), u_A.origin.offset, 0 if suf == "f64" else 1, _ptr(first),
                _ptr(second), _ptr(nonzeros(u_A)), _stream(self.dev), ctypes.byref(self._plan))
        _lib.check(st, create[10:], u_A.format, _BE, self.T)
        # The values the plan reads and torch's in-place version of them when
        # it last read them.  Sliced and binned layouts (and COO plans, whose
        # entries may have been reordered) run on a permuted copy of the
        # values, so an in-place write into them has to be gathered again;
        # merge and vector plans read the buffer itself.
        self._vals = nonzeros(u_A)
        self._ver = self._vals._version
        self._copies = coo or self.kernel() in ("sliced", "binned")
        self._exec_values = None

    takes_raw = True     # execute(h, x, y) on plain device tensors: the raw-array form

    def execute(self, *ts, alpha=1.0, beta=0.0):
        """execute(h, x, y) (the cuSPARSE handle form) or execute(h, A, x, y)
        (EmitterSpMVHandle, spmv.jl:531-544, which reads A's buffers at each
        call).  Both see A's values as they are at the call: values written
        in place through torch since the plan last read them (torch's version
        counter of the value tensor moved) are gathered again into the
        plan's copy, in stream order, before the product; an A whose value
        tensor is another one than the plan's becomes the plan's values
        (update_values! semantics).  Writes that bypass torch (raw device
        pointers) need update_values_.  The handle's input_fn/output_fn
        apply.  With plain device tensors x, y the call returns y, as the
        cuSPARSE handle's raw-array method does (ext/CUDAExt/ops/spmv.jl:
        63-78); with USTensors it returns u_y."""
        if len(ts) == 2 and isinstance(ts[0], torch.Tensor) and isinstance(ts[1], torch.Tensor):
            return self.execute_tensors(ts[0], ts[1], alpha, beta)
        ts = tuple(t if isinstance(t, USTensor) else ust(t) for t in ts)
        if len(ts) == 3:
            u_A, u_x, u_y = ts
            if nonzeros(u_A) is not self._vals:
                self._rebind(u_A)
        elif len(ts) == 2:
            u_x, u_y = ts
        else:
            raise TypeError("execute(handle, [A,] x, y)")
        return spmv_with_fns(self._execute_plain, self.u_A, u_x, u_y, alpha, beta,
                             self.input_fn, self.output_fn)

    def _rebind(self, u_A: USTensor):
        """Take u_A's value tensor as the plan's values; the next product
        reads them (a stale version forces the stream-ordered gather)."""
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A):
            raise IncompatibleExtents("execute(h, A, x, y): A's sparsity structure is not the plan's")
        _check_values(u_A, self.T)
        _check_same_device(nonzeros(u_A), self._vals)
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, nonzeros(u_A), self.u_A.owner, self.u_A.origin)
        self._vals = nonzeros(u_A)
        self._ver = -1        # never a tensor's version: the next product reads the values

    def _stale(self) -> bool:
        """Whether the plan must read its value tensor again before a product:
        a new tensor (_rebind), or one whose torch version moved (written in
        place: a copying plan gathers it again; for a plan that reads the
        tensor in place only its address is taken again, in case its storage
        was replaced)."""
        return self._ver < 0 or self._vals._version != self._ver

    def _launch(self, alpha, x_ptr, beta, y_ptr, stream):
        """One plan execute on raw pointers; through execute_values when the
        plan's values are stale (refresh on the same stream, then product)."""
        if self._stale():
            if self._exec_values is None:
                self._exec_values = getattr(_lib.lib(),
                                            f"jlust_hip_csr_spmv_plan_execute_values_{self.suf}")
            v = self._vals
            st = self._exec_values(self._plan, v.data_ptr() if v.numel() else None, alpha, x_ptr,
                                   beta, y_ptr, stream)
            if st == 0:
                self._ver = v._version
            return st
        if self._exec is None:
            self._exec = getattr(_lib.lib(), f"jlust_hip_csr_spmv_plan_execute_{self.suf}")
        return self._exec(self._plan, alpha, x_ptr, beta, y_ptr, stream)

    def _execute_plain(self, u_A, u_x: USTensor, u_y: USTensor, alpha=1.0, beta=0.0):
        x, y = _vec_checks(self.u_A, u_x, u_y)
        _check_same_device(nonzeros(self.u_A), x, y)
        with _on(self.dev):
            st = self._launch(float(alpha), _ptr(x), float(beta), _ptr(y), _stream(self.dev))
        _lib.check(st, "csr_spmv_plan_execute", self.u_A.format, _BE, self.T)
        return u_y

    def execute_tensors(self, x: torch.Tensor, y: torch.Tensor, alpha=1.0, beta=0.0):
        """execute on plain device vectors with the checks reduced to
        attribute compares (the raw-array hot path: a product here is a few
        microseconds of GPU time).  Anything else -- another dtype or device,
        a wrong length, strided vectors, input_fn/output_fn -- takes the
        checked USTensor path, which raises where that path raises."""
        m, n = self.u_A.extents
        di = self.dev.index
        if (x.dtype is not self.T or y.dtype is not self.T or x.get_device() != di or
                y.get_device() != di or x.numel() != n or y.numel() != m or
                not x.is_contiguous() or not y.is_contiguous() or
                self.input_fn is not None or self.output_fn is not None):
            self.execute(ust(x), ust(y), alpha=alpha, beta=beta)
            return y
        with _on(self.dev):
            st = self._launch(alpha, x.data_ptr(), beta, y.data_ptr(), _stream(self.dev))
        if st:
            _lib.check(st, "csr_spmv_plan_execute", self.u_A.format, _BE, self.T)
        return y

    def capture(self, x: torch.Tensor, y: torch.Tensor, alpha=1.0, beta=0.0) -> "SpMVGraph":
        """Record execute(h, x, y, alpha, beta) once as a HIP graph
        (jlust_hip_csr_spmv_plan_capture_*; the reference's CUDA.capture of
        its SpMV, ext/CUDAExt/ops/block_mul.jl:258-263).  Nothing runs until
        the graph is launched; x and y are plain contiguous vectors of the
        plan's type on its device, and the handle has no input_fn/output_fn."""
        m, n = self.u_A.extents
        di = self.dev.index
        if (x.dtype is not self.T or y.dtype is not self.T or x.get_device() != di or
                y.get_device() != di):
            raise UnsupportedValueType(x.dtype, _BE, f"capture takes {self.T} vectors on {self.dev}")
        if x.numel() != n or y.numel() != m or not x.is_contiguous() or not y.is_contiguous():
            raise IncompatibleExtents(f"capture: A is {m}x{n}, x has {tuple(x.shape)}, "
                                      f"y has {tuple(y.shape)} (contiguous vectors)")
        if self.input_fn is not None or self.output_fn is not None:
            raise UnsupportedFormat(self.u_A.format, _BE, "capture takes handles without input_fn/output_fn")
        return SpMVGraph(self, x.data_ptr(), y.data_ptr(), alpha, beta)

    def _capture_raw(self, x_ptr: int, y_ptr: int, alpha, beta) -> ctypes.c_void_p:
        if self._stale():
            self.update_values(self.u_A)
        g = ctypes.c_void_p()
        with _on(self.dev):
            st = getattr(_lib.lib(), f"jlust_hip_csr_spmv_plan_capture_{self.suf}")(
                self._plan, alpha, x_ptr, beta, y_ptr, ctypes.byref(g))
        _lib.check(st, "csr_spmv_plan_capture", self.u_A.format, _BE, self.T)
        return g

    def _info(self):
        k, lpr, nb = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
        st = _lib.lib().jlust_hip_csr_spmv_plan_info(self._plan, ctypes.byref(k), ctypes.byref(lpr),
                                                     ctypes.byref(nb))
        _lib.check(st, "csr_spmv_plan_info", self.u_A.format, _BE, self.T)
        return k.value, lpr.value, nb.value

    def kernel(self) -> str:
        """The kernel the plan runs: "merge", "vector", "sliced" or "binned"."""
        return ("merge", "vector", "sliced", "binned")[self._info()[0]]

    def device_bytes(self) -> int:
        """Device memory the plan holds until it is destroyed."""
        return self._info()[2]

    def update_values(self, u_A: USTensor):
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A):
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        _check_values(u_A, self.T)
        v = nonzeros(u_A)
        ver = v._version
        with _on(self.dev):
            st = _lib.lib().jlust_hip_csr_spmv_plan_update_values(self._plan, _ptr(v), _stream(self.dev))
        _lib.check(st, "csr_spmv_plan_update_values", u_A.format, _BE, self.T)
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, v, self.u_A.owner, self.u_A.origin)
        self._vals, self._ver = v, ver
        return self

    def __del__(self):
        plan, self._plan = getattr(self, "_plan", None), None
        if plan is not None and plan.value:
            try:
                _lib.lib().jlust_hip_csr_spmv_plan_destroy(plan)
            except Exception:
                pass


class SpMVGraph:
    """A captured plan execution (HIPSpMVHandle.capture).  launch() replays
    it on the current stream of the plan's device and returns True, or
    returns False without launching when that stream is itself being
    captured (the caller then executes the plan, so the outer capture records
    the kernels).  Like the reference's graphs (keyed by pointer(y),
    pointer(x)) it replays on the device addresses of x and y given at
    capture, which the caller keeps valid.  It holds its handle and the value
    tensor the captured kernels read, so neither is freed under it.  A launch sees
    the handle's values as they are then: a merge or vector plan whose value
    tensor was replaced (update_values_ or execute(h, A, ...) with another
    tensor) is captured again, and values a copying plan holds that were
    written in place through torch are gathered again first."""

    __slots__ = ("_g", "_h", "dev", "_launch", "_x", "_y", "_alpha", "_beta", "_vals")

    def __init__(self, h: "HIPSpMVHandle", x: int, y: int, alpha, beta):
        self._h, self.dev = h, h.dev
        self._x, self._y, self._alpha, self._beta = x, y, alpha, beta
        self._g = None
        self._launch = _lib.lib().jlust_hip_spmv_graph_launch
        self._g = h._capture_raw(x, y, alpha, beta)
        self._vals = h._vals

    def launch(self) -> bool:
        h = self._h
        if h._vals is not self._vals and not h._copies:
            # The graph's kernels hold the old value pointer: capture again.
            g = h._capture_raw(self._x, self._y, self._alpha, self._beta)
            self._destroy()
            self._g, self._vals = g, h._vals
        elif h._stale():
            h.update_values(h.u_A)
            self._vals = h._vals
        with _on(self.dev):
            st = self._launch(self._g, _stream(self.dev))
        if st == 0:
            return True
        if st == _lib.STREAM_CAPTURING:
            return False
        _lib.check(st, "spmv_graph_launch", h.u_A.format, _BE, h.T)
        return False

    def _destroy(self):
        g, self._g = getattr(self, "_g", None), None
        if g is not None and g.value:
            try:
                _lib.lib().jlust_hip_spmv_graph_destroy(g)
            except Exception:
                pass

    def __del__(self):
        self._destroy()


class HIPOpHandle(AbstractKernelHandle):
    """Prepared SpMV / SpMM of the formats without a plan of their own (DCSR,
    ShiftedDiag, PeriodicCSR, BSR): holds A and dispatches to the plain entry
    points, the contract of the cuSPARSE handles (ext/CUDAExt/ops/
    spmm.jl:8-70)."""

    def __init__(self, optype, u_A: USTensor, **kw):
        self.optype, self.u_A, self.kw = optype, u_A, kw
        _value_suffix(u_A)

    def execute(self, *ts, **kw):
        """execute(h, x, y) / execute(h, A, x, y): A given at the call wins,
        as EmitterSpMVHandle takes it per call; keywords given at prepare
        apply."""
        from .ops import execute as _execute
        kw = {**self.kw, **kw}
        if len(ts) == 3:
            return _execute(self.optype, *ts, backend=_BE, **kw)
        return _execute(self.optype, self.u_A, *ts, backend=_BE, **kw)

    def update_values(self, u_A: USTensor):
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A):
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, nonzeros(u_A), self.u_A.owner, self.u_A.origin)
        return self


class HIPSpMMHandle(AbstractKernelHandle):
    """Prepared CSR, COO or CSC SpMM (jlust_hip_csr_spmm_plan_*,
    jlust_hip_coo_spmm_plan_create): prepare(HIPBackend(), SpMMOp, A;
    n_cols=k) -> execute(h, B, C) -> update_values!(h, A), the cuSPARSE SpMM
    handle contract (ext/CUDAExt/ops/spmm.jl:8-70).  The plan analyses A once
    (COO/CSC entries put in row order; column chunk per pass for k, long rows
    split into segments) and owns the workspace.  A CSR plan, and a COO plan
    whose rows were already in order, read A's values in place; a reordered
    COO/CSC plan holds them in its row order, and values written into A's
    tensor through torch since the plan last read them (its version counter
    moved) are gathered again, in stream order, before the product.
    update_values_ or execute(h, A, B, C) with another value tensor points the
    plan at it.  B with another number of columns than the plan's rebuilds
    the plan.  skip_empty_rows applies to CSR (COO and CSC scale every row of
    C by beta, as the reference's pre-scale does)."""

    def __init__(self, u_A: USTensor, n_cols=None, skip_empty_rows=False):
        self.coo, self.csc = is_coo_shaped(u_A.format), is_csc_shaped(u_A.format)
        if not (is_csr_shaped(u_A.format) or self.coo or self.csc):
            raise UnsupportedFormat(u_A.format, _BE, "prepared SpMM plans take CSR, COO or CSC")
        self.suf = _value_suffix(u_A)
        self.T = nonzeros(u_A).dtype
        idx1, idx2 = self._index(u_A)
        _check_values(u_A, self.T)
        self.dev = _check_same_device(idx1, idx2, nonzeros(u_A))
        self.u_A = u_A
        self.skip_empty_rows = bool(skip_empty_rows) and not (self.coo or self.csc)
        self._plan = ctypes.c_void_p(0)
        self.k = None
        self._copies = False
        self._ver = nonzeros(u_A)._version
        if n_cols is not None:
            self._make(int(n_cols))

    def _index(self, u=None):
        u = self.u_A if u is None else u
        return _coo_parts(u) if self.coo else _csc_parts(u) if self.csc else _csr_parts(u)

    def _make(self, k: int):
        self._destroy()
        m, n = self.u_A.extents
        idx1, idx2 = self._index()
        vals = nonzeros(self.u_A)
        vt = 0 if self.suf == "f64" else 1
        plan = ctypes.c_void_p(0)
        with _on(self.dev):
            if self.coo or self.csc:
                st = _lib.lib().jlust_hip_coo_spmm_plan_create(
                    2 if self.coo else 1, m, n, k, nnz(self.u_A), self.u_A.origin.offset, vt, _ptr(idx1),
                    _ptr(idx2), _ptr(vals), _stream(self.dev), ctypes.byref(plan))
            else:
                st = _lib.lib().jlust_hip_csr_spmm_plan_create(
                    m, n, k, nnz(self.u_A), self.u_A.origin.offset, vt, _ptr(idx1), _ptr(idx2),
                    _ptr(vals), _stream(self.dev), ctypes.byref(plan))
        _lib.check(st, "spmm_plan_create", self.u_A.format, _BE, self.T)
        self._plan, self.k = plan, k
        self._ver = vals._version
        # A reordered COO/CSC plan holds its own copy of the values.
        self._copies = self.info()["reordered"]

    def execute(self, *ts, alpha=1.0, beta=0.0, skip_empty_rows=None):
        """execute(h, B, C) or execute(h, A, B, C); returns C (a USTensor)."""
        ts = tuple(t if isinstance(t, USTensor) else ust(t) for t in ts)
        if len(ts) == 3:
            u_A, u_B, u_C = ts
            if nonzeros(u_A) is not nonzeros(self.u_A):
                self.update_values(u_A)
        elif len(ts) == 2:
            u_B, u_C = ts
        else:
            raise TypeError("execute(handle, [A,] B, C)")
        B, C = nonzeros(u_B), nonzeros(u_C)
        m, n = self.u_A.extents
        if B.dtype != self.T or C.dtype != self.T:
            raise UnsupportedValueType(B.dtype if B.dtype != self.T else C.dtype, _BE)
        if B.dim() != 2 or C.dim() != 2 or B.shape[0] != n or C.shape[0] != m or \
                B.shape[1] != C.shape[1]:
            raise IncompatibleExtents(
                f"SpMM: A is {m}x{n}, B is {tuple(B.shape)}, C is {tuple(C.shape)}")
        for t, nm in ((B, "B"), (C, "C")):
            if t.shape[0] > 1 and t.shape[1] > 0 and t.stride(0) != 1:
                raise NonCanonicalStorage(f"SpMM: {nm} must be column-major (stride(0) == 1)")
        _check_same_device(nonzeros(self.u_A), B, C)
        k = B.shape[1]
        if self.k != k:
            self._make(k)
        elif self._copies and nonzeros(self.u_A)._version != self._ver:
            self._refresh()
        skip = self.skip_empty_rows if skip_empty_rows is None else bool(skip_empty_rows)
        if self.coo or self.csc:
            skip = False
        with _on(self.dev):
            st = getattr(_lib.lib(), f"jlust_hip_csr_spmm_plan_execute_{self.suf}")(
                self._plan, float(alpha), _ptr(B), leading_dim(B), float(beta), _ptr(C),
                leading_dim(C), int(skip), _stream(self.dev))
        _lib.check(st, "csr_spmm_plan_execute", self.u_A.format, _BE, self.T)
        return u_C

    def _refresh(self):
        """Make the plan read self.u_A's values now (stream-ordered: a pointer
        swap, or a gather into a reordered plan's copy)."""
        v = nonzeros(self.u_A)
        if self._plan.value:
            with _on(self.dev):
                st = _lib.lib().jlust_hip_csr_spmm_plan_update_values(self._plan, _ptr(v), _stream(self.dev))
            _lib.check(st, "csr_spmm_plan_update_values", self.u_A.format, _BE, self.T)
        self._ver = v._version

    def update_values(self, u_A: USTensor):
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A):
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        _check_values(u_A, self.T)
        _check_same_device(nonzeros(u_A), nonzeros(self.u_A))
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, nonzeros(u_A), self.u_A.owner, self.u_A.origin)
        self._refresh()
        return self

    def info(self) -> dict:
        """What the plan's analysis found: split rows, their segments, columns
        per pass, and whether COO/CSC entries were reordered."""
        if not self._plan.value:
            return {}
        a, b, c, r = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        st = _lib.lib().jlust_hip_csr_spmm_plan_info(self._plan, ctypes.byref(a), ctypes.byref(b),
                                                     ctypes.byref(c), ctypes.byref(r))
        _lib.check(st, "csr_spmm_plan_info", self.u_A.format, _BE, self.T)
        return {"split_rows": a.value, "segments": b.value, "cols_per_pass": c.value,
                "reordered": bool(r.value)}

    def _destroy(self):
        plan, self._plan = getattr(self, "_plan", None), ctypes.c_void_p(0)
        if plan is not None and plan.value:
            try:
                _lib.lib().jlust_hip_csr_spmm_plan_destroy(plan)
            except Exception:
                pass

    def __del__(self):
        self._destroy()


class HIPBSRSpMMHandle(AbstractKernelHandle):
    """Prepared BSR SpMM (jlust_hip_bsr_spmm_plan_*): prepare(HIPBackend(),
    SpMMOp, A::BSR; n_cols=k) -> execute(h, B, C) -> update_values!(h, A), the
    cuSPARSE SpMM handle contract (ext/CUDAExt/ops/spmm.jl:8-70) for BSR.
    16 x 16 blocks run the MFMA kernels (fp32 or fp64) on A's buffers; any
    other block shape is expanded to CSR once and runs through a CSR SpMM
    plan over the expansion.  A's values are read as they are at the
    call: on the expansion path, values written in place through torch since
    the plan last read them (the value tensor's version counter moved) are
    expanded again, in stream order, before the product.  B with another
    number of columns than the plan's rebuilds the plan."""

    def __init__(self, u_A: USTensor, n_cols=None):
        if not is_bsr(u_A.format):
            raise UnsupportedFormat(u_A.format, _BE, "prepared BSR SpMM plans take BSR")
        self.suf = _value_suffix(u_A)
        self.T = nonzeros(u_A).dtype
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u_A)
        _check_values(u_A, self.T)
        self.dev = _check_same_device(browptr, bcolind, nonzeros(u_A))
        self.u_A = u_A
        self._plan = ctypes.c_void_p(0)
        self.k = None
        self._vals = nonzeros(u_A)
        self._ver = self._vals._version
        if n_cols is not None:
            self._make(int(n_cols))

    def _make(self, k: int):
        self._destroy()
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(self.u_A)
        plan = ctypes.c_void_p(0)
        with _on(self.dev):
            st = _lib.lib().jlust_hip_bsr_spmm_plan_create(
                mb, nb, b1, b2, bcolind.numel(), self.u_A.origin.offset, 0 if self.suf == "f64" else 1,
                int(row_major), _ptr(browptr), _ptr(bcolind), _ptr(self._vals), k, _stream(self.dev),
                ctypes.byref(plan))
        _lib.check(st, "bsr_spmm_plan_create", self.u_A.format, _BE, self.T)
        self._plan, self.k = plan, k
        self._ver = self._vals._version

    def execute(self, *ts, alpha=1.0, beta=0.0):
        """execute(h, B, C) or execute(h, A, B, C); returns C (a USTensor)."""
        ts = tuple(t if isinstance(t, USTensor) else ust(t) for t in ts)
        if len(ts) == 3:
            u_A, u_B, u_C = ts
            if nonzeros(u_A) is not self._vals:
                self.update_values(u_A)
        elif len(ts) == 2:
            u_B, u_C = ts
        else:
            raise TypeError("execute(handle, [A,] B, C)")
        B, C = nonzeros(u_B), nonzeros(u_C)
        m, n = self.u_A.extents
        if B.dtype != self.T or C.dtype != self.T:
            raise UnsupportedValueType(B.dtype if B.dtype != self.T else C.dtype, _BE)
        if B.dim() != 2 or C.dim() != 2 or B.shape[0] != n or C.shape[0] != m or \
                B.shape[1] != C.shape[1]:
            raise IncompatibleExtents(
                f"SpMM: A is {m}x{n}, B is {tuple(B.shape)}, C is {tuple(C.shape)}")
        for t, nm in ((B, "B"), (C, "C")):
            if t.shape[0] > 1 and t.shape[1] > 0 and t.stride(0) != 1:
                raise NonCanonicalStorage(f"SpMM: {nm} must be column-major (stride(0) == 1)")
        _check_same_device(self._vals, B, C)
        k = B.shape[1]
        if self.k != k:
            self._make(k)
        elif self._vals._version != self._ver:
            self._refresh()
        with _on(self.dev):
            st = getattr(_lib.lib(), f"jlust_hip_bsr_spmm_plan_execute_{self.suf}")(
                self._plan, float(alpha), _ptr(B), leading_dim(B), float(beta), _ptr(C),
                leading_dim(C), _stream(self.dev))
        _lib.check(st, "bsr_spmm_plan_execute", self.u_A.format, _BE, self.T)
        return u_C

    def _refresh(self):
        """Point the plan at self._vals and re-read them (stream-ordered)."""
        if self._plan.value:
            with _on(self.dev):
                st = _lib.lib().jlust_hip_bsr_spmm_plan_update_values(self._plan, _ptr(self._vals),
                                                                      _stream(self.dev))
            _lib.check(st, "bsr_spmm_plan_update_values", self.u_A.format, _BE, self.T)
        self._ver = self._vals._version

    def update_values(self, u_A: USTensor):
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A) or u_A.format != self.u_A.format:
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        _check_values(u_A, self.T)
        _check_same_device(nonzeros(u_A), self._vals)
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, nonzeros(u_A), self.u_A.owner, self.u_A.origin)
        self._vals = nonzeros(u_A)
        self._refresh()
        return self

    def info(self) -> dict:
        """The path the plan chose: "mfma" or "csr_expansion"."""
        if not self._plan.value:
            return {}
        path = ctypes.c_int32()
        st = _lib.lib().jlust_hip_bsr_spmm_plan_info(self._plan, ctypes.byref(path))
        _lib.check(st, "bsr_spmm_plan_info", self.u_A.format, _BE, self.T)
        return {"path": "mfma" if path.value == 0 else "csr_expansion"}

    def _destroy(self):
        plan, self._plan = getattr(self, "_plan", None), ctypes.c_void_p(0)
        if plan is not None and plan.value:
            try:
                _lib.lib().jlust_hip_bsr_spmm_plan_destroy(plan)
            except Exception:
                pass

    def __del__(self):
        self._destroy()


class HIPBSRSpMVHandle(AbstractKernelHandle):
    """Prepared BSR SpMV (jlust_hip_bsr_spmv_plan_*): prepare(HIPBackend(),
    SpMVOp, A::BSR) -> execute(h, x, y) or execute(h, A, x, y) ->
    update_values!(h, A), the EmitterSpMVHandle contract (ext/
    KernelAbstractionsExt/ops/spmv.jl:518-544) with the block-rows' segment
    table built once instead of at every call.  The plan reads A's values in
    place, so a product sees them as they are at the call; an A with another
    value tensor becomes the plan's values (update_values! semantics).  Index
    buffers written in place through torch since the plan was built are
    checked and the table rebuilt.  input_fn/output_fn apply as in plain
    execute."""

    takes_raw = True

    def __init__(self, u_A: USTensor, input_fn=None, output_fn=None):
        if not is_bsr(u_A.format):
            raise UnsupportedFormat(u_A.format, _BE, "prepared BSR SpMV plans take BSR")
        self.input_fn, self.output_fn = input_fn, output_fn
        self.suf = _value_suffix(u_A)
        self.T = nonzeros(u_A).dtype
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(u_A)
        _check_values(u_A, self.T)
        self.dev = _check_same_device(browptr, bcolind, nonzeros(u_A))
        self.u_A = u_A                      # keeps the buffers alive (GC anchor)
        self._vals = nonzeros(u_A)
        self._plan = ctypes.c_void_p(0)
        self._make()

    def _make(self):
        self._destroy()
        b1, b2, row_major, browptr, bcolind, mb, nb = _bsr_parts(self.u_A)
        _check_pos_once(self.u_A, browptr, mb, bcolind.numel(), self.dev)
        _check_crd_once(self.u_A, bcolind, nb, False, self.dev)
        plan = ctypes.c_void_p(0)
        with _on(self.dev):
            st = _lib.lib().jlust_hip_bsr_spmv_plan_create(
                mb, nb, b1, b2, bcolind.numel(), self.u_A.origin.offset, 0 if self.suf == "f64" else 1,
                int(row_major), _ptr(browptr), _ptr(bcolind), _ptr(self._vals), _stream(self.dev),
                ctypes.byref(plan))
        _lib.check(st, "bsr_spmv_plan_create", self.u_A.format, _BE, self.T)
        self._plan = plan
        self._iver = (browptr._version, bcolind._version)

    def _current(self):
        """Rebuild the table if A's index buffers were written in place."""
        browptr, bcolind = self.u_A.pos_buffers[1], self.u_A.crd_buffers[1]
        if (browptr._version, bcolind._version) != self._iver:
            self._make()

    def execute(self, *ts, alpha=1.0, beta=0.0):
        """execute(h, x, y) or execute(h, A, x, y); with plain device tensors
        x, y the call returns y, with USTensors u_y."""
        if len(ts) == 2 and isinstance(ts[0], torch.Tensor) and isinstance(ts[1], torch.Tensor):
            self.execute(ust(ts[0]), ust(ts[1]), alpha=alpha, beta=beta)
            return ts[1]
        ts = tuple(t if isinstance(t, USTensor) else ust(t) for t in ts)
        if len(ts) == 3:
            u_A, u_x, u_y = ts
            if nonzeros(u_A) is not self._vals:
                self.update_values(u_A)
        elif len(ts) == 2:
            u_x, u_y = ts
        else:
            raise TypeError("execute(handle, [A,] x, y)")
        self._current()
        return spmv_with_fns(self._execute_plain, self.u_A, u_x, u_y, alpha, beta,
                             self.input_fn, self.output_fn)

    def _execute_plain(self, u_A, u_x: USTensor, u_y: USTensor, alpha=1.0, beta=0.0):
        x, y = _vec_checks(self.u_A, u_x, u_y)
        _check_same_device(self._vals, x, y)
        with _on(self.dev):
            st = getattr(_lib.lib(), f"jlust_hip_bsr_spmv_plan_execute_{self.suf}")(
                self._plan, float(alpha), _ptr(x), float(beta), _ptr(y), _stream(self.dev))
        _lib.check(st, "bsr_spmv_plan_execute", self.u_A.format, _BE, self.T)
        return u_y

    def update_values(self, u_A: USTensor):
        if u_A.extents != self.u_A.extents or nnz(u_A) != nnz(self.u_A) or u_A.format != self.u_A.format:
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        _check_values(u_A, self.T)
        _check_same_device(nonzeros(u_A), self._vals)
        self.u_A = USTensor(self.u_A.extents, self.u_A.format, self.u_A.pos_buffers,
                            self.u_A.crd_buffers, nonzeros(u_A), self.u_A.owner, self.u_A.origin)
        self._vals = nonzeros(u_A)
        with _on(self.dev):
            st = _lib.lib().jlust_hip_bsr_spmv_plan_update_values(self._plan, _ptr(self._vals),
                                                                  _stream(self.dev))
        _lib.check(st, "bsr_spmv_plan_update_values", self.u_A.format, _BE, self.T)
        return self

    def kernel(self) -> str:
        return "bsr_segments"

    def _destroy(self):
        plan, self._plan = getattr(self, "_plan", None), ctypes.c_void_p(0)
        if plan is not None and plan.value:
            try:
                _lib.lib().jlust_hip_bsr_spmv_plan_destroy(plan)
            except Exception:
                pass

    def __del__(self):
        self._destroy()


class HIPSDDMMHandle(AbstractKernelHandle):
    """Prepared SDDMM (jlust_hip_sddmm_plan_*): prepare(HIPBackend(), SDDMMOp,
    A, B, C) -> execute(h, A, B, C) -> update_values!(h, C), the cuSPARSE
    SDDMM handle contract (ext/CUDAExt/ops/sddmm.jl:10-76); prepare(...,
    SDDMMOp, C) also works, the inner dimension taken from the first A.  C
    (CSR, COO, CSC or DCSR) is the mask pattern; the plan holds its row order
    and work items.  execute(h, A, B) writes into the handle's C;
    update_values_(h, C2) makes C2 (same pattern) the handle's output."""

    # Mask formats of jlust_hip_sddmm_plan_create (enum jlust_format).
    _FMT = {"CSR": 0, "CSC": 1, "COO": 2}

    def __init__(self, u_C: USTensor, n_inner=None):
        f = u_C.format
        self.kind = ("COO" if is_coo_shaped(f) else "CSC" if is_csc_shaped(f) else
                     "CSR" if is_csr_shaped(f) else "DCSR" if f == Formats.DCSR else None)
        if self.kind is None:
            raise UnsupportedFormat(u_C.format, _BE, "prepared SDDMM plans take a CSR, COO, CSC or DCSR mask")
        self.suf = _value_suffix(u_C)
        self.T = nonzeros(u_C).dtype
        idx = self._index(u_C)
        self.dev = _check_same_device(*idx, nonzeros(u_C))
        if self.kind == "DCSR":
            _check_crd_once(u_C, idx[0], u_C.extents[0], True, self.dev)
        self.u_C = u_C
        self._plan = ctypes.c_void_p(0)
        self.K = None
        if n_inner is not None:
            self._make(int(n_inner))

    def _index(self, u):
        return {"COO": _coo_parts, "CSC": _csc_parts, "CSR": _csr_parts, "DCSR": _dcsr_parts}[self.kind](u)

    def _make(self, K: int):
        self._destroy()
        m, n = self.u_C.extents
        idx = self._index(self.u_C)
        vt = 0 if self.suf == "f64" else 1
        plan = ctypes.c_void_p(0)
        with _on(self.dev):
            if self.kind == "DCSR":
                rows, pos, cols = idx
                st = _lib.lib().jlust_hip_dcsr_sddmm_plan_create(
                    m, n, K, rows.numel(), nnz(self.u_C), self.u_C.origin.offset, vt, _ptr(rows), _ptr(pos),
                    _ptr(cols), _stream(self.dev), ctypes.byref(plan))
            else:
                st = _lib.lib().jlust_hip_sddmm_plan_create(
                    self._FMT[self.kind], m, n, K, nnz(self.u_C), self.u_C.origin.offset, vt, _ptr(idx[0]),
                    _ptr(idx[1]), _stream(self.dev), ctypes.byref(plan))
        _lib.check(st, "sddmm_plan_create", self.u_C.format, _BE, self.T)
        self._plan, self.K = plan, K

    def execute(self, *ts, alpha=1.0, beta=0.0, mask=None):
        """execute(h, A, B, C) or execute(h, A, B) (into the handle's C);
        returns C."""
        ts = tuple(t if isinstance(t, USTensor) else ust(t) for t in ts)
        if len(ts) == 3:
            u_A, u_B, u_C = ts
            if nonzeros(u_C) is not nonzeros(self.u_C):
                self.update_values(u_C)
        elif len(ts) == 2:
            u_A, u_B = ts
        else:
            raise TypeError("execute(handle, A, B[, C])")
        u_C = self.u_C
        A, B = _sddmm_dense_checks(u_A, u_B, u_C)
        mk = _sddmm_mask(mask, u_C, self.T)
        _check_same_device(nonzeros(u_C), A, B, mk)
        if self.K != A.shape[1]:
            self._make(A.shape[1])
        with _on(self.dev):
            st = getattr(_lib.lib(), f"jlust_hip_sddmm_plan_execute_{self.suf}")(
                self._plan, float(alpha), _ptr(A), leading_dim(A), _ptr(B), leading_dim(B),
                float(beta), _ptr(nonzeros(u_C)), _ptr(mk), _stream(self.dev))
        _lib.check(st, "sddmm_plan_execute", u_C.format, _BE, self.T)
        return u_C

    def update_values(self, u_C: USTensor):
        if u_C.extents != self.u_C.extents or nnz(u_C) != nnz(self.u_C):
            raise IncompatibleExtents("update_values!: the sparsity structure must not change")
        _check_values(u_C, self.T)
        _check_same_device(nonzeros(u_C), nonzeros(self.u_C))
        self.u_C = USTensor(self.u_C.extents, self.u_C.format, self.u_C.pos_buffers,
                            self.u_C.crd_buffers, nonzeros(u_C), self.u_C.owner, self.u_C.origin)
        return self

    def info(self) -> dict:
        """Work items of the plan and whether a COO mask was reordered."""
        if not self._plan.value:
            return {}
        a, b = ctypes.c_int64(), ctypes.c_int32()
        st = _lib.lib().jlust_hip_sddmm_plan_info(self._plan, ctypes.byref(a), ctypes.byref(b))
        _lib.check(st, "sddmm_plan_info", self.u_C.format, _BE, self.T)
        return {"work_items": a.value, "reordered": bool(b.value)}

    def _destroy(self):
        plan, self._plan = getattr(self, "_plan", None), ctypes.c_void_p(0)
        if plan is not None and plan.value:
            try:
                _lib.lib().jlust_hip_sddmm_plan_destroy(plan)
            except Exception:
                pass

    def __del__(self):
        self._destroy()


def prepare(optype, u_A: USTensor, *more, **kw):
    """prepare(HIPBackend(), OpType, A; kw...) (src/ops.jl:163-177).  SpMV:
    input_fn/output_fn; SpMM: n_cols, skip_empty_rows; SDDMM: (A, B, C) as
    the cuSPARSE handle takes them, or the mask C alone (n_inner = K).  A
    sparse operand with Int64 index buffers is prepared over their Int32
    narrowing as it is at this call."""
    u_A = _narrowed(u_A)
    more = tuple(_narrowed(t) for t in more)
    tag = getattr(optype, "tag", None)
    if tag == "SpMV":
        bad = set(kw) - {"input_fn", "output_fn"}
        if bad or more:
            raise TypeError(f"prepare(SpMVOp): unexpected keywords {sorted(bad)} or tensors ({len(more)})")
        if is_csr_shaped(u_A.format) or is_coo_shaped(u_A.format):
            return HIPSpMVHandle(u_A, kw.get("input_fn"), kw.get("output_fn"))
        if is_bsr(u_A.format):
            return HIPBSRSpMVHandle(u_A, kw.get("input_fn"), kw.get("output_fn"))
        return HIPOpHandle(SpMVOp, u_A, **kw)
    if tag == "SpMM":
        bad = set(kw) - {"n_cols", "skip_empty_rows"}
        if bad or more:
            raise TypeError(f"prepare(SpMMOp): unexpected keywords {sorted(bad)} or tensors ({len(more)})")
        if is_csr_shaped(u_A.format) or is_coo_shaped(u_A.format) or is_csc_shaped(u_A.format):
            return HIPSpMMHandle(u_A, kw.get("n_cols"), kw.get("skip_empty_rows", False))
        if is_bsr(u_A.format) and not kw.get("skip_empty_rows"):
            return HIPBSRSpMMHandle(u_A, kw.get("n_cols"))
        kw.pop("n_cols", None)
        return HIPOpHandle(SpMMOp, u_A, **kw)
    if tag == "SDDMM":
        bad = set(kw) - {"n_inner"}
        if bad:
            raise TypeError(f"prepare(SDDMMOp): unexpected keywords {sorted(bad)}")
        if len(more) == 2:                     # (A, B, C)
            A = nonzeros(u_A)
            return HIPSDDMMHandle(more[1], A.shape[1] if A.dim() == 2 else None)
        if more:
            raise TypeError("prepare(SDDMMOp, A, B, C) or prepare(SDDMMOp, C)")
        return HIPSDDMMHandle(u_A, kw.get("n_inner"))
    raise UnsupportedFormat(u_A.format, _BE, f"prepare: {optype} is not supported")
