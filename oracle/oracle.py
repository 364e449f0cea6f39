"""ctypes front-end of the CPU oracle (oracle/jlust_cpu.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg, as the checker.  The product package
(``jlust_amd``) never imports this module.

Every function takes and returns numpy arrays.  Index arrays are int32 with the
tensor's origin (0 or 1) still applied, dense matrices are column-major
(Fortran order) like Julia arrays.  See the C file for the reference file:line
each routine restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# JLUST_ORACLE_LIB points the loader at another build of jlust_cpu.c, such as
# the AddressSanitizer one (`make -C oracle asan`; run with the sanitizer's
# runtime in LD_PRELOAD).
_LIBPATH = os.environ.get("JLUST_ORACLE_LIB") or os.path.join(_HERE, "libjlust_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_D = ctypes.c_double
_F = ctypes.c_float

SPMM_STRATEGIES = {0: "ColFirst", 1: "NNZFirst", 2: "Tiled", 3: "2D"}


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_LIBPATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE],
                       check=True, capture_output=True)
    return _LIBPATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIBPATH):
            build()
        L = ctypes.CDLL(_LIBPATH)
        for suf, S in (("f64", _D), ("f32", _F)):
            getattr(L, f"oracle_csr_spmv_{suf}").argtypes = [
                _I32, _I32, _P, _P, _P, S, _P, S, _P, _INT]
            getattr(L, f"oracle_csr_spmv_absref_{suf}").argtypes = [
                _I32, _I32, _P, _P, _P, _D, _P, _D, _P, _P, _INT]
            getattr(L, f"oracle_coo_spmv_{suf}").argtypes = [
                _I64, _I32, _I32, _P, _P, _P, S, _P, S, _P]
            getattr(L, f"oracle_csc_spmv_{suf}").argtypes = [
                _I32, _I32, _I32, _P, _P, _P, S, _P, S, _P]
            getattr(L, f"oracle_coo_spmm_{suf}").argtypes = [
                _I64, _I32, _I32, _P, _P, _P, _I64, S, _P, _I64, S, _P, _I64]
            getattr(L, f"oracle_csc_spmm_{suf}").argtypes = [
                _I32, _I32, _I32, _P, _P, _P, _I64, S, _P, _I64, S, _P, _I64]
            getattr(L, f"oracle_coo_sddmm_{suf}").argtypes = [
                _I64, _I32, _P, _P, _I64, S, _P, _I64, _P, _I64, S, _P, _P]
            f = getattr(L, f"oracle_csr_spmm_{suf}")
            f.argtypes = [_I32, _I32, _P, _P, _P, _I64, S, _P, _I64, S, _P,
                          _I64, _INT, _INT]
            f.restype = _INT
            getattr(L, f"oracle_csr_spmm_absref_{suf}").argtypes = [
                _I32, _I32, _P, _P, _P, _I64, _D, _P, _I64, _D, _P, _I64, _P,
                _INT]
            getattr(L, f"oracle_csr_sddmm_{suf}").argtypes = [
                _I32, _I32, _P, _P, _I64, S, _P, _I64, _P, _I64, S, _P, _P,
                _INT]
            getattr(L, f"oracle_csr_sddmm_absref_{suf}").argtypes = [
                _I32, _I32, _P, _P, _I64, _D, _P, _I64, _P, _I64, _D, _P, _P,
                _P, _INT]
            getattr(L, f"oracle_bsr_to_csr_{suf}").argtypes = [
                _I32, _I32, _I32, _I32, _P, _P, _P, _INT, _P, _P, _P]
            for name, args in (
                    ("csr_to_csc", [_I32, _I32, _I32, _P, _P, _P, _P, _P, _P]),
                    ("csr_to_coo", [_I32, _I32, _P, _P, _P, _P, _P, _P, _P]),
                    ("coo_to_csr", [_I64, _I32, _I32, _I32, _P, _P, _P, _P, _P,
                                    _P])):
                g = getattr(L, f"oracle_{name}_{suf}")
                g.argtypes = args
                g.restype = _I64
        L.oracle_spmm_strategy.argtypes = [_I64, _I64, _I64, _INT]
        L.oracle_spmm_strategy.restype = _INT
        L.oracle_max_threads.restype = _INT
        _lib = L
    return _lib


def _suf(dtype) -> str:
    dt = np.dtype(dtype)
    if dt == np.float64:
        return "f64"
    if dt == np.float32:
        return "f32"
    raise TypeError(f"oracle: unsupported value type {dt}")


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype=None):
    """Contiguous (C order for 1-D) copy-free view when possible."""
    return np.ascontiguousarray(a, dtype=dtype)


def _f(a, dtype=None):
    return np.asfortranarray(a, dtype=dtype)


def default_threads() -> int:
    return int(lib().oracle_max_threads())


def csr_spmv(rowptr, colind, val, x, alpha=1.0, beta=0.0, y0=None,
             origin=1, nthreads=None):
    """y = alpha*A*x (+beta*y0 iff beta != 0); returns a new array."""
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    x = _c(x, dt)
    m = rowptr.size - 1
    y = np.zeros(m, dt) if y0 is None else _c(y0, dt).copy()
    getattr(L, f"oracle_csr_spmv_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), _ptr(val), alpha, _ptr(x),
        beta, _ptr(y), nthreads or default_threads())
    return y


def csr_spmv_absref(rowptr, colind, val, x, alpha=1.0, beta=0.0, y0=None,
                    origin=1, nthreads=None):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    x = _c(x, dt)
    m = rowptr.size - 1
    out = np.empty(m, np.float64)
    y0c = None if y0 is None else _c(y0, dt)
    getattr(L, f"oracle_csr_spmv_absref_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), _ptr(val), float(alpha),
        _ptr(x), float(beta), _ptr(y0c), _ptr(out),
        nthreads or default_threads())
    return out


def dcsr_spmv(outer, inner_pos, inner_crd, val, x, m, alpha=1.0, beta=0.0, y0=None, origin=1):
    """DCSR SpMV as JLUST's walker runs it (n_outer = stored rows,
    ext/KernelAbstractionsExt/ops/spmv.jl:449-502): stored row f writes
    y[outer[f]] = alpha*sum + beta*y0[outer[f]]; rows that are not stored keep
    y0 (zeros when y0 is None)."""
    dt = np.asarray(val).dtype
    outer = np.asarray(outer, np.int64) - origin
    y = np.zeros(m, dt) if y0 is None else _c(y0, dt).copy()
    yc = csr_spmv(inner_pos, inner_crd, val, x, alpha, beta, y[outer], origin)
    y[outer] = yc
    return y


def dcsr_spmm(outer, inner_pos, inner_crd, val, B, m, alpha=1.0, beta=0.0, C0=None, origin=1):
    """DCSR SpMM: the stored rows' C rows as csr_spmm computes them, the other
    rows of C0 untouched."""
    dt = np.asarray(val).dtype
    outer = np.asarray(outer, np.int64) - origin
    B = _f(B, dt)
    C = np.zeros((m, B.shape[1]), dt, order="F") if C0 is None else _f(C0, dt).copy(order="F")
    Cc, _ = csr_spmm(inner_pos, inner_crd, val, B, alpha, beta, C[outer, :], origin)
    C[outer, :] = Cc
    return C


def coo_spmv(rows, cols, val, x, m, alpha=1.0, beta=0.0, y0=None, origin=1):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rows = _c(rows, np.int32)
    cols = _c(cols, np.int32)
    val = _c(val, dt)
    x = _c(x, dt)
    y = np.zeros(m, dt) if y0 is None else _c(y0, dt).copy()
    getattr(L, f"oracle_coo_spmv_{suf}")(
        val.size, m, origin, _ptr(rows), _ptr(cols), _ptr(val), alpha,
        _ptr(x), beta, _ptr(y))
    return y


def csc_spmv(colptr, rowind, val, x, m, alpha=1.0, beta=0.0, y0=None, origin=1):
    """Scatter-mode CSC SpMV: y = beta*y, then y[row] += (alpha*val)*x[col]
    column by column in storage order (oracle_csc_spmv_*)."""
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    colptr = _c(colptr, np.int32)
    rowind = _c(rowind, np.int32)
    val = _c(val, dt)
    x = _c(x, dt)
    y = np.zeros(m, dt) if y0 is None else _c(y0, dt).copy()
    getattr(L, f"oracle_csc_spmv_{suf}")(
        m, colptr.size - 1, origin, _ptr(colptr), _ptr(rowind), _ptr(val), alpha, _ptr(x), beta,
        _ptr(y))
    return y


def coo_sddmm(rows, cols, A, B, alpha=1.0, beta=0.0, C0=None, mask=None, origin=1):
    """SDDMM over a COO mask, outputs in the mask's storage order
    (oracle_coo_sddmm_*)."""
    L = lib()
    dt = np.asarray(A).dtype
    suf = _suf(dt)
    rows = _c(rows, np.int32)
    cols = _c(cols, np.int32)
    A = _f(A, dt)
    B = _f(B, dt)
    nnz = rows.size
    C = np.zeros(nnz, dt) if C0 is None else _c(C0, dt).copy()
    mk = None if mask is None else _c(mask, dt)
    getattr(L, f"oracle_coo_sddmm_{suf}")(
        nnz, origin, _ptr(rows), _ptr(cols), A.shape[1], alpha, _ptr(A), max(A.shape[0], 1),
        _ptr(B), max(B.shape[0], 1), beta, _ptr(C), _ptr(mk))
    return C


def coo_spmm(rows, cols, val, B, m, alpha=1.0, beta=0.0, C0=None, origin=1):
    """COO SpMM as the reference's ColFirst atomic path computes it: C
    pre-scaled by beta (zero fill when beta == 0), then C[row, :] +=
    (alpha*val)*B[col, :] entry by entry in storage order (oracle_coo_spmm_*)."""
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rows = _c(rows, np.int32)
    cols = _c(cols, np.int32)
    val = _c(val, dt)
    B = _f(B, dt)
    k = B.shape[1]
    C = np.zeros((m, k), dt, order="F") if C0 is None else _f(C0, dt).copy(order="F")
    getattr(L, f"oracle_coo_spmm_{suf}")(
        val.size, m, origin, _ptr(rows), _ptr(cols), _ptr(val), k, alpha, _ptr(B),
        max(B.shape[0], 1), beta, _ptr(C), max(m, 1))
    return C


def csc_spmm(colptr, rowind, val, B, m, alpha=1.0, beta=0.0, C0=None, origin=1):
    """CSC SpMM in the reference's scatter direction: C pre-scaled by beta,
    then column by column C[row, :] += (alpha*val)*B[col, :] (oracle_csc_spmm_*)."""
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    colptr = _c(colptr, np.int32)
    rowind = _c(rowind, np.int32)
    val = _c(val, dt)
    B = _f(B, dt)
    k = B.shape[1]
    C = np.zeros((m, k), dt, order="F") if C0 is None else _f(C0, dt).copy(order="F")
    getattr(L, f"oracle_csc_spmm_{suf}")(
        m, colptr.size - 1, origin, _ptr(colptr), _ptr(rowind), _ptr(val), k, alpha, _ptr(B),
        max(B.shape[0], 1), beta, _ptr(C), max(m, 1))
    return C


def expand_pos(pos, outer=None, origin=1):
    """The outer coordinate of every stored entry of a compressed level:
    outer[s] (or s + origin) repeated pos[s+1] - pos[s] times -- the
    coordinate the walker binds at the outer level for each inner entry
    (ext/KernelAbstractionsExt/ops/_walker.jl:271-392)."""
    pos = np.asarray(pos, np.int64)
    lens = np.diff(pos)
    o = np.arange(lens.size, dtype=np.int64) + origin if outer is None else np.asarray(outer, np.int64)
    return np.repeat(o, lens).astype(np.int32)


def dcsr_sddmm(outer, pos, cols, A, B, alpha=1.0, beta=0.0, C0=None, mask=None, origin=1):
    """SDDMM over a DCSR mask: the walker's compressed outer level binds the
    stored row (sddmm.jl:23-30 with _walker.jl:323-392), so entry p of stored
    row f is (outer[f], cols[p]); outputs in storage order."""
    return coo_sddmm(expand_pos(pos, outer, origin), cols, A, B, alpha, beta, C0, mask, origin)


def csc_sddmm(colptr, rowind, A, B, alpha=1.0, beta=0.0, C0=None, mask=None, origin=1):
    """SDDMM over a CSC mask by the operator's definition (C <- alpha*(A*B) o
    sparsity(C) + beta*C, sddmm.jl:1-6): entry p of column j is
    (rowind[p], j); outputs in storage order."""
    return coo_sddmm(rowind, expand_pos(colptr, None, origin), A, B, alpha, beta, C0, mask, origin)


def row_order(rows, m, origin=1):
    """(rowptr, perm): the stable row order of COO entries -- perm[q] is the
    storage position of the q-th entry in row order (ties in storage order),
    rowptr the origin-based row pointers of that order."""
    r = np.asarray(rows, np.int64) - origin
    perm = np.argsort(r, kind="stable").astype(np.int32)
    rowptr = (np.searchsorted(r[perm], np.arange(m + 1), side="left") + origin).astype(np.int32)
    return rowptr, perm


def spmm_strategy(m, k, nnz, skip_empty_rows=False) -> str:
    return SPMM_STRATEGIES[int(lib().oracle_spmm_strategy(
        m, k, nnz, int(bool(skip_empty_rows))))]


def csr_spmm(rowptr, colind, val, B, alpha=1.0, beta=0.0, C0=None, origin=1,
             skip_empty_rows=False, nthreads=None):
    """C = alpha*A*B + beta*C0 with JLUST's CPU strategy semantics.

    B is n x k column-major; returns (C, strategy_name) with C m x k
    column-major (Fortran order).
    """
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    B = _f(B, dt)
    m = rowptr.size - 1
    k = B.shape[1]
    C = np.zeros((m, k), dt, order="F") if C0 is None else _f(C0, dt).copy(
        order="F")
    strat = getattr(L, f"oracle_csr_spmm_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), _ptr(val), k, alpha, _ptr(B),
        max(B.shape[0], 1), beta, _ptr(C), max(m, 1),
        int(bool(skip_empty_rows)), nthreads or default_threads())
    return C, SPMM_STRATEGIES[strat]


def csr_spmm_absref(rowptr, colind, val, B, alpha=1.0, beta=0.0, C0=None,
                    origin=1, nthreads=None):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    B = _f(B, dt)
    m = rowptr.size - 1
    k = B.shape[1]
    out = np.empty((m, k), np.float64, order="F")
    C0f = None if C0 is None else _f(C0, dt)
    getattr(L, f"oracle_csr_spmm_absref_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), _ptr(val), k, float(alpha),
        _ptr(B), max(B.shape[0], 1), float(beta), _ptr(C0f), max(m, 1),
        _ptr(out), nthreads or default_threads())
    return out


def csr_sddmm(rowptr, colind, A, B, alpha=1.0, beta=0.0, C0=None, mask=None,
              origin=1, nthreads=None):
    """Cval = alpha*(A@B) sampled at the stored (i,j) (+beta*C0), A m x K and
    B K x n column-major; with `mask`, the alpha*dot term is multiplied by it."""
    L = lib()
    dt = np.asarray(A).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    A = _f(A, dt)
    B = _f(B, dt)
    m = rowptr.size - 1
    nnz = colind.size
    K = A.shape[1]
    C = np.zeros(nnz, dt) if C0 is None else _c(C0, dt).copy()
    mk = None if mask is None else _c(mask, dt)
    getattr(L, f"oracle_csr_sddmm_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), K, alpha, _ptr(A),
        max(A.shape[0], 1), _ptr(B), max(B.shape[0], 1), beta, _ptr(C),
        _ptr(mk), nthreads or default_threads())
    return C


def csr_sddmm_absref(rowptr, colind, A, B, alpha=1.0, beta=0.0, C0=None,
                     mask=None, origin=1, nthreads=None):
    L = lib()
    dt = np.asarray(A).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    A = _f(A, dt)
    B = _f(B, dt)
    m = rowptr.size - 1
    out = np.empty(colind.size, np.float64)
    C0c = None if C0 is None else _c(C0, dt)
    mk = None if mask is None else _c(mask, dt)
    getattr(L, f"oracle_csr_sddmm_absref_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), A.shape[1], float(alpha),
        _ptr(A), max(A.shape[0], 1), _ptr(B), max(B.shape[0], 1),
        float(beta), _ptr(C0c), _ptr(mk), _ptr(out),
        nthreads or default_threads())
    return out


def bsr_to_csr(browptr, bcolind, bval, bs, origin=1, row_major_blocks=True, b2=None):
    """Bit-exact expansion of a BSR matrix of bs x b2 blocks (b2 = bs when
    None; block values flat, nnzb*bs*b2), every stored entry kept."""
    L = lib()
    dt = np.asarray(bval).dtype
    suf = _suf(dt)
    b1 = bs
    b2 = bs if b2 is None else b2
    browptr = _c(browptr, np.int32)
    bcolind = _c(bcolind, np.int32)
    bval = _c(bval, dt).reshape(-1)
    mb = browptr.size - 1
    nnzb = bcolind.size
    rowptr = np.empty(mb * b1 + 1, np.int32)
    colind = np.empty(nnzb * b1 * b2, np.int32)
    val = np.empty(nnzb * b1 * b2, dt)
    getattr(L, f"oracle_bsr_to_csr_{suf}")(
        mb, b1, b2, origin, _ptr(browptr), _ptr(bcolind), _ptr(bval),
        int(bool(row_major_blocks)), _ptr(rowptr), _ptr(colind), _ptr(val))
    return rowptr, colind, val


def bsr_spmm(browptr, bcolind, bval, bs, B, alpha=1.0, beta=0.0, C0=None,
             origin=1, row_major_blocks=True, nthreads=None, b2=None):
    """BSR SpMM pinned by its definition: expand to CSR, run the CSR path."""
    rp, ci, v = bsr_to_csr(browptr, bcolind, bval, bs, origin,
                           row_major_blocks, b2)
    return csr_spmm(rp, ci, v, B, alpha, beta, C0, origin,
                    nthreads=nthreads)[0]


def csr_to_csc(rowptr, colind, val, n, origin=1):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    m = rowptr.size - 1
    colptr = np.empty(n + 1, np.int32)
    rowind = np.empty(colind.size, np.int32)
    cval = np.empty(colind.size, dt)
    nk = getattr(L, f"oracle_csr_to_csc_{suf}")(
        m, n, origin, _ptr(rowptr), _ptr(colind), _ptr(val), _ptr(colptr),
        _ptr(rowind), _ptr(cval))
    return colptr, rowind[:nk].copy(), cval[:nk].copy()


def csr_to_coo(rowptr, colind, val, origin=1):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rowptr = _c(rowptr, np.int32)
    colind = _c(colind, np.int32)
    val = _c(val, dt)
    m = rowptr.size - 1
    pos = np.empty(2, np.int32)
    rows = np.empty(colind.size, np.int32)
    cols = np.empty(colind.size, np.int32)
    cval = np.empty(colind.size, dt)
    nk = getattr(L, f"oracle_csr_to_coo_{suf}")(
        m, origin, _ptr(rowptr), _ptr(colind), _ptr(val), _ptr(pos),
        _ptr(rows), _ptr(cols), _ptr(cval))
    return pos, rows[:nk].copy(), cols[:nk].copy(), cval[:nk].copy()


def coo_to_csr(rows, cols, val, m, n, origin=1):
    L = lib()
    dt = np.asarray(val).dtype
    suf = _suf(dt)
    rows = _c(rows, np.int32)
    cols = _c(cols, np.int32)
    val = _c(val, dt)
    rowptr = np.empty(m + 1, np.int32)
    colind = np.empty(val.size, np.int32)
    cval = np.empty(val.size, dt)
    nk = getattr(L, f"oracle_coo_to_csr_{suf}")(
        val.size, m, n, origin, _ptr(rows), _ptr(cols), _ptr(val),
        _ptr(rowptr), _ptr(colind), _ptr(cval))
    return rowptr, colind[:nk].copy(), cval[:nk].copy()
