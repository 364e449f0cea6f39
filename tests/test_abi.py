"""The C ABI library (no GPU needed): it loads, exports every symbol that
include/jlust_hip.h declares, and its host-only entry points behave.  No
compute entry point is called here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "jlust_hip.h")
LIB = os.path.join(ROOT, "jlust_amd", "libjlust_hip.so")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jlust_hip_\w+)\s*\(", text)))


def test_header_declares_expected_surface():
    syms = declared_symbols()
    for must in ("jlust_hip_csr_spmv_f64_i32", "jlust_hip_csr_spmv_f32_i32",
                 "jlust_hip_coo_spmv_f64_i32", "jlust_hip_csr_spmm_f32_i32",
                 "jlust_hip_csr_sddmm_f32_i32", "jlust_hip_bsr_spmm_f32_i32",
                 "jlust_hip_csr_spmv_plan_create", "jlust_hip_last_error"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build first: python -m jlust_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (jlust_hip_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_python_signatures_cover_header():
    from jlust_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_load_version_and_error_buffer():
    from jlust_amd import _lib
    L = _lib.lib()
    assert L.jlust_hip_version() == 2
    assert isinstance(_lib.last_error(), str)


def _check(rowptr, colind, m, n, origin=1, sorted_=1):
    from jlust_amd import _lib
    rp = np.ascontiguousarray(rowptr, np.int32)
    ci = np.ascontiguousarray(colind, np.int32)
    return _lib.lib().jlust_hip_check_csr(m, n, ci.size, origin, rp.ctypes.data_as(ctypes.c_void_p),
                                          ci.ctypes.data_as(ctypes.c_void_p), sorted_)


def test_host_structural_check():
    from jlust_amd import _lib
    assert _check([1, 3, 4, 6], [1, 3, 2, 1, 3], 3, 3) == 0
    assert _check([0, 2, 3, 5], [0, 2, 1, 0, 2], 3, 3, origin=0) == 0
    assert _check([1, 3, 2, 6], [1, 3, 2, 1, 3], 3, 3) == 4          # rowptr decreases
    assert "decreases" in _lib.last_error()
    assert _check([1, 3, 4, 6], [1, 4, 2, 1, 3], 3, 3) == 4          # column out of range
    assert _check([1, 3, 4, 6], [3, 1, 2, 1, 3], 3, 3) == 4          # unsorted
    assert _check([1, 3, 4, 6], [3, 1, 2, 1, 3], 3, 3, sorted_=0) == 0
    assert _check([2, 3, 4, 6], [1, 3, 2, 1, 3], 3, 3) == 4          # rowptr[0] != origin
    assert _check([1, 3, 4, 6], [1, 3, 2, 1, 3], 3, 3, origin=2) == 5


def test_status_mapping_to_reference_exceptions():
    import jlust_amd as J
    from jlust_amd import _lib
    for code, exc in ((1, J.IncompatibleExtents), (2, J.UnsupportedValueType),
                      (3, J.UnsupportedFormat), (4, J.NonCanonicalStorage),
                      (5, J.IndexOriginMismatch), (7, J.NoDevice), (6, J.HIPError),
                      (10, J.UnsupportedIndexType)):
        with pytest.raises(exc):
            _lib.check(code, "test")
    _lib.check(0, "ok")


def test_bbm_periodic_argument_checks():
    """jlust_hip_bbm_periodic_spmv_*: sizes, block extents and block formats
    are checked on the host before anything reaches the device (the host
    addresses below stand in for device buffers and are never read)."""
    from jlust_amd import _lib
    from jlust_amd.block_sparse import Placement
    from jlust_amd.convert import Sparse
    L = _lib.lib()
    buf = np.zeros(64, np.int64)
    p = buf.ctypes.data

    def csr(m, n, fmt=0):
        s = Sparse(format=fmt, origin=0, m=m, n=n, nnz=4, pos1=p, crd1=p, pos2=p, crd2=p, val=p)
        return Placement(block=ctypes.pointer(s))

    def sd(m, n):
        return Placement(diag_m=m, diag_n=n, diag_shift=0, diag_val=1.0)

    def call(T, nd, no, nc, d, neg, pos):
        return L.jlust_hip_bbm_periodic_spmv_f64(T, nd, no, nc, ctypes.byref(d), ctypes.byref(neg),
                                                 ctypes.byref(pos), 1.0, p, 0.0, p, None)

    assert call(0, 4, 2, 5, csr(4, 5), sd(2, 5), sd(2, 5)) == 1            # T < 1
    assert call(3, 2 ** 31, 2, 5, csr(4, 5), sd(2, 5), sd(2, 5)) == 1      # rows beyond 32 bits
    assert "32-bit" in _lib.last_error()
    assert call(3, 4, 2, 5, csr(4, 6), sd(2, 5), sd(2, 5)) == 1            # diagonal extents
    assert "diagonal block is 4 x 6" in _lib.last_error()
    assert call(3, 4, 2, 5, csr(4, 5), sd(3, 5), sd(2, 5)) == 1            # neg extents
    assert call(3, 4, 2, 5, csr(4, 5), sd(2, 5), csr(2, 4)) == 1           # pos extents
    assert call(3, 4, 2, 5, csr(4, 5, fmt=2), sd(2, 5), sd(2, 5)) == 3     # COO diagonal
    assert call(3, 4, 2, 5, csr(4, 5), csr(2, 5, fmt=3), sd(2, 5)) == 3    # DCSR coupling
    assert "CSR or a shifted diagonal" in _lib.last_error()
    with pytest.raises(TypeError):
        L.jlust_hip_bbm_periodic_spmv_f64(3, 4, 2, 5)                      # arity from the header
