"""GPU parity of the operators over the remaining operand formats the
reference's EmitterBackend takes (ext/KernelAbstractionsExt/
KernelAbstractionsExt.jl:31-37, ops/sddmm.jl:12-14): SpMM with COO, CSC,
ShiftedDiag and PeriodicCSR operands; SDDMM with DCSR and CSC masks; plain
calls and prepared handles, against the CPU oracle.  Tolerance scales are
|alpha|.|A||B| + |beta||C0| computed by scipy in float64 (pinned against the
oracle's own scales in tests/test_oracle_scatter.py)."""
import numpy as np
import pytest
import scipy.sparse as sp

from tests._util import assert_within, dev, host, random_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def _origin(J, origin):
    return J.OneBased() if origin == 1 else J.ZeroBased()


def _absref_spmm(rows0, cols0, val, B, m, alpha, beta, C0):
    S = sp.coo_matrix((np.abs(np.asarray(val, np.float64)), (rows0, cols0)), shape=(m, B.shape[0]))
    r = abs(alpha) * (S @ np.abs(B.astype(np.float64)))
    if C0 is not None and beta != 0:
        r = r + abs(beta) * np.abs(C0.astype(np.float64))
    return r


def _coo(m, n, lengths, seed, origin, dtype, dup=False, shuffle=True):
    rowptr, colind, val = random_csr(m, n, lengths=lengths, seed=seed, origin=origin, dtype=dtype)
    rows = np.repeat(np.arange(origin, m + origin, dtype=np.int32), np.diff(rowptr))
    cols = colind.copy()
    if dup and rows.size:
        k = max(1, rows.size // 8)
        rows, cols, val = np.r_[rows, rows[:k]], np.r_[cols, cols[:k]], np.r_[val, val[:k]]
    if shuffle:
        p = np.random.default_rng(seed + 100).permutation(rows.size)
        rows, cols, val = rows[p], cols[p], val[p]
    return rows.astype(np.int32), cols.astype(np.int32), val.astype(dtype)


def _C(J, m, k, dtype, C0):
    import torch
    if C0 is None:
        return J.dense_matrix(m, k, dtype=torch.float64 if dtype == np.float64 else torch.float32,
                              fill=float("nan"))
    return dev(np.asfortranarray(C0))


# ------------------------------------------------------------------ COO SpMM

@pytest.mark.parametrize("k", [1, 3, 8, 40, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_coo_spmm_plain(J, O, k, dtype):
    m, n = 2500, 1800
    origin = 1 if k % 2 else 0
    lens = np.random.default_rng(k).integers(0, 40, m)
    lens[5] = 1500                                       # a long row (split in plans)
    rows, cols, val = _coo(m, n, lens, k, origin, dtype, dup=True)
    rng = np.random.default_rng(k + 1)
    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    alpha, beta = (1.0, 0.0) if k < 8 else (0.75, -0.5)
    C0 = None if beta == 0 else np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n), origin=_origin(J, origin))
    C = _C(J, m, k, dtype, C0)
    J.execute(J.SpMMOp, A, dev(B), C, alpha=alpha, beta=beta)
    ref = O.coo_spmm(rows, cols, val, B, m, alpha, beta, C0, origin)
    assert_within(host(C), ref, _absref_spmm(rows - origin, cols - origin, val, B, m, alpha, beta, C0),
                  dtype, f"COO SpMM k={k}")


def test_coo_spmm_sorted_rows_and_empty(J, O):
    """Row-ordered COO (no reordering) and an all-empty matrix (C = beta*C)."""
    m, n, k = 900, 700, 16
    rows, cols, val = _coo(m, n, np.random.default_rng(3).integers(0, 9, m), 3, 1, np.float64,
                           shuffle=False)
    B = np.asfortranarray(np.random.default_rng(4).standard_normal((n, k)))
    A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n))
    C = _C(J, m, k, np.float64, None)
    J.execute(J.SpMMOp, A, dev(B), C)
    ref = O.coo_spmm(rows, cols, val, B, m)
    assert_within(host(C), ref, _absref_spmm(rows - 1, cols - 1, val, B, m, 1.0, 0.0, None),
                  np.float64, "sorted COO")
    E = J.coo_tensor(dev(np.zeros(0, np.int32)), dev(np.zeros(0, np.int32)), dev(np.zeros(0)), (m, n))
    C0 = np.asfortranarray(np.random.default_rng(5).standard_normal((m, k)))
    C = dev(C0)
    J.execute(J.SpMMOp, E, dev(B), C, alpha=2.0, beta=0.5)
    np.testing.assert_array_equal(host(C), 0.5 * C0)
    C = _C(J, m, k, np.float64, None)
    J.execute(J.SpMMOp, E, dev(B), C)
    assert (host(C) == 0).all()


def test_coo_spmm_bad_row(J):
    A = J.coo_tensor(dev(np.array([1, 5], np.int32)), dev(np.array([1, 1], np.int32)),
                     dev(np.ones(2)), (3, 3))
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(J.SpMMOp, A, dev(np.asfortranarray(np.ones((3, 2)))), J.dense_matrix(3, 2))


# ------------------------------------------------------------------ CSC SpMM

@pytest.mark.parametrize("k", [1, 5, 64, 130])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csc_spmm_plain(J, O, k, dtype):
    m, n = 2100, 2600
    origin = 0 if k % 2 else 1
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(k + 7).integers(0, 30, m),
                                     seed=k + 7, origin=origin, dtype=dtype)
    cp, ri, cv = O.csr_to_csc(rowptr, colind, val, n, origin)
    rng = np.random.default_rng(k + 8)
    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    alpha, beta = (-1.25, 0.5) if k > 1 else (1.0, 0.0)
    C0 = None if beta == 0 else np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    A = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n), origin=_origin(J, origin))
    C = _C(J, m, k, dtype, C0)
    J.execute(J.SpMMOp, A, dev(B), C, alpha=alpha, beta=beta)
    ref = O.csc_spmm(cp, ri, cv, B, m, alpha, beta, C0, origin)
    cols0 = O.expand_pos(cp, None, origin) - origin
    assert_within(host(C), ref, _absref_spmm(ri - origin, cols0, cv, B, m, alpha, beta, C0), dtype,
                  f"CSC SpMM k={k}")


def test_csc_spmm_bad_colptr(J):
    A = J.csc_tensor(dev(np.array([1, 3, 2, 4], np.int32)), dev(np.array([1, 2, 3], np.int32)),
                     dev(np.ones(3)), (3, 3))
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(J.SpMMOp, A, dev(np.asfortranarray(np.ones((3, 2)))), J.dense_matrix(3, 2))


# --------------------------------------------------- prepared COO/CSC SpMM

@pytest.mark.parametrize("fmt", ["COO", "COO_sorted", "CSC"])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_coo_csc_spmm_plans(J, O, fmt, dtype):
    """prepare(SpMMOp, A) for COO/CSC: equal to the plain call's result within
    the bar; values written in place through torch are seen; update_values_
    with another tensor; a second k rebuilds the plan."""
    import torch
    m, n, k = 1700, 1300, 24
    if fmt.startswith("COO"):
        rows, cols, val = _coo(m, n, np.random.default_rng(9).integers(0, 25, m), 9, 1, dtype,
                               dup=fmt == "COO", shuffle=fmt == "COO")
        A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n))
        ref_of = lambda v, B, a, b, C0: O.coo_spmm(rows, cols, v, B, m, a, b, C0)  # noqa: E731
        r0, c0 = rows - 1, cols - 1
    else:
        rowptr, colind, v0 = random_csr(m, n, lengths=np.random.default_rng(9).integers(0, 25, m),
                                        seed=9, dtype=dtype)
        cp, ri, val = O.csr_to_csc(rowptr, colind, v0, n)
        A = J.csc_tensor(dev(cp), dev(ri), dev(val), (m, n))
        ref_of = lambda v, B, a, b, C0: O.csc_spmm(cp, ri, v, B, m, a, b, C0)  # noqa: E731
        r0, c0 = ri - 1, O.expand_pos(cp, None, 1) - 1
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    assert h.info()["reordered"] == (fmt != "COO_sorted")
    rng = np.random.default_rng(10)
    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    C = dev(C0)
    J.execute(h, dev(B), C, alpha=1.5, beta=-0.25)
    assert_within(host(C), ref_of(val, B, 1.5, -0.25, C0),
                  _absref_spmm(r0, c0, val, B, m, 1.5, -0.25, C0), dtype, f"{fmt} plan")
    # values written in place through torch
    J.nonzeros(A).mul_(-2.0)
    val2 = (-2.0 * val).astype(dtype)
    C = _C(J, m, k, dtype, None)
    J.execute(h, dev(B), C)
    assert_within(host(C), ref_of(val2, B, 1.0, 0.0, None), _absref_spmm(r0, c0, val2, B, m, 1.0, 0.0, None),
                  dtype, f"{fmt} plan after in-place write")
    # another value tensor through update_values_
    val3 = rng.uniform(-1, 1, val.size).astype(dtype)
    A3 = J.USTensor(A.extents, A.format, A.pos_buffers, A.crd_buffers, dev(val3), None, A.origin)
    J.update_values_(h, A3)
    C = _C(J, m, k, dtype, None)
    J.execute(h, dev(B), C)
    assert_within(host(C), ref_of(val3, B, 1.0, 0.0, None), _absref_spmm(r0, c0, val3, B, m, 1.0, 0.0, None),
                  dtype, f"{fmt} plan after update_values_")
    # another k
    B5 = np.asfortranarray(rng.standard_normal((n, 5)).astype(dtype))
    C = _C(J, m, 5, dtype, None)
    J.execute(h, dev(B5), C)
    assert_within(host(C), ref_of(val3, B5, 1.0, 0.0, None),
                  _absref_spmm(r0, c0, val3, B5, m, 1.0, 0.0, None), dtype, f"{fmt} plan k=5")
    torch.cuda.synchronize()


# ---------------------------------------------- ShiftedDiag / PeriodicCSR SpMM

@pytest.mark.parametrize("shift", [0, 3, -5])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_shifted_diag_spmm(J, O, shift, dtype):
    import torch
    m, n, k = 300, 280, 7
    T = torch.float64 if dtype == np.float64 else torch.float32
    A = J.shifted_diag_tensor(T, m, n, shift=shift, val=-2.5)
    rng = np.random.default_rng(11)
    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    C = dev(C0)
    J.execute(J.SpMMOp, A, dev(B), C, alpha=0.5, beta=2.0)
    r = np.arange(m)
    ok = (r + shift >= 0) & (r + shift < n)
    rowptr = np.r_[0, np.cumsum(ok)].astype(np.int32) + 1
    colind = (r[ok] + shift + 1).astype(np.int32)
    val = np.full(colind.size, -2.5, dtype)
    ref, _ = O.csr_spmm(rowptr, colind, val, B, 0.5, 2.0, C0)
    absref = O.csr_spmm_absref(rowptr, colind, val, B, 0.5, 2.0, C0)
    assert_within(host(C), ref, absref, dtype, f"ShiftedDiag SpMM shift={shift}")


@pytest.mark.parametrize("T", [1, 3, 8])
def test_periodic_csr_spmm(J, O, T):
    br, bc, k = 60, 45, 6
    rowptr, colind, val = random_csr(br, bc, density=0.2, seed=12 + T)
    block = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (br, bc))
    A = J.periodic_csr_tensor(block, T)
    rng = np.random.default_rng(13)
    B = np.asfortranarray(rng.standard_normal((T * bc, k)))
    C0 = np.asfortranarray(rng.standard_normal((T * br, k)))
    C = dev(C0)
    J.execute(J.SpMMOp, A, dev(B), C, alpha=1.5, beta=-1.0)
    S = sp.block_diag([sp.csr_matrix((val, colind - 1, rowptr - 1), shape=(br, bc))] * T, format="csr")
    S.sort_indices()
    rp = (S.indptr + 1).astype(np.int32)
    ci = (S.indices + 1).astype(np.int32)
    ref, _ = O.csr_spmm(rp, ci, S.data, B, 1.5, -1.0, C0)
    absref = O.csr_spmm_absref(rp, ci, S.data, B, 1.5, -1.0, C0)
    assert_within(host(C), ref, absref, np.float64, f"PeriodicCSR SpMM T={T}")


# -------------------------------------------------------------- DCSR SDDMM

def _dcsr_mask(m, n, seed, origin, dtype):
    lens = np.random.default_rng(seed).integers(0, 14, m)
    lens[::4] = 0
    lens[7] = min(n, 900)                                  # one long stored row
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=seed, origin=origin, dtype=dtype)
    keep = np.flatnonzero(np.diff(rowptr) > 0)
    outer = (keep + origin).astype(np.int32)
    pos = (np.r_[0, np.cumsum(np.diff(rowptr)[keep])] + origin).astype(np.int32)
    return outer, pos, colind, val


@pytest.mark.parametrize("K", [1, 4, 16, 128, 9000])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_dcsr_sddmm(J, O, K, dtype):
    m, n = 1200, 1000
    origin = 1 if K % 2 else 0
    outer, pos, cols, val = _dcsr_mask(m, n, K, origin, dtype)
    rng = np.random.default_rng(K + 1)
    Ad = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    Bd = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    mask = rng.uniform(0.5, 1.5, cols.size).astype(dtype)
    C = J.dcsr_tensor(dev(outer), dev(pos), dev(cols), dev(val), (m, n), origin=_origin(J, origin))
    J.execute(J.SDDMMOp, dev(Ad), dev(Bd), C, alpha=0.5, beta=-1.0, mask=dev(mask))
    ref = O.dcsr_sddmm(outer, pos, cols, Ad, Bd, 0.5, -1.0, val, mask, origin)
    rows0 = O.expand_pos(pos, outer, origin) - origin
    dots = (np.abs(Ad.astype(np.float64)) @ np.abs(Bd.astype(np.float64)))[rows0, cols - origin]
    absref = 0.5 * np.abs(mask) * dots + np.abs(val.astype(np.float64))
    assert_within(host(J.nonzeros(C)), ref, absref, dtype, f"DCSR SDDMM K={K}")
    # the prepared handle, on the original values
    C2 = J.dcsr_tensor(dev(outer), dev(pos), dev(cols), dev(val), (m, n), origin=_origin(J, origin))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, dev(Ad), dev(Bd), C2)
    J.execute(h, dev(Ad), dev(Bd), C2, alpha=0.5, beta=-1.0, mask=dev(mask))
    assert_within(host(J.nonzeros(C2)), ref, absref, dtype, f"DCSR SDDMM plan K={K}")


def test_dcsr_sddmm_rows_not_increasing(J):
    C = J.dcsr_tensor(dev(np.array([2, 1], np.int32)), dev(np.array([1, 2, 3], np.int32)),
                      dev(np.array([1, 2], np.int32)), dev(np.zeros(2)), (3, 3))
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(J.SDDMMOp, dev(np.asfortranarray(np.ones((3, 4)))),
                  dev(np.asfortranarray(np.ones((4, 3)))), C)


# --------------------------------------------------------------- CSC SDDMM

@pytest.mark.parametrize("K", [2, 8, 64, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csc_sddmm(J, O, K, dtype):
    m, n = 1400, 1100
    origin = 0 if K % 16 else 1
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(K + 20).integers(0, 20, m),
                                     seed=K + 20, origin=origin, dtype=dtype)
    cp, ri, cv = O.csr_to_csc(rowptr, colind, val, n, origin)
    rng = np.random.default_rng(K + 21)
    Ad = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    Bd = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    cols0 = O.expand_pos(cp, None, origin) - origin
    dots = (np.abs(Ad.astype(np.float64)) @ np.abs(Bd.astype(np.float64)))[ri - origin, cols0]
    for beta in (0.0, 0.5):
        C = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n), origin=_origin(J, origin))
        if beta == 0:
            J.nonzeros(C).fill_(float("nan"))
        J.execute(J.SDDMMOp, dev(Ad), dev(Bd), C, alpha=2.0, beta=beta)
        ref = O.csc_sddmm(cp, ri, Ad, Bd, 2.0, beta, cv, None, origin)
        absref = 2.0 * dots + abs(beta) * np.abs(cv.astype(np.float64))
        assert_within(host(J.nonzeros(C)), ref, absref, dtype, f"CSC SDDMM K={K} beta={beta}")
    C2 = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n), origin=_origin(J, origin))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, C2, n_inner=K)
    assert h.info()["reordered"]
    J.execute(h, dev(Ad), dev(Bd), alpha=2.0, beta=0.5)
    ref = O.csc_sddmm(cp, ri, Ad, Bd, 2.0, 0.5, cv, None, origin)
    absref = 2.0 * dots + 0.5 * np.abs(cv.astype(np.float64))
    assert_within(host(J.nonzeros(C2)), ref, absref, dtype, f"CSC SDDMM plan K={K}")
