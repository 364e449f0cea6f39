"""Pins the oracle's COO/CSC SpMM, DCSR/CSC SDDMM and index helpers, and the
tolerance scales (|alpha||A||x| + |beta||y0|) every GPU parity test uses:
  - scipy.sparse: coo_matvecs adds data*X[col] into Y[row] entry by entry in
    storage order and csc_matvecs column by column, from zero -- the
    reference's atomic/scatter sums applied in storage order, so alpha = 1,
    beta = 0 must be bit-identical;
  - the pre-scale semantics of ext/KernelAbstractionsExt/ops/spmm.jl:412-416
    (zero fill when beta == 0, NaN in C dropped; beta*C otherwise) by closed
    form;
  - SDDMM over DCSR/CSC masks against the plain float64 dense product sampled
    at the stored positions;
  - the absref scales against independent numpy/scipy |A|.|x| in float64,
    with planted mistakes (a scale off by a factor, a dropped beta term) that
    the comparison rejects.
"""
import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle as O
from tests._util import random_csr


def _coo_of(m, n, density, seed, origin=1, dtype=np.float64, dup=False):
    rowptr, colind, val = random_csr(m, n, density=density, seed=seed, origin=origin, dtype=dtype)
    rows = np.repeat(np.arange(origin, m + origin, dtype=np.int32), np.diff(rowptr))
    cols = colind.copy()
    if dup:                                   # duplicate entries, as COO allows
        k = max(1, rows.size // 10)
        rows = np.r_[rows, rows[:k]]
        cols = np.r_[cols, cols[:k]]
        val = np.r_[val, val[:k]]
    perm = np.random.default_rng(seed + 1).permutation(rows.size)
    return rows[perm], cols[perm], val[perm].astype(dtype)


# ---------------------------------------------------------------- COO SpMM

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [1, 0])
def test_coo_spmm_bitexact_scipy(dtype, origin):
    m, n, k = 300, 250, 7
    rows, cols, val = _coo_of(m, n, 0.05, 3, origin, dtype, dup=True)
    B = np.asfortranarray(np.random.default_rng(4).standard_normal((n, k)).astype(dtype))
    C = O.coo_spmm(rows, cols, val, B, m, origin=origin)
    S = sp.coo_matrix((val, (rows - origin, cols - origin)), shape=(m, n))
    Cs = S @ B
    assert Cs.dtype == dtype
    np.testing.assert_array_equal(C, Cs)
    # planted mistakes: rows and columns swapped (square part), B reversed.
    assert not np.array_equal(O.coo_spmm(rows, cols, val, B[::-1].copy(order="F"), m, origin=origin), Cs)
    rs, cs, vs = _coo_of(200, 200, 0.05, 5, origin, dtype)
    Bs = np.asfortranarray(np.random.default_rng(6).standard_normal((200, 3)).astype(dtype))
    good = sp.coo_matrix((vs, (rs - origin, cs - origin)), shape=(200, 200)) @ Bs
    np.testing.assert_array_equal(O.coo_spmm(rs, cs, vs, Bs, 200, origin=origin), good)
    assert not np.array_equal(O.coo_spmm(cs, rs, vs, Bs, 200, origin=origin), good)


def test_coo_spmm_prescale():
    """beta == 0 fills C with zeros first (a NaN in C0 does not survive);
    beta != 0 scales C0, then the alpha*val*B terms are added."""
    m, n, k = 40, 30, 4
    rows, cols, val = _coo_of(m, n, 0.2, 7)
    B = np.asfortranarray(np.random.default_rng(8).standard_normal((n, k)))
    C0 = np.asfortranarray(np.full((m, k), np.nan))
    C = O.coo_spmm(rows, cols, val, B, m, 1.0, 0.0, C0)
    assert not np.isnan(C).any()
    C0 = np.asfortranarray(np.random.default_rng(9).standard_normal((m, k)))
    C = O.coo_spmm(rows, cols, val, B, m, 2.0, 0.5, C0)
    want = 0.5 * C0
    for p in range(rows.size):
        want[rows[p] - 1, :] += (2.0 * val[p]) * B[cols[p] - 1, :]
    np.testing.assert_array_equal(C, want)
    # an empty row keeps beta*C0 only
    empty = np.setdiff1d(np.arange(m), rows - 1)
    if empty.size:
        np.testing.assert_array_equal(C[empty], 0.5 * C0[empty])


# ---------------------------------------------------------------- CSC SpMM

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [1, 0])
def test_csc_spmm_bitexact_scipy(dtype, origin):
    m, n, k = 260, 310, 9
    rowptr, colind, val = random_csr(m, n, density=0.04, seed=11, origin=origin, dtype=dtype)
    cp, ri, cv = O.csr_to_csc(rowptr, colind, val, n, origin)
    B = np.asfortranarray(np.random.default_rng(12).standard_normal((n, k)).astype(dtype))
    C = O.csc_spmm(cp, ri, cv, B, m, origin=origin)
    Cs = sp.csc_matrix((cv, ri - origin, cp - origin), shape=(m, n)) @ B
    np.testing.assert_array_equal(C, Cs)
    # the CSC arrays read as CSR (A^T B on a square problem) fail the check
    rs, cs, vs = random_csr(150, 150, density=0.05, seed=13, origin=origin, dtype=dtype)
    cps, ris, cvs = O.csr_to_csc(rs, cs, vs, 150, origin)
    Bs = np.asfortranarray(np.random.default_rng(14).standard_normal((150, 3)).astype(dtype))
    good = sp.csc_matrix((cvs, ris - origin, cps - origin), shape=(150, 150)) @ Bs
    np.testing.assert_array_equal(O.csc_spmm(cps, ris, cvs, Bs, 150, origin=origin), good)
    bad, _ = O.csr_spmm(cps, ris, cvs, Bs, origin=origin)
    assert not np.array_equal(bad, good)


def test_csc_spmm_column_equals_csc_spmv():
    """Column c of the CSC SpMM is the CSC scatter SpMV with x = B[:, c],
    alpha and beta included (the same sequential adds)."""
    m, n, k = 90, 70, 5
    rowptr, colind, val = random_csr(m, n, density=0.1, seed=15)
    cp, ri, cv = O.csr_to_csc(rowptr, colind, val, n)
    rng = np.random.default_rng(16)
    B = np.asfortranarray(rng.standard_normal((n, k)))
    C0 = np.asfortranarray(rng.standard_normal((m, k)))
    C = O.csc_spmm(cp, ri, cv, B, m, 0.75, -1.25, C0)
    for c in range(k):
        np.testing.assert_array_equal(C[:, c], O.csc_spmv(cp, ri, cv, B[:, c], m, 0.75, -1.25, C0[:, c]))


# ---------------------------------------------------------- DCSR / CSC SDDMM

def _sampled_dense(A, B, rows0, cols0):
    D = A.astype(np.float64) @ B.astype(np.float64)
    return D[rows0, cols0]


@pytest.mark.parametrize("origin", [1, 0])
def test_dcsr_sddmm_reference_fixture_rows_and_dense(origin):
    """The DCSR mask of test_emitter.jl's fixture matrix (rows 1 and 3 of
    [1 0 2; 0 0 0; 4 0 5]): entry p of stored row f is (outer[f], cols[p]);
    against the float64 dense product sampled there, and the CSR result with
    the empty row present (bit-identical: the same sequential dot)."""
    outer = np.array([0, 2], np.int32) + origin
    pos = np.array([0, 2, 4], np.int32) + origin
    cols = np.array([0, 2, 0, 2], np.int32) + origin
    rng = np.random.default_rng(17)
    A = np.asfortranarray(rng.standard_normal((3, 5)))
    B = np.asfortranarray(rng.standard_normal((5, 3)))
    out = O.dcsr_sddmm(outer, pos, cols, A, B, origin=origin)
    np.testing.assert_allclose(out, _sampled_dense(A, B, [0, 0, 2, 2], [0, 2, 0, 2]), rtol=1e-14)
    rowptr = np.array([0, 2, 2, 4], np.int32) + origin
    np.testing.assert_array_equal(out, O.csr_sddmm(rowptr, cols, A, B, origin=origin))


def test_dcsr_sddmm_random_equals_csr():
    m, n, K = 500, 300, 16
    lens = np.random.default_rng(18).integers(0, 12, m)
    lens[::3] = 0                                     # every third row empty
    rowptr, colind, _ = random_csr(m, n, lengths=lens, seed=19)
    keep = np.flatnonzero(np.diff(rowptr) > 0)
    outer = (keep + 1).astype(np.int32)
    pos = np.r_[0, np.cumsum(np.diff(rowptr)[keep])].astype(np.int32) + 1
    rng = np.random.default_rng(20)
    A = np.asfortranarray(rng.standard_normal((m, K)))
    B = np.asfortranarray(rng.standard_normal((K, n)))
    C0 = rng.standard_normal(colind.size)
    mask = rng.uniform(0.5, 1.5, colind.size)
    np.testing.assert_array_equal(O.dcsr_sddmm(outer, pos, colind, A, B, 1.5, -0.5, C0, mask),
                                  O.csr_sddmm(rowptr, colind, A, B, 1.5, -0.5, C0, mask))


@pytest.mark.parametrize("origin", [1, 0])
def test_csc_sddmm_definition(origin):
    """A CSC mask's entry p of column j is (rowind[p], j): outputs in CSC
    storage order equal the CSR-mask outputs permuted the way csr_to_csc
    permutes the entries, and the dense product sampled there.  The
    reference's gather walker would read (j, rowind[p]) instead (a transposed
    mask): that reading fails the dense check on a non-symmetric problem."""
    m, n, K = 120, 90, 11
    rowptr, colind, val = random_csr(m, n, density=0.06, seed=21, origin=origin)
    # the CSR entry index as the value: csr_to_csc carries it to the CSC order
    idx = np.arange(colind.size, dtype=np.float64)
    cp, ri, ci = O.csr_to_csc(rowptr, colind, idx + 1.0, n, origin)
    perm = (ci - 1.0).astype(np.int64)
    rng = np.random.default_rng(22)
    A = np.asfortranarray(rng.standard_normal((m, K)))
    B = np.asfortranarray(rng.standard_normal((K, n)))
    C0 = rng.standard_normal(colind.size)
    csr = O.csr_sddmm(rowptr, colind, A, B, 0.5, 2.0, C0, origin=origin)
    csc = O.csc_sddmm(cp, ri, A, B, 0.5, 2.0, C0[perm], origin=origin)
    np.testing.assert_array_equal(csc, csr[perm])
    cols0 = O.expand_pos(cp, None, origin) - origin
    plain = O.csc_sddmm(cp, ri, A, B, origin=origin)
    np.testing.assert_allclose(plain, _sampled_dense(A, B, ri - origin, cols0), rtol=1e-12, atol=1e-13)
    # planted: the transposed reading (A[j,:].B[:,i]) on a square problem
    As = np.asfortranarray(rng.standard_normal((m, K)))
    Bs = np.asfortranarray(rng.standard_normal((K, m)))
    rs, cs, vs = random_csr(m, m, density=0.06, seed=23, origin=origin)
    cps, ris, _ = O.csr_to_csc(rs, cs, vs, m, origin)
    cols_s = O.expand_pos(cps, None, origin)
    good = O.csc_sddmm(cps, ris, As, Bs, origin=origin)
    np.testing.assert_allclose(good, _sampled_dense(As, Bs, ris - origin, cols_s - origin), rtol=1e-12,
                               atol=1e-13)
    swapped = O.coo_sddmm(cols_s, ris, As, Bs, origin=origin)
    assert not np.allclose(swapped, good)


# ------------------------------------------------------------ index helpers

def test_expand_pos_and_row_order():
    pos = np.array([1, 1, 3, 3, 4, 7], np.int32)          # empty segments 0 and 2
    assert O.expand_pos(pos, None, 1).tolist() == [2, 2, 4, 5, 5, 5]
    assert O.expand_pos(pos, np.array([10, 20, 30, 40, 50]), 1).tolist() == [20, 20, 40, 50, 50, 50]
    rows = np.array([3, 1, 3, 2, 1, 3], np.int32)
    rowptr, perm = O.row_order(rows, 4, origin=1)
    assert perm.tolist() == [1, 4, 3, 0, 2, 5]            # stable: ties keep storage order
    assert rowptr.tolist() == [1, 3, 4, 7, 7]              # row 4 empty
    # against scipy's canonical COO -> CSR on entries without duplicates
    r, c, v = _coo_of(60, 50, 0.1, 24)
    rp, pm = O.row_order(r, 60)
    S = sp.coo_matrix((v, (r - 1, c - 1)), shape=(60, 50)).tocsr()
    assert (rp - 1).tolist() == S.indptr.tolist()


# --------------------------------------------------------- tolerance scales

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_absref_scales_against_numpy(dtype):
    """csr_spmv_absref, csr_spmm_absref and csr_sddmm_absref equal
    |alpha|.|A||x| + |beta||y0| computed independently (scipy with absolute
    values, float64), elementwise to the last bits of float64; planted scales
    (off by a factor 2, beta term dropped) are rejected."""
    m, n, k, K = 400, 300, 6, 10
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(25).integers(0, 30, m),
                                     seed=26, dtype=dtype)
    rng = np.random.default_rng(27)
    Sabs = sp.csr_matrix((np.abs(val.astype(np.float64)), colind - 1, rowptr - 1), shape=(m, n))
    alpha, beta = -1.5, 0.25
    x = rng.uniform(-1, 1, n).astype(dtype)
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    want = abs(alpha) * (Sabs @ np.abs(x.astype(np.float64))) + abs(beta) * np.abs(y0.astype(np.float64))
    got = O.csr_spmv_absref(rowptr, colind, val, x, alpha, beta, y0)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=0)
    assert not np.allclose(2.0 * got, want, rtol=1e-3)
    got_nob = O.csr_spmv_absref(rowptr, colind, val, x, alpha, 0.0, y0)
    assert not np.allclose(got_nob, want, rtol=1e-3)

    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    want = abs(alpha) * (Sabs @ np.abs(B.astype(np.float64))) + abs(beta) * np.abs(C0.astype(np.float64))
    got = O.csr_spmm_absref(rowptr, colind, val, B, alpha, beta, C0)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=0)
    assert not np.allclose(0.5 * got, want, rtol=1e-3)

    A = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    Bd = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    Cv = rng.standard_normal(colind.size).astype(dtype)
    mask = rng.uniform(0.5, 1.5, colind.size).astype(dtype)
    rows0 = np.repeat(np.arange(m), np.diff(rowptr))
    dots = (np.abs(A.astype(np.float64)) @ np.abs(Bd.astype(np.float64)))[rows0, colind - 1]
    want = abs(alpha) * np.abs(mask.astype(np.float64)) * dots + abs(beta) * np.abs(Cv.astype(np.float64))
    got = O.csr_sddmm_absref(rowptr, colind, A, Bd, alpha, beta, Cv, mask)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=0)
    assert not np.allclose(got - abs(beta) * np.abs(Cv.astype(np.float64)), want, rtol=1e-3)
