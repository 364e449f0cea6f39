"""Pins the CPU oracle (oracle/jlust_cpu.c) before it is trusted as the
parity reference:
  - the reference's own known answers (tests/golden, transcribed from
    test/test_emitter.jl, test/test_convert.jl, test/test_cuda.jl);
  - scipy.sparse, whose csr_matvec/csr_matvecs sum each output sequentially
    from zero in storage order without FMA, exactly like JLUST's scalar walker
    (_walker.jl:123-132): results must be bit-identical;
  - brute force in extended precision, invariants (SpMM column == SpMV,
    BSR == dense block product) and closed forms (permutation, shifted
    diagonal);
  - planted mistakes (wrong origin, transposed operand, dropped term) that the
    checks above must reject.
"""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import oracle as O
from tests._util import random_csr

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))


def dcsr_to_csr(case):
    """DCSR (outer_crd, inner_pos, inner_crd) -> CSR with empty absent rows."""
    o = case["origin"]
    m = case["m"]
    lens = np.zeros(m, np.int64)
    ip = np.array(case["inner_pos"])
    for f, r in enumerate(case["outer_crd"]):
        lens[r - o] = ip[f + 1] - ip[f]
    rowptr = (np.r_[0, np.cumsum(lens)] + o).astype(np.int32)
    return rowptr, np.array(case["inner_crd"], np.int32)


def to_scipy(rowptr, colind, val, shape, origin=1):
    return sp.csr_matrix((val, colind - origin, rowptr - origin), shape=shape)


# ---------------------------------------------------------------- fixtures

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmv_reference_fixtures(dtype):
    for c in GOLDEN["spmv"]:
        x = np.array(c["x"], dtype)
        if c["format"] == "CSR":
            y = O.csr_spmv(c["rowptr"], c["colind"], np.array(c["val"], dtype), x,
                           origin=c["origin"])
        elif c["format"] == "DCSR":
            rp, ci = dcsr_to_csr(c)
            y = O.csr_spmv(rp, ci, np.array(c["val"], dtype), x, origin=c["origin"])
        else:
            y = O.coo_spmv(c["rows"], c["cols"], np.array(c["val"], dtype), x, c["m"],
                           origin=c["origin"])
        np.testing.assert_array_equal(y, np.array(c["y"], dtype), err_msg=c["name"])


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_reference_fixtures(dtype):
    for c in GOLDEN["spmm"]:
        B = np.asfortranarray(np.array(c["B"], dtype))
        if c["format"] == "CSR":
            rp, ci = np.array(c["rowptr"], np.int32), np.array(c["colind"], np.int32)
        else:
            rp, ci = dcsr_to_csr(c)
        C, strat = O.csr_spmm(rp, ci, np.array(c["val"], dtype), B, origin=c["origin"])
        assert strat == "2D"          # k = 2 <= 32 and m <= 15360 (spmm.jl:337-343)
        np.testing.assert_array_equal(C, np.array(c["C"], dtype), err_msg=c["name"])


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_reference_fixtures(dtype):
    for c in GOLDEN["sddmm"]:
        A = np.asfortranarray(np.array(c["A"], dtype))
        B = np.asfortranarray(np.array(c["B"], dtype))
        if c["format"] == "CSR":
            rp, ci = c["rowptr"], c["colind"]
        else:   # COO rows sorted: rowptr from counts
            cnt = np.bincount(np.array(c["rows"]) - 1, minlength=c["m"])
            rp, ci = np.r_[0, np.cumsum(cnt)] + 1, c["cols"]
        out = O.csr_sddmm(rp, ci, A, B, beta=c["beta"], C0=np.array(c["c0"], dtype))
        np.testing.assert_array_equal(out, np.array(c["cval"], dtype), err_msg=c["name"])


def test_to_dense_fixture():
    c = GOLDEN["to_dense"][0]
    pos, rows, cols, val = O.csr_to_coo(c["rowptr"], c["colind"], np.array(c["val"]),
                                        origin=c["origin"])
    D = np.zeros((c["m"], c["n"]))
    D[rows - 1, cols - 1] = val
    np.testing.assert_array_equal(D, np.array(c["dense"]))


def test_convert_fixtures():
    c = GOLDEN["convert"]
    val = np.array(c["val"], np.float32)
    colptr, rowind, cval = O.csr_to_csc(c["rowptr"], c["colind"], val, c["n"], origin=0)
    assert colptr.tolist() == c["csc_colptr"]
    assert rowind.tolist() == c["csc_rowind"]
    assert cval.tolist() == c["csc_val"]
    pos, rows, cols, v = O.csr_to_coo(c["rowptr"], c["colind"], val, origin=0)
    assert pos.tolist() == c["coo_pos"]
    assert rows.tolist() == c["coo_rows"] and cols.tolist() == c["coo_cols"]
    assert v.tolist() == c["coo_val"]
    # round trips CSR -> CSC -> CSR and CSR -> COO -> CSR (test_convert.jl:97-116)
    rp2, ci2, v2 = O.csr_to_csc(colptr, rowind, cval, c["m"], origin=0)
    assert rp2.tolist() == c["rowptr"] and ci2.tolist() == c["colind"]
    assert v2.tolist() == c["val"]
    rp3, ci3, v3 = O.coo_to_csr(rows, cols, v, c["m"], c["n"], origin=0)
    assert rp3.tolist() == c["rowptr"] and ci3.tolist() == c["colind"]
    # origin preserved (test_convert.jl:161-168)
    colptr1, rowind1, _ = O.csr_to_csc(c["onebased_rowptr"], c["onebased_colind"], val, c["n"],
                                       origin=1)
    assert colptr1.tolist() == [p + 1 for p in c["csc_colptr"]]
    assert rowind1.tolist() == [r + 1 for r in c["csc_rowind"]]


def test_convert_drops_explicit_zeros():
    """convert.jl:316: explicit zeros are dropped by every conversion."""
    colptr, rowind, cval = O.csr_to_csc([1, 3, 4], [1, 2, 2], np.array([0.0, 5.0, 6.0]), 2)
    assert colptr.tolist() == [1, 1, 3] and rowind.tolist() == [1, 2]
    assert cval.tolist() == [5.0, 6.0]


def test_bsr_layout_fixture():
    c = GOLDEN["bsr_layout"]
    val = np.array(c["val_row_major"], np.float64)
    assert val.size == c["nnz"]
    rp, ci, v = O.bsr_to_csr(c["browptr"], c["bcolind"], val, c["bs"])
    D = to_scipy(rp, ci, v, (c["m"], c["n"])).toarray()
    np.testing.assert_array_equal(D, np.array(c["dense"]))
    # column-major blocks (BSRLeft) of the same matrix expand to the same CSR
    blocks = val.reshape(-1, 2, 2)
    val_left = np.ascontiguousarray(blocks.transpose(0, 2, 1)).reshape(-1)
    rpl, cil, vl = O.bsr_to_csr(c["browptr"], c["bcolind"], val_left, c["bs"],
                                row_major_blocks=False)
    assert rpl.tolist() == rp.tolist() and cil.tolist() == ci.tolist()
    np.testing.assert_array_equal(vl, v)


# ------------------------------------------------------------ bit-exact scipy

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [0, 1])
def test_spmv_bitexact_scipy(dtype, origin):
    m, n = 4000, 3000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(0).integers(0, 90, m),
                                     seed=1, origin=origin, dtype=dtype)
    x = np.random.default_rng(2).uniform(-1, 1, n).astype(dtype)
    y = O.csr_spmv(rowptr, colind, val, x, origin=origin)
    ys = to_scipy(rowptr, colind, val, (m, n), origin) @ x
    assert ys.dtype == dtype
    np.testing.assert_array_equal(y, ys)


@pytest.mark.parametrize("k", [2, 40, 128])
def test_spmm_bitexact_scipy(k):
    m, n = 1500, 1200
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(k).integers(0, 40, m),
                                     seed=k)
    B = np.asfortranarray(np.random.default_rng(3).standard_normal((n, k)))
    C, _ = O.csr_spmm(rowptr, colind, val, B)
    Cs = to_scipy(rowptr, colind, val, (m, n)) @ B
    np.testing.assert_array_equal(C, Cs)


def test_spmm_column_equals_spmv():
    m, n, k = 800, 700, 48
    rowptr, colind, val = random_csr(m, n, density=0.03, seed=4)
    B = np.asfortranarray(np.random.default_rng(5).standard_normal((n, k)))
    C, strat = O.csr_spmm(rowptr, colind, val, B, 1.5, 0.0)
    assert strat == "Tiled"
    for c in (0, 17, 47):
        np.testing.assert_array_equal(C[:, c], O.csr_spmv(rowptr, colind, val, B[:, c], 1.5))


def test_sddmm_sequential_order_exact():
    """Every output is alpha*(sequential k sum) + beta*C (sddmm.jl:24-29)."""
    rng = np.random.default_rng(6)
    m, n, K = 30, 25, 7
    rowptr, colind, _ = random_csr(m, n, density=0.3, seed=7)
    A = np.asfortranarray(rng.standard_normal((m, K)))
    B = np.asfortranarray(rng.standard_normal((K, n)))
    C0 = rng.standard_normal(colind.size)
    out = O.csr_sddmm(rowptr, colind, A, B, 0.75, -2.0, C0)
    for i in range(m):
        for p in range(rowptr[i] - 1, rowptr[i + 1] - 1):
            j = colind[p] - 1
            dot = 0.0
            for kk in range(K):
                dot += A[i, kk] * B[kk, j]
            assert out[p] == 0.75 * dot + -2.0 * C0[p]


def test_sddmm_mask_form():
    rng = np.random.default_rng(8)
    m, n, K = 50, 40, 16
    rowptr, colind, _ = random_csr(m, n, density=0.2, seed=9, dtype=np.float32)
    A = np.asfortranarray(rng.standard_normal((m, K)).astype(np.float32))
    B = np.asfortranarray(rng.standard_normal((K, n)).astype(np.float32))
    S = rng.uniform(0.5, 1.5, colind.size).astype(np.float32)
    plain = O.csr_sddmm(rowptr, colind, A, B)
    np.testing.assert_array_equal(O.csr_sddmm(rowptr, colind, A, B, mask=S), S * plain)


# ---------------------------------------------------- brute force / closed forms

def test_spmv_brute_force_longdouble():
    rng = np.random.default_rng(10)
    m, n = 40, 30
    rowptr, colind, val = random_csr(m, n, density=0.4, seed=11)
    x = rng.uniform(-1, 1, n)
    D = to_scipy(rowptr, colind, val, (m, n)).toarray().astype(np.longdouble)
    exact = D @ x.astype(np.longdouble)
    y = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    assert np.all(np.abs(y - exact.astype(np.float64)) <= 64 * np.finfo(float).eps * absref)


def test_spmv_permutation_and_shifted_diagonal():
    n = 1000
    perm = np.random.default_rng(12).permutation(n)
    x = np.random.default_rng(13).standard_normal(n)
    rowptr = np.arange(n + 1, dtype=np.int32) + 1
    y = O.csr_spmv(rowptr, (perm + 1).astype(np.int32), np.ones(n), x)
    np.testing.assert_array_equal(y, x[perm])
    # ShiftedDiag(shift=3, val=2.5): y[r] = 2.5*x[r+3] (test_emitter_cuda.jl:326-341)
    m = n - 3
    y2 = O.csr_spmv(np.arange(m + 1, dtype=np.int32) + 1,
                    (np.arange(m) + 3 + 1).astype(np.int32), np.full(m, 2.5), x)
    np.testing.assert_array_equal(y2, 2.5 * x[3:])


def test_bsr_equals_dense_block_product():
    rng = np.random.default_rng(14)
    mb, nb, bs, k = 6, 5, 16, 20
    counts = rng.integers(0, 4, mb)
    bcol = [np.sort(rng.choice(nb, c, replace=False)) for c in counts]
    browptr = (np.r_[0, np.cumsum(counts)] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcol) + 1).astype(np.int32)
    val = rng.integers(-3, 4, bcolind.size * bs * bs).astype(np.float64)
    B = np.asfortranarray(rng.integers(-3, 4, (nb * bs, k)).astype(np.float64))
    D = np.zeros((mb * bs, nb * bs))
    for R in range(mb):
        for q in range(browptr[R] - 1, browptr[R + 1] - 1):
            c = bcolind[q] - 1
            D[R * bs:(R + 1) * bs, c * bs:(c + 1) * bs] = val[q * bs * bs:(q + 1) * bs * bs] \
                .reshape(bs, bs)
    np.testing.assert_array_equal(O.bsr_spmm(browptr, bcolind, val, bs, B), D @ B)


@pytest.mark.parametrize("b1,b2", [(2, 2), (4, 8), (3, 5), (1, 7)])
@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_rectangular_expansion_against_scipy(b1, b2, row_major):
    """Rectangular blocks, both block orders: the expansion keeps every stored
    entry (explicit zeros too) and equals scipy's bsr_matrix densely; the
    product equals the dense product exactly on small integers."""
    import scipy.sparse as sp
    rng = np.random.default_rng(40 + b1 * 10 + b2)
    mb, nb, k = 7, 6, 5
    counts = rng.integers(0, 4, mb)
    bcol = [np.sort(rng.choice(nb, c, replace=False)) for c in counts]
    indptr = np.r_[0, np.cumsum(counts)].astype(np.int32)
    indices = np.concatenate(bcol).astype(np.int32)
    blocks = rng.integers(-3, 4, (indices.size, b1, b2)).astype(np.float64)
    blocks[blocks == 3] = 0.0              # explicit zeros stay stored
    flat = blocks.reshape(-1) if row_major else blocks.transpose(0, 2, 1).reshape(-1)
    rp, ci, v = O.bsr_to_csr(indptr + 1, indices + 1, flat, b1, 1, row_major, b2)
    assert rp.size == mb * b1 + 1 and v.size == indices.size * b1 * b2
    ref = sp.bsr_matrix((blocks, indices, indptr), shape=(mb * b1, nb * b2)).toarray()
    got = sp.csr_matrix((v, ci - 1, rp - 1), shape=(mb * b1, nb * b2)).toarray()
    np.testing.assert_array_equal(got, ref)
    B = np.asfortranarray(rng.integers(-3, 4, (nb * b2, k)).astype(np.float64))
    np.testing.assert_array_equal(
        O.bsr_spmm(indptr + 1, indices + 1, flat, b1, B, row_major_blocks=row_major, b2=b2),
        ref @ B)


# -------------------------------------------------------- strategy semantics

def test_spmm_strategy_selection():
    """spmm.jl:329-349 with the CPU backend's 80-SM fallback."""
    assert O.spmm_strategy(100, 2, 300) == "2D"              # m <= 15360
    assert O.spmm_strategy(100_000, 16, 100_000) == "NNZFirst"
    assert O.spmm_strategy(100_000, 16, 400_000) == "2D"     # nnz > 3m
    assert O.spmm_strategy(100_000, 16, 10, True) == "2D"    # skip_empty_rows
    assert O.spmm_strategy(10, 128, 10) == "Tiled"
    assert O.spmm_strategy(10, 100, 10) == "ColFirst"


def test_spmm_tiled_reads_c_when_beta_zero():
    """Reference quirk (spmm.jl:273-276): the Tiled/ColFirst write reads C even
    when beta == 0, so NaN in C propagates; the 2-D path is write-only."""
    rowptr, colind, val = random_csr(20, 20, density=0.3, seed=15)
    for k, expect_nan in ((128, True), (2, False)):
        B = np.asfortranarray(np.ones((20, k)))
        C0 = np.asfortranarray(np.full((20, k), np.nan))
        C, _ = O.csr_spmm(rowptr, colind, val, B, 1.0, 0.0, C0)
        assert np.isnan(C).all() == expect_nan


def test_coo_matches_csr():
    m, n = 3000, 2000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(16).integers(0, 30, m),
                                     seed=17)
    x = np.random.default_rng(18).uniform(-1, 1, n)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    y_coo = O.coo_spmv(rows, colind, val, x, m)
    y_csr = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    assert np.all(np.abs(y_coo - y_csr) <= 1e-14 * absref)


# ----------------------------------------------------------- planted mistakes

def _pinned_by_scipy(spmv):
    """The scipy bit-exactness check, applied to any SpMV implementation."""
    n = 500
    rowptr, colind, val = random_csr(n, n, density=0.05, seed=19)
    x = np.random.default_rng(20).uniform(-1, 1, n)
    return np.array_equal(spmv(rowptr, colind, val, x), to_scipy(rowptr, colind, val, (n, n)) @ x)


def test_planted_mistakes_are_caught():
    assert _pinned_by_scipy(lambda rp, ci, v, x: O.csr_spmv(rp, ci, v, x))
    # origin off by one: reads x[col] instead of x[col-1]
    assert not _pinned_by_scipy(
        lambda rp, ci, v, x: O.csr_spmv(rp, ci, v, np.r_[x[1:], 0.0]))

    def dropped(rp, ci, v, x):          # last nonzero of every row ignored
        v2 = v.copy()
        nonempty = rp[1:] > rp[:-1]
        v2[(rp[1:] - 2)[nonempty]] = 0.0
        return O.csr_spmv(rp, ci, v2, x)
    assert not _pinned_by_scipy(dropped)

    def transposed(rp, ci, v, x):       # A^T x: the CSC arrays read as CSR
        cp, ri, cv = O.csr_to_csc(rp, ci, v, rp.size - 1)
        return O.csr_spmv(cp, ri, cv, x)
    assert not _pinned_by_scipy(transposed)
    # wrong sign on beta term is caught by the fixture with beta != 0
    c = GOLDEN["spmv"][0]
    y0 = np.ones(3)
    good = O.csr_spmv(c["rowptr"], c["colind"], np.array(c["val"]), np.array(c["x"]), 1.0, 2.0, y0)
    np.testing.assert_array_equal(good, np.array(c["y"]) + 2.0)
    bad = O.csr_spmv(c["rowptr"], c["colind"], np.array(c["val"]), np.array(c["x"]), 1.0, -2.0, y0)
    assert not np.array_equal(bad, np.array(c["y"]) + 2.0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_dcsr_fixtures_and_untouched_rows(dtype):
    """test_emitter.jl:127-157 and :230-260; rows not stored keep y0 / C0
    whatever beta is (the walker only visits stored rows)."""
    c = next(c for c in GOLDEN["spmv"] if c["format"] == "DCSR")
    y = O.dcsr_spmv(c["outer_crd"], c["inner_pos"], c["inner_crd"], np.array(c["val"], dtype),
                    np.array(c["x"], dtype), c["m"], origin=c["origin"])
    np.testing.assert_array_equal(y, np.array(c["y"], dtype))
    y0 = np.array([10.0, -3.0, 0.5], dtype)
    y = O.dcsr_spmv(c["outer_crd"], c["inner_pos"], c["inner_crd"], np.array(c["val"], dtype),
                    np.array(c["x"], dtype), c["m"], alpha=2.0, beta=0.5, y0=y0, origin=c["origin"])
    D = np.array([[1, 0, 2], [0, 0, 0], [4, 0, 5]], np.float64)
    want = 2.0 * D @ np.array(c["x"], np.float64) + 0.5 * y0
    want[1] = y0[1]                                      # absent row untouched, beta or not
    np.testing.assert_allclose(y, want, rtol=1e-6)
    s = next(c for c in GOLDEN["spmm"] if c["format"] == "DCSR")
    B = np.asfortranarray(np.array(s["B"], dtype))
    C = O.dcsr_spmm(s["outer_crd"], s["inner_pos"], s["inner_crd"], np.array(s["val"], dtype), B,
                    s["m"], origin=s["origin"])
    np.testing.assert_array_equal(C, np.array(s["C"], dtype))
    C0 = np.full((3, 2), 7.0, dtype)
    C = O.dcsr_spmm(s["outer_crd"], s["inner_pos"], s["inner_crd"], np.array(s["val"], dtype), B,
                    s["m"], beta=1.0, C0=C0, origin=s["origin"])
    assert C[1].tolist() == [7.0, 7.0]
    np.testing.assert_allclose(C[[0, 2]], np.array(s["C"], dtype)[[0, 2]] + 7.0, rtol=1e-6)


# ------------------------------------------------------- CSC SpMV (scatter)

def _csc_of(rowptr, colind, val, n, origin=1):
    """CSC arrays of a CSR matrix through the oracle's conversion (pinned by
    the test_convert.jl fixtures in test_convert_fixtures)."""
    return O.csr_to_csc(rowptr, colind, val, n, origin)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csc_spmv_reference_answer(dtype):
    """A = [1 0 2; 0 3 0; 4 0 5] stored column-major, x = [1, 2, 3] ->
    [7, 6, 19] (the matrix of test_emitter.jl:85-102 in Formats.CSC)."""
    c = GOLDEN["spmv"][0]
    cp, ri, cv = _csc_of(np.array(c["rowptr"]), np.array(c["colind"]), np.array(c["val"], dtype), 3)
    assert cp.tolist() == [1, 3, 4, 6] and ri.tolist() == [1, 3, 2, 1, 3]
    y = O.csc_spmv(cp, ri, cv, np.array(c["x"], dtype), 3)
    np.testing.assert_array_equal(y, np.array(c["y"], dtype))


@pytest.mark.parametrize("origin", [1, 0])
def test_csc_spmv_bitexact_scipy(origin):
    """scipy's csc_matvec adds val*x[col] into y[row] column by column in
    storage order from zero: with alpha = 1 the scatter is the same sum."""
    m, n = 700, 900
    rowptr, colind, val = random_csr(m, n, density=0.03, seed=41, origin=origin)
    cp, ri, cv = _csc_of(rowptr, colind, val, n, origin)
    x = np.random.default_rng(42).uniform(-1, 1, n)
    y = O.csc_spmv(cp, ri, cv, x, m, origin=origin)
    S = sp.csc_matrix((cv, ri - origin, cp - origin), shape=(m, n))
    np.testing.assert_array_equal(y, S @ x)
    # alpha = 2, beta = 0.5 scale every term by powers of two: exact.
    y0 = np.random.default_rng(43).uniform(-1, 1, m)
    y2 = O.csc_spmv(cp, ri, cv, x, m, alpha=2.0, beta=0.5, y0=y0, origin=origin)
    want = 0.5 * y0
    for j in range(n):
        for p in range(cp[j] - origin, cp[j + 1] - origin):
            want[ri[p] - origin] += (2.0 * cv[p]) * x[j]
    np.testing.assert_array_equal(y2, want)
    # planted mistakes: x reversed, and (square) the CSC arrays read as CSR,
    # i.e. A^T x, both fail the scipy check.
    assert not np.array_equal(O.csc_spmv(cp, ri, cv, x[::-1].copy(), m, origin=origin), y)
    rs, cs, vs = random_csr(400, 400, density=0.03, seed=46, origin=origin)
    cps, ris, cvs = _csc_of(rs, cs, vs, 400, origin)
    xs = np.random.default_rng(47).uniform(-1, 1, 400)
    want_s = sp.csc_matrix((cvs, ris - origin, cps - origin), shape=(400, 400)) @ xs
    np.testing.assert_array_equal(O.csc_spmv(cps, ris, cvs, xs, 400, origin=origin), want_s)
    assert not np.array_equal(O.csr_spmv(cps, ris, cvs, xs, origin=origin), want_s)


# ------------------------------------------------------------- COO SDDMM

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_coo_sddmm_reference_fixture(dtype):
    c = next(c for c in GOLDEN["sddmm"] if c["format"] == "COO")
    A = np.asfortranarray(np.array(c["A"], dtype))
    B = np.asfortranarray(np.array(c["B"], dtype))
    out = O.coo_sddmm(c["rows"], c["cols"], A, B, beta=c["beta"], C0=np.array(c["c0"], dtype),
                      origin=c["origin"])
    np.testing.assert_array_equal(out, np.array(c["cval"], dtype))


def test_coo_sddmm_equals_csr_and_permutes():
    """Row-ordered COO = the CSR result bit for bit (the same sequential dot
    per stored entry); shuffled entries give the shuffled outputs."""
    m, n, K = 400, 300, 24
    rowptr, colind, _ = random_csr(m, n, density=0.04, seed=44)
    rng = np.random.default_rng(45)
    A = np.asfortranarray(rng.standard_normal((m, K)))
    B = np.asfortranarray(rng.standard_normal((K, n)))
    mask = rng.uniform(0.5, 1.5, colind.size)
    C0 = rng.standard_normal(colind.size)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    csr = O.csr_sddmm(rowptr, colind, A, B, 1.5, -0.5, C0, mask)
    coo = O.coo_sddmm(rows, colind, A, B, 1.5, -0.5, C0, mask)
    np.testing.assert_array_equal(coo, csr)
    perm = rng.permutation(colind.size)
    shuf = O.coo_sddmm(rows[perm], colind[perm], A, B, 1.5, -0.5, C0[perm], mask[perm])
    np.testing.assert_array_equal(shuf, csr[perm])
    # planted mistakes: rows and columns swapped (a transposed mask read on a
    # square problem), and a wrong sign of beta, both differ.
    assert not np.array_equal(O.coo_sddmm(rows, colind, A, B, 1.5, 0.5, C0, mask), csr)
    rs, cs, _ = random_csr(200, 200, density=0.05, seed=48)
    rr = np.repeat(np.arange(1, 201, dtype=np.int32), np.diff(rs))
    As = np.asfortranarray(rng.standard_normal((200, K)))
    Bs = np.asfortranarray(rng.standard_normal((K, 200)))
    good = O.coo_sddmm(rr, cs, As, Bs)
    np.testing.assert_array_equal(good, O.csr_sddmm(rs, cs, As, Bs))
    assert not np.array_equal(O.coo_sddmm(cs, rr, As, Bs), good)
