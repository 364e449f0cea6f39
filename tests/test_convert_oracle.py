"""Pins of the conversion oracle (oracle/convert_oracle.py, a numpy restatement
of src/convert.jl:302-388) on the CPU: the reference's own expected arrays,
scipy on canonical inputs, and closed forms for the composer's rules (zero
drop, keep-first on unique levels, no merging on COO's non-unique level)."""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import convert_oracle as CO

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))


def csr_dict(rowptr, colind, val, m, n, origin):
    return dict(format="CSR", origin=origin, m=m, n=n, pos2=np.int32(rowptr),
                crd2=np.int32(colind), val=np.asarray(val))


def fixture(origin=0):
    c = GOLDEN["convert"]
    if origin == 0:
        return csr_dict(c["rowptr"], c["colind"], np.float32(c["val"]), c["m"], c["n"], 0)
    return csr_dict(c["onebased_rowptr"], c["onebased_colind"], np.float32(c["val"]), c["m"],
                    c["n"], 1)


def test_csr_to_csc_reference_arrays():
    """test/test_convert.jl:44-58."""
    c = GOLDEN["convert"]
    u = CO.convert_format(fixture(), "CSC")
    assert u["pos2"].tolist() == c["csc_colptr"]
    assert u["crd2"].tolist() == c["csc_rowind"]
    assert u["val"].tolist() == c["csc_val"]
    assert u["origin"] == 0


def test_csr_to_coo_reference_arrays():
    """test/test_convert.jl:62-79 (pos = [0, nnz])."""
    c = GOLDEN["convert"]
    u = CO.convert_format(fixture(), "COO")
    assert u["pos1"].tolist() == c["coo_pos"]
    assert u["crd1"].tolist() == c["coo_rows"]
    assert u["crd2"].tolist() == c["coo_cols"]
    assert u["val"].tolist() == c["coo_val"]


@pytest.mark.parametrize("mid", ["CSC", "COO", "DCSR", "CSR"])
@pytest.mark.parametrize("origin", [0, 1])
def test_round_trips_and_origin(mid, origin):
    """test/test_convert.jl:97-116, 155-168 (origin preserved)."""
    u = fixture(origin)
    w = CO.convert_format(CO.convert_format(u, mid), "CSR")
    assert w["origin"] == origin
    assert w["pos2"].tolist() == u["pos2"].tolist()
    assert w["crd2"].tolist() == u["crd2"].tolist()
    assert w["val"].tolist() == u["val"].tolist()


def test_dcsr_of_fixture():
    u = CO.convert_format(fixture(), "DCSR")
    assert u["pos1"].tolist() == [0, 3]
    assert u["crd1"].tolist() == [0, 1, 2]
    assert u["pos2"].tolist() == [0, 2, 3, 5]
    assert u["crd2"].tolist() == [0, 2, 1, 0, 2]


def test_csr_to_bsr_matches_reference_layout():
    """test/test_cuda.jl:85-97: the 4x4 matrix in 2x2 blocks, zero-filled."""
    g = GOLDEN["bsr_layout"]
    D = np.array(g["dense"])
    A = sp.csr_matrix(D)
    u = CO.convert_format(csr_dict(A.indptr + 1, A.indices + 1, A.data, 4, 4, 1), "BSR", 2, 2, True)
    assert u["pos2"].tolist() == g["browptr"]
    assert u["crd2"].tolist() == g["bcolind"]
    assert u["val"].tolist() == g["val_row_major"]


def test_to_dense_reference():
    """test/test_emitter.jl:311-327."""
    g = GOLDEN["to_dense"][0]
    u = csr_dict(g["rowptr"], g["colind"], np.float64(g["val"]), g["m"], g["n"], g["origin"])
    assert CO.to_dense(u).tolist() == g["dense"]


def random_canonical(m, n, density, seed, dtype=np.float64):
    rng = np.random.default_rng(seed)
    A = sp.random(m, n, density=density, format="csr", random_state=rng, dtype=dtype)
    A.data[A.data == 0] = 1.0
    A.sort_indices()
    return A


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_canonical_matches_scipy(seed):
    A = random_canonical(57, 43, 0.1, seed)
    u = csr_dict(A.indptr + 1, A.indices + 1, A.data, 57, 43, 1)
    C = A.tocsc()
    C.sort_indices()
    c = CO.convert_format(u, "CSC")
    assert np.array_equal(c["pos2"] - 1, C.indptr) and np.array_equal(c["crd2"] - 1, C.indices)
    assert np.array_equal(c["val"], C.data)
    o = CO.convert_format(u, "COO")
    Q = A.tocoo()
    assert np.array_equal(o["crd1"] - 1, Q.row) and np.array_equal(o["crd2"] - 1, Q.col)
    assert np.array_equal(o["val"], Q.data)


@pytest.mark.parametrize("bs", [(2, 2), (4, 2), (16, 16)])
def test_bsr_matches_scipy(bs):
    b1, b2 = bs
    A = random_canonical(b1 * 9, b2 * 7, 0.08, 5)
    u = csr_dict(A.indptr, A.indices, A.data, b1 * 9, b2 * 7, 0)
    B = A.tobsr(blocksize=bs)
    B.sort_indices()
    b = CO.convert_format(u, "BSR", b1, b2, True)
    assert np.array_equal(b["pos2"], B.indptr) and np.array_equal(b["crd2"], B.indices)
    assert np.array_equal(b["val"], B.data.reshape(-1))
    back = CO.convert_format(b, "CSR")
    assert np.array_equal(back["pos2"], A.indptr) and np.array_equal(back["crd2"], A.indices)
    assert np.array_equal(back["val"], A.data)
    # BSRLeft: column-major inside a block.
    l = CO.convert_format(u, "BSR", b1, b2, False)
    assert np.array_equal(l["val"], B.data.transpose(0, 2, 1).reshape(-1))


def test_explicit_zeros_dropped_nan_kept():
    u = csr_dict([0, 3, 5], [0, 1, 2, 0, 2], np.array([0.0, 1.0, -0.0, np.nan, 2.0]), 2, 3, 0)
    w = CO.convert_format(u, "CSC")
    assert w["crd2"].tolist() == [1, 0, 1]
    v = w["val"]
    assert np.isnan(v[0]) and v[1:].tolist() == [1.0, 2.0]
    assert w["pos2"].tolist() == [0, 1, 2, 3]


def test_duplicates_keep_first_on_unique_levels():
    """convert.jl:232-250: adjacent equal coordinates form one segment whose
    first value is appended.  Summing or keeping the last fails here."""
    coo = dict(format="COO", origin=0, m=2, n=3, crd1=np.int32([0, 0, 0, 1, 1]),
               crd2=np.int32([1, 1, 2, 0, 0]), val=np.array([10.0, 20.0, 30.0, 40.0, 50.0]))
    w = CO.convert_format(coo, "CSR")
    assert w["pos2"].tolist() == [0, 2, 3]
    assert w["crd2"].tolist() == [1, 2, 0]
    assert w["val"].tolist() == [10.0, 30.0, 40.0]
    # COO's first level is non-unique: no merging.
    assert CO.convert_format(coo, "COO")["val"].tolist() == [10.0, 20.0, 30.0, 40.0, 50.0]
    # CSC sorts first (stable), then keeps the first of each (col, row).
    c = CO.convert_format(coo, "CSC")
    assert c["crd2"].tolist() == [1, 0, 0] and c["val"].tolist() == [40.0, 10.0, 30.0]


def test_unsorted_rows_assert_for_csr_target():
    """The Dense row level asserts non-decreasing rows (convert.jl:254); COO and
    DCSR targets keep the order."""
    coo = dict(format="COO", origin=0, m=3, n=3, crd1=np.int32([2, 0, 1]),
               crd2=np.int32([0, 1, 2]), val=np.array([1.0, 2.0, 3.0]))
    with pytest.raises(AssertionError):
        CO.convert_format(coo, "CSR")
    assert CO.convert_format(coo, "COO")["crd1"].tolist() == [2, 0, 1]
    d = CO.convert_format(coo, "DCSR")
    assert d["crd1"].tolist() == [2, 0, 1] and d["pos2"].tolist() == [0, 1, 2, 3]
    # CSC sorts: rows order is irrelevant there.
    assert CO.convert_format(coo, "CSC")["crd2"].tolist() == [2, 0, 1]


def test_dense_equivalence_random():
    rng = np.random.default_rng(9)
    A = random_canonical(33, 41, 0.2, 3)
    A.data[rng.random(A.data.size) < 0.2] = 0.0      # explicit zeros stay stored
    u = csr_dict(A.indptr, A.indices, A.data, 33, 41, 0)
    D = A.toarray()
    for fmt, extra in (("CSC", ()), ("COO", ()), ("DCSR", ()), ("BSR", (3, 1, True)),
                       ("BSR", (11, 41, False))):
        w = CO.convert_format(u, fmt, *extra)
        assert np.array_equal(CO.to_dense(w), D), fmt
        if fmt != "BSR":                     # BSR blocks are zero-filled
            assert (np.asarray(w["val"]) != 0).all(), fmt
