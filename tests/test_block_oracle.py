"""Pins of the block-aggregate oracle (oracle/block_oracle.py) on the CPU: the
reference's known answers (test/test_emitter_cuda.jl:297-408), scipy's bmat
for the assembled CSR of canonical blocks, the block layout drawn in
src/block_banded.jl:5-14 written out by hand, and closed forms of the period
starts."""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import block_oracle as BO

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))


def csr_block(rowptr, colind, val, m, n, origin):
    return dict(format="CSR", origin=origin, m=m, n=n, pos2=np.int32(rowptr),
                crd2=np.int32(colind), val=np.asarray(val, np.float64))


def fixture_blocks():
    g = GOLDEN["block_sparse"]
    return {k: csr_block(g[k]["rowptr"], g[k]["colind"], g[k]["val"], g[k]["m"], g[k]["n"], 1)
            for k in ("A1", "A2")}


@pytest.mark.parametrize("case", ["diagonal", "accumulate"])
def test_bsm_reference_answers(case):
    g = GOLDEN["block_sparse"][case]
    blk = fixture_blocks()
    grid = [[None if b is None else blk[b] for b in row] for row in g["grid"]]
    A = BO.BSM(grid)
    assert list(A.shape) == g["size"]
    x = np.array(g["x"])
    assert A.matvec(x).tolist() == g["y"]
    rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
    assert BO.csr_matvec(rowptr, colind, val, x).tolist() == g["y"]


def random_canonical(m, n, density, seed):
    rng = np.random.default_rng(seed)
    A = sp.random(m, n, density=density, format="csr", random_state=rng)
    A.data[A.data == 0] = 1.0
    A.sort_indices()
    return A


def as_block(A, origin):
    return csr_block(A.indptr + origin, A.indices + origin, A.data, A.shape[0], A.shape[1], origin)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_assemble_matches_bmat(seed):
    """Canonical blocks in block-column order give scipy's canonical CSR of
    the block matrix, array for array."""
    rng = np.random.default_rng(seed)
    rs, cs = [5, 9, 3], [7, 4, 6, 2]
    S = [[None if rng.random() < 0.35 and not (i == j or (i, j) == (0, 3)) else
          random_canonical(rs[i], cs[j], 0.3, 10 * seed + 4 * i + j) for j in range(4)]
         for i in range(3)]
    grid = [[None if S[i][j] is None else as_block(S[i][j], (i + j) % 2) for j in range(4)]
            for i in range(3)]
    A = BO.BSM(grid)
    rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
    B = sp.bmat(S, format="csr")
    B.sort_indices()
    assert np.array_equal(rowptr, B.indptr) and np.array_equal(colind, B.indices)
    assert np.array_equal(val, B.data)
    assert np.array_equal(A.dense(), B.toarray())


def test_assemble_keeps_storage_order_and_zeros():
    """Unsorted columns, explicit zeros and empty rows stay as stored: the
    assembly copies rows, it does not canonicalise them."""
    a = csr_block([0, 3, 3, 4], [2, 0, 1, 1], [1.0, 0.0, 3.0, 4.0], 3, 3, 0)
    b = csr_block([0, 1, 1, 2], [1, 0], [5.0, 6.0], 3, 2, 0)
    A = BO.BSM([[a, b]])
    rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
    assert rowptr.tolist() == [0, 4, 4, 6]
    assert colind.tolist() == [2, 0, 1, 4, 1, 3]
    assert val.tolist() == [1.0, 0.0, 3.0, 5.0, 4.0, 6.0]


def test_shifted_diag_entries():
    d = dict(format="ShiftedDiag", m=4, n=6, shift=2, val=-1.5)
    assert BO.dense(d).tolist() == (-1.5 * np.eye(4, 6, k=2)).tolist()
    d = dict(format="ShiftedDiag", m=5, n=3, shift=-1, val=2.0)
    r, c, v = BO.entries(d)
    assert r.tolist() == [1, 2, 3] and c.tolist() == [0, 1, 2] and v.tolist() == [2.0] * 3


def test_multiple_shifted_closed_form():
    """test_emitter_cuda.jl:367-379: [3I  -I  2I] x = 3x1 - x2 + 2x3."""
    n = GOLDEN["shifted_diag"]["multiple"]["n"]
    I3 = csr_block(np.arange(n + 1), np.arange(n), np.full(n, 3.0), n, n, 0)
    A = BO.BSM([[I3, dict(format="ShiftedDiag", m=n, n=n, shift=0, val=-1.0),
                 dict(format="ShiftedDiag", m=n, n=n, shift=0, val=2.0)]])
    x = np.random.default_rng(0).random(3 * n)
    want = 3 * x[:n] - x[n:2 * n] + 2 * x[2 * n:]
    assert np.allclose(A.matvec(x), want, rtol=0, atol=1e-15)
    rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
    assert np.allclose(BO.csr_matvec(rowptr, colind, val, x), want, rtol=0, atol=1e-15)


def test_diag_starts_closed_forms():
    # bw = 1: every period is n_diag + n_off rows apart.
    assert BO.diag_starts(5, [3], 4) == [0, 8, 16, 24]
    # bw = 2, T = 3 (the diagram in block_banded.jl:5-14): D1 C1 C2 | D2 C1 | D3.
    assert BO.diag_starts(5, [3, 2], 3) == [0, 10, 18]
    # bw = 0: diagonal blocks only.
    assert BO.diag_starts(4, [], 3) == [0, 4, 8]


def test_bbm_layout_by_hand():
    """T = 3, bw = 2 laid out from the diagram, block by block."""
    rng = np.random.default_rng(4)
    nd, n1, n2, nc = 3, 2, 1, 4

    def blk(m, seed):
        return as_block(random_canonical(m, nc, 0.6, seed), 0)
    D, N1, P1, N2, P2 = blk(nd, 1), blk(n1, 2), blk(n1, 3), blk(n2, 4), blk(n2, 5)
    M = BO.BBM(D, [(N1, P1), (N2, P2)], 3, nd, [n1, n2], nc)
    assert M.shape == (3 * nd + 2 * n1 + n2, 3 * nc)
    d = BO.dense
    Z = lambda m: np.zeros((m, nc))  # noqa: E731
    full = np.block([
        [d(D), Z(nd), Z(nd)],
        [d(N1), d(P1), Z(n1)],
        [d(N2), Z(n2), d(P2)],
        [Z(nd), d(D), Z(nd)],
        [Z(n1), d(N1), d(P1)],
        [Z(nd), Z(nd), d(D)],
    ])
    x = rng.random(3 * nc)
    assert np.allclose(M.matvec(x), full @ x, rtol=0, atol=1e-14)
    rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
    A = sp.csr_matrix((val, colind, rowptr), shape=M.shape).toarray()
    assert np.array_equal(A, full)


def test_bbm_time_varying_and_per_transition():
    rng = np.random.default_rng(5)
    T, nd, no, nc = 4, 3, 2, 5
    Ds = [as_block(random_canonical(nd, nc, 0.5, 10 + t), 1) for t in range(T)]
    pairs = [(as_block(random_canonical(no, nc, 0.5, 20 + t), 0),
              as_block(random_canonical(no, nc, 0.5, 30 + t), 1)) for t in range(T - 1)]
    M = BO.BBM(Ds, [pairs], T, nd, [no], nc)
    full = np.zeros(M.shape)
    s = BO.diag_starts(nd, [no], T)
    for t in range(T):
        full[s[t]:s[t] + nd, t * nc:(t + 1) * nc] = BO.dense(Ds[t])
        if t < T - 1:
            full[s[t] + nd:s[t] + nd + no, t * nc:(t + 1) * nc] = BO.dense(pairs[t][0])
            full[s[t] + nd:s[t] + nd + no, (t + 1) * nc:(t + 2) * nc] = BO.dense(pairs[t][1])
    x = rng.random(T * nc)
    assert np.allclose(M.matvec(x), full @ x, rtol=0, atol=1e-14)
    rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
    assert np.array_equal(sp.csr_matrix((val, colind, rowptr), shape=M.shape).toarray(), full)


def test_bsm_matmat_is_columnwise_matvec():
    blk = fixture_blocks()
    A = BO.BSM([[blk["A1"], blk["A2"]], [blk["A2"], None]])
    X = np.random.default_rng(1).random((6, 3))
    Y = A.matmat(X)
    for k in range(3):
        assert np.allclose(Y[:, k], A.matvec(X[:, k]), rtol=0, atol=1e-15)
