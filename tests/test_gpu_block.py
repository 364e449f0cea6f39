"""BlockSparseMatrix, BlockBandedMatrix and ShiftedDiag on the GPU against the
numpy restatement (oracle/block_oracle.py): the reference's known answers
(test/test_emitter_cuda.jl:297-408), the assembled CSR array for array,
products within the parity tolerance for f64/f32, value updates, and the
per-block fallback for blocks the assembly does not take."""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

from tests._util import assert_within, dev, host

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


@pytest.fixture(scope="module")
def BO():
    from oracle import block_oracle
    return block_oracle


def to_ust(J, d):
    """oracle block dict -> device USTensor."""
    import torch
    if d["format"] == "ShiftedDiag":
        dt = torch.float32 if d.get("dtype") == np.float32 else torch.float64
        return J.shifted_diag_tensor(dt, d["m"], d["n"], shift=d["shift"], val=d["val"])
    o = J.OneBased() if d["origin"] == 1 else J.ZeroBased()
    f, m, n = d["format"], d["m"], d["n"]
    if f == "CSR":
        return J.csr_tensor(dev(d["pos2"]), dev(d["crd2"]), dev(d["val"]), (m, n), origin=o)
    if f == "DCSR":
        return J.dcsr_tensor(dev(d["crd1"]), dev(d["pos2"]), dev(d["crd2"]), dev(d["val"]), (m, n),
                             origin=o)
    if f == "COO":
        return J.coo_tensor(dev(d["crd1"]), dev(d["crd2"]), dev(d["val"]), (m, n), origin=o)
    raise ValueError(f)


def csr_block(rowptr, colind, val, m, n, origin, dtype=np.float64):
    return dict(format="CSR", origin=origin, m=m, n=n, pos2=np.int32(rowptr),
                crd2=np.int32(colind), val=np.asarray(val, dtype))


def random_block(m, n, density, seed, origin=0, dtype=np.float64, fmt="CSR", zeros=0.0,
                 shuffle=False):
    rng = np.random.default_rng(seed)
    A = sp.random(m, n, density=density, format="csr", random_state=rng, dtype=np.float64)
    A.sort_indices()
    val = rng.uniform(-1, 1, A.nnz).astype(dtype)
    val[rng.random(A.nnz) < zeros] = 0.0                  # explicit zeros stay stored
    cols = A.indices.copy()
    if shuffle:                                            # unsorted columns inside rows
        for r in range(m):
            s, e = A.indptr[r], A.indptr[r + 1]
            p = rng.permutation(e - s)
            cols[s:e], val[s:e] = cols[s:e][p], val[s:e][p]
    if fmt == "CSR":
        return csr_block(A.indptr + origin, cols + origin, val, m, n, origin, dtype)
    if fmt == "DCSR":
        lens = np.diff(A.indptr)
        rows = np.flatnonzero(lens)
        pos = np.concatenate([[0], np.cumsum(lens[rows])])
        return dict(format="DCSR", origin=origin, m=m, n=n, crd1=np.int32(rows + origin),
                    pos2=np.int32(pos + origin), crd2=np.int32(cols + origin), val=val)
    if fmt == "COO":
        rows = np.repeat(np.arange(m), np.diff(A.indptr))
        return dict(format="COO", origin=origin, m=m, n=n, crd1=np.int32(rows + origin),
                    crd2=np.int32(cols + origin), val=val)
    raise ValueError(fmt)


def abs_bound(D, x):
    return np.abs(D) @ np.abs(x)


# ------------------------------------------------------- reference answers

@pytest.mark.parametrize("case", ["diagonal", "accumulate"])
def test_bsm_reference_answers(J, case):
    """test_emitter_cuda.jl:297-325."""
    import torch
    g = GOLDEN["block_sparse"]
    blk = {k: J.csr_tensor(dev(np.int32(g[k]["rowptr"])), dev(np.int32(g[k]["colind"])),
                           dev(np.float64(g[k]["val"])), (g[k]["m"], g[k]["n"]))
           for k in ("A1", "A2")}
    c = g[case]
    BM = J.BlockSparseMatrix([[None if b is None else blk[b] for b in row] for row in c["grid"]])
    assert list(BM.size()) == c["size"]
    x = dev(np.float64(c["x"]))
    assert host(J.matmul(BM, x)).tolist() == c["y"]
    y = torch.zeros(len(c["y"]), dtype=torch.float64, device="cuda")
    J.mul_(y, BM, x)
    assert host(y).tolist() == c["y"]
    y.zero_()
    J.execute(J.BlockSpMVOp, BM, x, y)
    assert host(y).tolist() == c["y"]


@pytest.mark.parametrize("case", range(2))
def test_shifted_diag_standalone(J, case):
    """test_emitter_cuda.jl:329-343: y = val * x[shift:]."""
    import torch
    c = GOLDEN["shifted_diag"]["standalone"][case]
    u = J.shifted_diag_tensor(torch.float64, c["m"], c["n"], shift=c["shift"], val=c["val"])
    assert J.nnz(u) == 0 and J.size(u) == (c["m"], c["n"])
    xs = np.random.default_rng(case).random(c["n"])
    y = torch.zeros(c["m"], dtype=torch.float64, device="cuda")
    J.mul_(y, u, dev(xs))
    assert np.array_equal(host(y), c["val"] * xs[c["shift"]:c["shift"] + c["m"]])
    y2 = torch.ones(c["m"], dtype=torch.float64, device="cuda")
    J.mul_(y2, u, dev(xs), 2.0, 0.5)
    assert np.array_equal(host(y2), 2.0 * (c["val"] * xs[c["shift"]:c["shift"] + c["m"]]) + 0.5)


def test_bsm_shifted_block_equals_csr_block(J):
    """test_emitter_cuda.jl:345-363: a CSR -I block and ShiftedDiag(-1) agree."""
    import torch
    n = 16
    rp, cv = dev(np.arange(1, n + 2, dtype=np.int32)), dev(np.arange(1, n + 1, dtype=np.int32))
    A = J.csr_tensor(rp, cv, dev(np.full(n, 2.0)), (n, n))
    negI = J.csr_tensor(rp, cv, dev(np.full(n, -1.0)), (n, n))
    negS = J.shifted_diag_tensor(torch.float64, n, n, shift=0, val=-1.0)
    x = dev(np.random.default_rng(0).random(2 * n))
    y1 = J.matmul(J.BlockSparseMatrix([[A, negI]]), x)
    y2 = J.matmul(J.BlockSparseMatrix([[A, negS]]), x)
    assert np.array_equal(host(y1), host(y2))


def test_bsm_multiple_shifted(J):
    """test_emitter_cuda.jl:365-380: [3I  -I  2I] x = 3 x1 - x2 + 2 x3."""
    import torch
    n = GOLDEN["shifted_diag"]["multiple"]["n"]
    rp, cv = dev(np.arange(1, n + 2, dtype=np.int32)), dev(np.arange(1, n + 1, dtype=np.int32))
    A = J.csr_tensor(rp, cv, dev(np.full(n, 3.0)), (n, n))
    BM = J.BlockSparseMatrix([[A, J.shifted_diag_tensor(torch.float64, n, n, val=-1.0),
                               J.shifted_diag_tensor(torch.float64, n, n, val=2.0)]])
    xs = np.random.default_rng(1).random(3 * n)
    want = 3 * xs[:n] - xs[n:2 * n] + 2 * xs[2 * n:]
    assert_within(host(J.matmul(BM, dev(xs))), want, 6 * np.abs(xs[:n]) + 3, np.float64)


def test_bbm_shifted_equals_csr(J):
    """test_emitter_cuda.jl:382-408: the BBM over [A  -I] with a (-R, R)
    coupling is the same whether -I is CSR or ShiftedDiag."""
    import torch
    g = GOLDEN["shifted_diag"]["bbm"]
    n, T = g["n"], g["T"]
    rp, cv = dev(np.arange(1, n + 2, dtype=np.int32)), dev(np.arange(1, n + 1, dtype=np.int32))
    A = J.csr_tensor(rp, cv, dev(np.full(n, 3.0)), (n, n))
    negI = J.csr_tensor(rp, cv, dev(np.full(n, -1.0)), (n, n))
    negS = J.shifted_diag_tensor(torch.float64, n, n, val=-1.0)
    R = J.csr_tensor(rp, cv, dev(np.full(n, 1.0)), (n, 2 * n))
    negR = J.csr_tensor(rp, cv, dev(np.full(n, -1.0)), (n, 2 * n))
    B1 = J.BlockBandedMatrix(J.BlockSparseMatrix([[A, negI]]), negR, R, T, n, n, 2 * n)
    B2 = J.BlockBandedMatrix(J.BlockSparseMatrix([[A, negS]]), negR, R, T, n, n, 2 * n)
    assert B1.size() == (g["rows"], g["cols"])
    x = dev(np.random.default_rng(2).random(T * 2 * n))
    y1 = torch.zeros(g["rows"], dtype=torch.float64, device="cuda")
    y2 = torch.zeros_like(y1)
    J.mul_(y1, B1, x)
    J.execute(J.BBMSpMVOp, B2, x, y2)
    assert np.array_equal(host(y1), host(y2))


# ------------------------------------------------------ assembly, products

def mixed_grid(seed, dtype=np.float64):
    """3 x 4 grid: CSR (both origins, unsorted columns, explicit zeros, empty
    rows), DCSR and shifted diagonals."""
    rs, cs = [40, 7, 25], [30, 25, 9, 40]
    g = [[None] * 4 for _ in range(3)]
    g[0][0] = random_block(40, 30, 0.2, seed, 1, dtype, "CSR", zeros=0.1)
    g[0][3] = random_block(40, 40, 0.05, seed + 1, 0, dtype, "DCSR")
    g[1][1] = random_block(7, 25, 0.3, seed + 2, 0, dtype, "CSR", shuffle=True)
    g[1][2] = dict(format="ShiftedDiag", m=7, n=9, shift=2, val=-1.5, dtype=dtype)
    g[2][1] = dict(format="ShiftedDiag", m=25, n=25, shift=0, val=2.0, dtype=dtype)
    g[2][2] = random_block(25, 9, 0.0, seed + 3, 1, dtype, "CSR")          # no entries at all
    g[2][3] = random_block(25, 40, 0.15, seed + 4, 1, dtype, "DCSR", shuffle=True)
    assert [next(b["m"] for b in r if b) for r in g] == rs
    return g


def device_bsm(J, grid):
    return J.BlockSparseMatrix([[None if b is None else to_ust(J, b) for b in row] for row in grid])


@pytest.mark.parametrize("seed", [0, 7])
def test_assembled_csr_bit_exact(J, BO, seed):
    grid = mixed_grid(seed)
    A = BO.BSM(grid)
    rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
    BM = device_bsm(J, grid)
    asm = BM.assembled().asm
    assert host(J.positions(asm, 2)).tolist() == rowptr.tolist()
    assert host(J.coordinates(asm, 2)).tolist() == colind.tolist()
    assert np.array_equal(host(J.nonzeros(asm)), val)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_bsm_spmv_spmm_batch(J, BO, dtype):
    grid = mixed_grid(3, dtype)
    A = BO.BSM(grid)
    D = A.dense().astype(np.float64)
    BM = device_bsm(J, grid)
    rng = np.random.default_rng(11)
    xs = rng.uniform(-1, 1, A.shape[1]).astype(dtype)
    assert_within(host(J.matmul(BM, dev(xs))), A.matvec(xs.astype(np.float64)), abs_bound(D, xs),
                  dtype, "BlockSpMV")
    X = rng.uniform(-1, 1, (A.shape[1], 5)).astype(dtype)
    ref = A.matmat(X.astype(np.float64))
    bound = np.abs(D) @ np.abs(X.astype(np.float64))
    assert_within(host(J.matmul(BM, dev(X))), ref, bound, dtype, "BlockSpMM")
    assert_within(host(J.batch_mul(BM, dev(X))), ref, bound, dtype, "batch_mul")
    # five-argument mul!: y = 2 A x - 0.5 y
    y0 = rng.uniform(-1, 1, A.shape[0]).astype(dtype)
    y = dev(y0)
    J.mul_(y, BM, dev(xs), 2.0, -0.5)
    assert_within(host(y), 2 * A.matvec(xs.astype(np.float64)) - 0.5 * y0,
                  2 * abs_bound(D, xs) + 0.5 * np.abs(y0), dtype, "mul! alpha beta")


def test_update_block_values(J, BO):
    import torch
    grid = mixed_grid(5)
    BM = device_bsm(J, grid)
    rng = np.random.default_rng(6)
    xs = rng.uniform(-1, 1, BM.size(2))
    J.matmul(BM, dev(xs))                           # assemble and plan first
    for step in range(2):
        for (i, j) in ((1, 1), (3, 4)):
            b = grid[i - 1][j - 1]
            b["val"] = rng.uniform(-1, 1, b["val"].size)
            J.update_block_values_(BM, i, j, dev(b["val"]))
            assert np.array_equal(host(J.nonzeros(BM.blocks[i - 1][j - 1])), b["val"])
        A = BO.BSM(grid)
        assert_within(host(J.matmul(BM, dev(xs))), A.matvec(xs), abs_bound(A.dense(), xs),
                      np.float64, f"after update {step}")
        rowptr, colind, val = BO.assemble(*A.shape, list(A.placements()))
        assert np.array_equal(host(J.nonzeros(BM.assembled().asm)), val)
    with pytest.raises(J.BlockStructureError):
        J.update_block_values_(BM, 1, 2, dev(np.zeros(3)))         # a None block
    with pytest.raises(J.BlockStructureError):
        J.update_block_values_(BM, 1, 1, dev(np.zeros(3)))         # wrong length
    with pytest.raises(J.UnsupportedValueType):
        J.update_block_values_(BM, 1, 1, torch.zeros(J.nnz(BM.blocks[0][0]), dtype=torch.float32,
                                                       device="cuda"))


def test_bsm_fallback_per_block(J, BO):
    """A COO block is not assembled: block-by-block products
    (block_sparse.jl:259-302)."""
    grid = [[random_block(20, 15, 0.3, 1, 1, fmt="COO"), random_block(20, 10, 0.3, 2, 0)],
            [None, random_block(9, 10, 0.4, 3, 1)]]
    A = BO.BSM(grid)
    BM = device_bsm(J, grid)
    assert not BM.assemblable()
    xs = np.random.default_rng(2).uniform(-1, 1, A.shape[1])
    assert_within(host(J.matmul(BM, dev(xs))), A.matvec(xs), abs_bound(A.dense(), xs),
                  np.float64, "fallback spmv")
    with pytest.raises(J.UnsupportedFormat):
        BM.assembled()


def test_assembly_rejects_bad_storage(J):
    bad_ptr = csr_block([0, 2, 5], [0, 1, 0, 1], [1.0, 2.0, 3.0, 4.0], 2, 2, 0)
    with pytest.raises(J.NonCanonicalStorage):
        device_bsm(J, [[bad_ptr]]).assembled()
    dec = csr_block([0, 3, 2, 4], [0, 1, 0, 1], [1.0, 2.0, 3.0, 4.0], 3, 2, 0)
    with pytest.raises(J.NonCanonicalStorage):
        device_bsm(J, [[dec]]).assembled()
    dcsr = dict(format="DCSR", origin=0, m=3, n=2, crd1=np.int32([2, 1]), pos2=np.int32([0, 1, 2]),
                crd2=np.int32([0, 1]), val=np.array([1.0, 2.0]))
    with pytest.raises(J.NonCanonicalStorage):
        device_bsm(J, [[dcsr]]).assembled()
    col = csr_block([0, 1, 2], [0, 5], [1.0, 2.0], 2, 2, 0)
    with pytest.raises(J.NonCanonicalStorage):
        device_bsm(J, [[col]]).assembled()


# -------------------------------------------------------------- block banded

def dcopf_like(n_bus, n_line, n_gen, seed, dtype=np.float64):
    """Synthetic blocks of the DCOPF constraint operator in the reference's
    benchmark (benchmark/sweep_cases.jl:103-166): [Cg 0 -Bbus; 0 -I Bf]."""
    rng = np.random.default_rng(seed)
    f = rng.integers(0, n_bus, n_line)
    t = (f + 1 + rng.integers(0, n_bus - 1, n_line)) % n_bus
    b = rng.uniform(1, 10, n_line)
    Bf = sp.csr_matrix((np.r_[b, -b], (np.r_[np.arange(n_line), np.arange(n_line)], np.r_[f, t])),
                       shape=(n_line, n_bus))
    Bbus = (Bf.T @ sp.csr_matrix((np.ones(2 * n_line), (np.r_[np.arange(n_line), np.arange(n_line)],
                                                        np.r_[f, t])), shape=(n_line, n_bus))).tocsr()
    Cg = sp.csr_matrix((np.ones(n_gen), (rng.integers(0, n_bus, n_gen), np.arange(n_gen))),
                       shape=(n_bus, n_gen))
    out = []
    for M in (Cg, -Bbus, Bf):
        M = M.tocsr()
        M.sum_duplicates()
        M.sort_indices()
        out.append(csr_block(M.indptr + 1, M.indices + 1, M.data.astype(dtype), *M.shape, 1, dtype))
    return out


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_bbm_dcopf_bw1(J, BO, dtype):
    import torch
    n_bus, n_line, n_gen, T = 60, 90, 15, 6
    Cg, negB, Bf = dcopf_like(n_bus, n_line, n_gen, 0, dtype)
    negI = dict(format="ShiftedDiag", m=n_line, n=n_line, shift=0, val=-1.0, dtype=dtype)
    grid = [[Cg, None, negB], [None, negI, Bf]]
    n_var, n_con = n_gen + n_line + n_bus, n_bus + n_line
    R = csr_block(np.arange(n_gen + 1), np.arange(n_gen), np.ones(n_gen), n_gen, n_var, 0, dtype)
    negR = csr_block(np.arange(n_gen + 1), np.arange(n_gen), -np.ones(n_gen), n_gen, n_var, 0, dtype)
    A = BO.BSM(grid)
    M = BO.BBM(A, [(negR, R)], T, n_con, [n_gen], n_var)
    BM = device_bsm(J, grid)
    MM = J.BlockBandedMatrix(BM, to_ust(J, negR), to_ust(J, R), T, n_con, n_gen, n_var)
    assert MM.size() == M.shape
    xs = np.random.default_rng(3).uniform(-1, 1, M.shape[1]).astype(dtype)
    y = torch.empty(M.shape[0], dtype=MM.dtype, device="cuda")
    J.mul_(y, MM, dev(xs))
    rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
    D = sp.csr_matrix((val.astype(np.float64), colind, rowptr), shape=M.shape)
    assert_within(host(y), M.matvec(xs.astype(np.float64)), abs(D) @ np.abs(xs.astype(np.float64)),
                  dtype, "BBM bw=1")
    asm = MM.assembled().asm
    assert host(J.positions(asm, 2)).tolist() == rowptr.tolist()
    assert host(J.coordinates(asm, 2)).tolist() == colind.tolist()
    assert np.array_equal(host(J.nonzeros(asm)), val)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("T", [1, 2, 7])
def test_bbm_periodic(J, BO, monkeypatch, dtype, T):
    """The periodic kernel (block_periodic.jl:108-236, periodic view
    block_mul.jl:584-676): one BlockSparseMatrix diagonal (CSR of both
    origins, DCSR, ShiftedDiag blocks) shared by every period, coupling pairs
    of CSR (both origins) and ShiftedDiag blocks (shifts 0, 3, -2), against
    the oracle's BBM product and the assembled-CSR path, with alpha and beta,
    and after update_block_values! of the diagonal."""
    import torch
    from jlust_amd import block_banded as bb
    monkeypatch.setattr(bb, "USE_PERIODIC", True)
    grid = mixed_grid(4, dtype)
    nd, nc, no = 72, 104, 5
    sd = lambda shift, val: dict(format="ShiftedDiag", m=no, n=nc, shift=shift, val=val, dtype=dtype)
    cases = [(random_block(no, nc, 0.2, 31, 0, dtype), random_block(no, nc, 0.2, 32, 1, dtype)),
             (sd(3, -1.0), random_block(no, nc, 0.3, 33, 1, dtype, shuffle=True)),
             (sd(0, -1.0), sd(-2, 2.5))]
    rng = np.random.default_rng(34)
    for ci, (neg, pos) in enumerate(cases):
        BM = device_bsm(J, grid)
        MM = J.BlockBandedMatrix(BM, to_ust(J, neg), to_ust(J, pos), T, nd, no, nc)
        assert MM.periodic() is not None
        for step in range(2):
            if step == 1:
                b = grid[0][0]
                b["val"] = rng.uniform(-1, 1, b["val"].size).astype(dtype)
                J.update_block_values_(BM, 1, 1, dev(b["val"]))
            M = BO.BBM(BO.BSM(grid), [(neg, pos)], T, nd, [no], nc)
            assert MM.size() == M.shape
            rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
            D = abs(sp.csr_matrix((val.astype(np.float64), colind, rowptr), shape=M.shape))
            xs = rng.uniform(-1, 1, M.shape[1]).astype(dtype)
            y0 = rng.uniform(-1, 1, M.shape[0]).astype(dtype)
            x64, y64 = xs.astype(np.float64), y0.astype(np.float64)
            y = dev(y0)
            J.mul_(y, MM, dev(xs), 1.5, -0.5)
            what = f"case {ci} step {step}"
            assert_within(host(y), 1.5 * M.matvec(x64) - 0.5 * y64,
                          1.5 * (D @ np.abs(x64)) + 0.5 * np.abs(y64), dtype, what)
            y = torch.empty(M.shape[0], dtype=MM.dtype, device="cuda")
            J.mul_(y, MM, dev(xs))
            got = host(y).copy()
            assert_within(got, M.matvec(x64), D @ np.abs(x64), dtype, what + " beta 0")
            monkeypatch.setattr(bb, "USE_PERIODIC", False)
            J.mul_(y, MM, dev(xs))
            monkeypatch.setattr(bb, "USE_PERIODIC", True)
            assert_within(got, host(y).astype(np.float64), D @ np.abs(x64), dtype, what + " vs assembled")


def test_bbm_periodic_eligibility(J):
    """The periodic view exists only for bandwidth 1 with a BlockSparseMatrix
    diagonal and one shared (neg, pos) pair of CSR or ShiftedDiag tensors
    (_bbm_supports_periodic, block_mul.jl:600-606)."""
    T, nd, no, nc = 3, 10, 3, 10
    grid = [[random_block(nd, 6, 0.4, 41), random_block(nd, 4, 0.4, 42, 1)]]
    neg, pos = random_block(no, nc, 0.3, 43), random_block(no, nc, 0.3, 44)
    BM = device_bsm(J, grid)
    assert J.BlockBandedMatrix(BM, to_ust(J, neg), to_ust(J, pos), T, nd, no, nc).periodic() is not None
    D = to_ust(J, random_block(nd, nc, 0.3, 45))
    assert J.BlockBandedMatrix(D, to_ust(J, neg), to_ust(J, pos), T, nd, no, nc).periodic() is None
    coo = to_ust(J, random_block(no, nc, 0.3, 46, fmt="COO"))
    assert J.BlockBandedMatrix(BM, coo, to_ust(J, pos), T, nd, no, nc).periodic() is None
    pairs = [(to_ust(J, neg), to_ust(J, pos))] * (T - 1)
    assert J.BlockBandedMatrix(BM, [pairs], T, 1, nd, [no], nc).periodic() is None


def test_bbm_bw2_time_varying(J, BO):
    import torch
    T, nd, n1, n2, nc = 5, 12, 4, 3, 10
    Ds = [random_block(nd, nc, 0.3, 10 + t, t % 2, fmt="CSR" if t % 2 else "DCSR") for t in range(T)]
    band1 = [(random_block(n1, nc, 0.3, 20 + t), random_block(n1, nc, 0.3, 30 + t, 1))
             for t in range(T - 1)]
    band2 = (random_block(n2, nc, 0.4, 40), random_block(n2, nc, 0.4, 41, 1))
    M = BO.BBM(Ds, [band1, band2], T, nd, [n1, n2], nc)
    MM = J.BlockBandedMatrix([to_ust(J, d) for d in Ds],
                             [[(to_ust(J, a), to_ust(J, b)) for a, b in band1],
                              (to_ust(J, band2[0]), to_ust(J, band2[1]))],
                             T, 2, nd, [n1, n2], nc)
    assert MM.size() == M.shape and MM.d_starts() == BO.diag_starts(nd, [n1, n2], T)
    xs = np.random.default_rng(4).uniform(-1, 1, M.shape[1])
    y = torch.empty(M.shape[0], dtype=torch.float64, device="cuda")
    J.mul_(y, MM, dev(xs))
    rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
    D = sp.csr_matrix((val, colind, rowptr), shape=M.shape)
    assert_within(host(y), M.matvec(xs), abs(D) @ np.abs(xs), np.float64, "BBM bw=2")
    assert host(J.coordinates(MM.assembled().asm, 2)).tolist() == colind.tolist()


def test_bsm_graph_replay(J, BO, monkeypatch):
    """Repeated products with the same (y, x, alpha, beta) replay a captured
    graph (block_mul.jl:233-267).  Every call -- after new x values, with
    beta != 0 reading y, after update_block_values! -- equals the direct
    launch bit for bit; new buffers or coefficients get their own capture, the
    oldest is dropped past the cache size, and a call made inside an outer
    capture launches directly so that the outer graph records it."""
    import torch
    from jlust_amd import block_sparse as bs
    monkeypatch.setattr(bs, "USE_GRAPHS", True)
    grid = mixed_grid(9)
    BM = device_bsm(J, grid)
    m, n = BM.shape
    rng = np.random.default_rng(12)
    y0 = dev(rng.uniform(-1, 1, m))
    x1, x2 = torch.empty(n, dtype=torch.float64, device="cuda"), \
        torch.empty(n, dtype=torch.float64, device="cuda")
    y1, yr = torch.empty(m, dtype=torch.float64, device="cuda"), \
        torch.empty(m, dtype=torch.float64, device="cuda")

    def direct(x, alpha, beta):
        monkeypatch.setattr(bs, "USE_GRAPHS", False)
        yr.copy_(y0)
        J.mul_(yr, BM, x, alpha, beta)
        monkeypatch.setattr(bs, "USE_GRAPHS", True)
        return host(yr).copy()

    def check(x, alpha, beta, what):
        x.uniform_(-1.0, 1.0)
        y1.copy_(y0)
        J.mul_(y1, BM, x, alpha, beta)
        got = host(y1).copy()
        np.testing.assert_array_equal(got, direct(x, alpha, beta), err_msg=what)

    for call in range(4):
        check(x1, 1.5, -0.5, f"call {call}")
    asm = BM.assembled()
    assert len(asm._graphs) == 1 and asm._last_graph is not None
    A = BO.BSM(grid)
    xs = host(x1).copy()
    y1.copy_(y0)
    J.mul_(y1, BM, x1, 1.5, -0.5)
    assert_within(host(y1), 1.5 * A.matvec(xs) - 0.5 * host(y0),
                  1.5 * abs_bound(A.dense(), xs) + 0.5 * np.abs(host(y0)), np.float64, "replayed")
    for (i, j) in ((1, 1), (3, 4)):
        b = grid[i - 1][j - 1]
        b["val"] = rng.uniform(-1, 1, b["val"].size)
        J.update_block_values_(BM, i, j, dev(b["val"]))
        check(x1, 1.5, -0.5, f"after update of ({i},{j})")
    assert len(asm._graphs) == 1
    check(x2, 1.5, -0.5, "second x buffer")
    check(x2, 1.5, -0.5, "second x buffer, replay")
    check(x1, 1.0, 0.0, "other coefficients")
    check(x1, 1.0, 0.0, "other coefficients, replay")
    check(x1, 1.5, -0.5, "first key again")
    assert len(asm._graphs) == 3

    monkeypatch.setattr(bs, "GRAPH_CACHE", 3)
    for a in (2.0, 3.0, 2.0, 4.0, 4.0):
        check(x1, a, 0.25, f"alpha {a}")
        assert len(asm._graphs) <= 3

    # Inside an outer capture the product is recorded, not replayed.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        J.mul_(y1, BM, x1, 1.5, -0.5)
    for rep in range(3):
        x1.uniform_(-1.0, 1.0)
        y1.copy_(y0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(y1), direct(x1, 1.5, -0.5), err_msg=f"outer {rep}")


def test_bbm_graph_replay(J, BO, monkeypatch):
    """A block-banded product through the assembled CSR replays its capture
    too, and follows value updates of its diagonal block matrix (the periodic
    kernel, this matrix's default, launches directly)."""
    import torch
    from jlust_amd import block_banded as bb
    from jlust_amd import block_sparse as bs
    monkeypatch.setattr(bs, "USE_GRAPHS", True)
    monkeypatch.setattr(bb, "USE_PERIODIC", False)
    T = 5
    grid = [[random_block(10, 6, 0.4, 21), random_block(10, 4, 0.4, 22, 1)]]
    negR, R = random_block(3, 10, 0.3, 23), random_block(3, 10, 0.3, 24)
    BM = device_bsm(J, grid)
    MM = J.BlockBandedMatrix(BM, to_ust(J, negR), to_ust(J, R), T, 10, 3, 10)
    x = torch.empty(T * 10, dtype=torch.float64, device="cuda")
    y = torch.empty(MM.size(1), dtype=torch.float64, device="cuda")
    rng = np.random.default_rng(25)
    for call in range(4):
        if call == 2:
            grid[0][0]["val"] = rng.uniform(-1, 1, grid[0][0]["val"].size)
            J.update_block_values_(BM, 1, 1, dev(grid[0][0]["val"]))
        x.uniform_(-1.0, 1.0)
        J.mul_(y, MM, x)
        xs = host(x).copy()
        M = BO.BBM(BO.BSM(grid), [(negR, R)], T, 10, [3], 10)
        rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
        D = sp.csr_matrix((val, colind, rowptr), shape=M.shape)
        assert_within(host(y), M.matvec(xs), abs(D) @ np.abs(xs), np.float64, f"BBM call {call}")
    assert len(MM.assembled()._graphs) == 1


def test_bbm_follows_bsm_updates(J, BO):
    import torch
    T = 3
    grid = [[random_block(10, 6, 0.4, 1), random_block(10, 4, 0.4, 2, 1)]]
    negR = random_block(3, 10, 0.3, 3)
    R = random_block(3, 10, 0.3, 4)
    BM = device_bsm(J, grid)
    MM = J.BlockBandedMatrix(BM, to_ust(J, negR), to_ust(J, R), T, 10, 3, 10)
    xs = np.random.default_rng(5).uniform(-1, 1, T * 10)
    y = torch.empty(MM.size(1), dtype=torch.float64, device="cuda")
    J.mul_(y, MM, dev(xs))
    grid[0][1]["val"] = np.random.default_rng(6).uniform(-1, 1, grid[0][1]["val"].size)
    J.update_block_values_(BM, 1, 2, dev(grid[0][1]["val"]))
    J.mul_(y, MM, dev(xs))
    M = BO.BBM(BO.BSM(grid), [(negR, R)], T, 10, [3], 10)
    rowptr, colind, val = BO.assemble(*M.shape, list(M.placements()))
    D = sp.csr_matrix((val, colind, rowptr), shape=M.shape)
    assert_within(host(y), M.matvec(xs), abs(D) @ np.abs(xs), np.float64, "BBM after update")
    assert np.array_equal(host(J.nonzeros(MM.assembled().asm)), val)


def test_bbm_fallback_per_period(J, BO):
    """A COO coupling block is not assembled: per-period products at d_starts."""
    import torch
    T, nd, no, nc = 4, 8, 3, 6
    D = random_block(nd, nc, 0.4, 1)
    neg, pos = random_block(no, nc, 0.4, 2, fmt="COO"), random_block(no, nc, 0.4, 3, 1)
    M = BO.BBM(D, [(neg, pos)], T, nd, [no], nc)
    MM = J.BlockBandedMatrix(to_ust(J, D), to_ust(J, neg), to_ust(J, pos), T, nd, no, nc)
    assert not MM.assemblable()
    xs = np.random.default_rng(7).uniform(-1, 1, M.shape[1])
    y = torch.empty(M.shape[0], dtype=torch.float64, device="cuda")
    J.mul_(y, MM, dev(xs))
    full = np.zeros(M.shape)
    for b, r0, c0 in M.placements():
        d = BO.dense(b)
        full[r0:r0 + d.shape[0], c0:c0 + d.shape[1]] += d
    assert_within(host(y), M.matvec(xs), np.abs(full) @ np.abs(xs), np.float64, "BBM fallback")
