"""Repeated plain SpMV calls reuse a cached plan (hip_backend.PLAN_CACHE, the
counterpart of the reference's per-matrix cache in its GPU mul!,
ext/CUDAExt/ops/block_mul.jl:53,227,327-357): every call matches the oracle,
before and after the switch to the plan; the plan is dropped when an index
tensor is written in place, when other tensors are passed, and when the
matrix's tensors are freed (its device memory is given back); values written
in place are seen."""
import gc

import numpy as np
import pytest

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


@pytest.fixture()
def cache():
    from jlust_amd import hip_backend as HB
    c = HB.PLAN_CACHE
    saved = (c.enabled, c.after, c.max_plans, c.max_bytes)
    c.clear()
    c.enabled, c.after = True, 2
    yield c
    c.clear()
    c.enabled, c.after, c.max_plans, c.max_bytes = saved


def _powerlaw(m, n, seed):
    rng = np.random.default_rng(seed)
    lens = np.minimum((rng.pareto(1.8, m) + 1) * 6, n).astype(np.int64)
    return random_csr(m, n, lengths=lens, seed=seed)


@pytest.mark.parametrize("slice_mode", ["auto", "2"])
def test_plain_calls_switch_to_a_plan(J, O, cache, slice_mode, monkeypatch):
    import torch
    if slice_mode == "2":
        monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")     # the binned layout
    m, n = 60000, 50000
    rowptr, colind, val = _powerlaw(m, n, 90)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    rng = np.random.default_rng(91)
    for call in range(6):
        x = rng.uniform(-1, 1, n)
        y0 = rng.uniform(-1, 1, m)
        y = dev(y0)
        J.execute(J.SpMVOp, A, dev(x), y, alpha=1.5, beta=-0.5)
        ref = O.csr_spmv(rowptr, colind, val, x, 1.5, -0.5, y0)
        absref = O.csr_spmv_absref(rowptr, colind, val, x, 1.5, -0.5, y0)
        assert_within(host(y), ref, absref, np.float64, f"call {call}")
        assert len(cache.info()) == (1 if call >= 2 else 0), (call, cache.info())
    if slice_mode == "2":
        assert cache.info()[0]["kernel"] == "binned"
        # values written in place through torch: the plan's copy is refreshed
        J.nonzeros(A).mul_(2.0)
        x = rng.uniform(-1, 1, n)
        y = torch.empty(m, dtype=torch.float64, device="cuda")
        J.execute(J.SpMVOp, A, dev(x), y)
        assert_within(host(y), O.csr_spmv(rowptr, colind, 2.0 * val, x),
                      O.csr_spmv_absref(rowptr, colind, 2.0 * val, x), np.float64, "in-place values")


def test_cache_invalidation_and_release(J, O, cache):
    import torch
    m, n = 40000, 40000
    rowptr, colind, val = _powerlaw(m, n, 92)
    rp, ci, v = dev(rowptr), dev(colind), dev(val)
    A = J.csr_tensor(rp, ci, v, (m, n))
    x = np.random.default_rng(93).uniform(-1, 1, n)
    xd = dev(x)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    for _ in range(3):
        J.execute(J.SpMVOp, A, xd, y)
    assert len(cache.info()) == 1
    # an index tensor written in place (another valid pattern): the plan is dropped
    colind2 = colind.copy()
    row0 = slice(rowptr[0] - 1, rowptr[1] - 1)
    colind2[row0] = np.sort(np.random.default_rng(94).choice(n, size=row0.stop - row0.start,
                                                              replace=False)) + 1
    ci.copy_(dev(colind2))
    J.execute(J.SpMVOp, A, xd, y)
    assert len(cache.info()) == 0
    assert_within(host(y), O.csr_spmv(rowptr, colind2, val, x), O.csr_spmv_absref(rowptr, colind2, val, x),
                  np.float64, "after an in-place pattern write")
    for _ in range(3):
        J.execute(J.SpMVOp, A, xd, y)
    assert len(cache.info()) == 1
    # other tensors (copies of the same arrays) are another matrix
    A2 = J.csr_tensor(rp.clone(), ci.clone(), v.clone(), (m, n))
    J.execute(J.SpMVOp, A2, xd, y)
    assert len(cache.info()) == 1
    assert_within(host(y), O.csr_spmv(rowptr, colind2, val, x), O.csr_spmv_absref(rowptr, colind2, val, x),
                  np.float64, "another matrix")
    # freeing the matrix's tensors drops the plan and gives its memory back
    torch.cuda.synchronize()
    del A, A2, rp, ci, v
    gc.collect()
    torch.cuda.synchronize()
    assert cache.info() == []


def test_cache_budget_and_switch(J, O, cache):
    import torch
    m, n = 30000, 30000
    mats = [_powerlaw(m, n, s) for s in (95, 96, 97)]
    As = [J.csr_tensor(dev(a), dev(b), dev(c), (m, n)) for a, b, c in mats]
    x = np.random.default_rng(98).uniform(-1, 1, n)
    xd = dev(x)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    cache.max_plans = 2
    for A in As:
        for _ in range(3):
            J.execute(J.SpMVOp, A, xd, y)
    assert len(cache.info()) == 2                        # the least recently used one is out
    for (rowptr, colind, val), A in zip(mats, As):
        J.execute(J.SpMVOp, A, xd, y)
        assert_within(host(y), O.csr_spmv(rowptr, colind, val, x), O.csr_spmv_absref(rowptr, colind, val, x),
                      np.float64, "budget")
    cache.clear()
    cache.enabled = False
    for _ in range(4):
        J.execute(J.SpMVOp, As[0], xd, y)
    assert cache.info() == []


def test_coo_plain_calls_switch_to_a_plan(J, O, cache):
    import torch
    m, n = 20000, 25000
    rowptr, colind, val = _powerlaw(m, n, 99)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    p = np.random.default_rng(100).permutation(rows.size)
    A = J.coo_tensor(dev(rows[p]), dev(colind[p]), dev(val[p]), (m, n))
    x = np.random.default_rng(101).uniform(-1, 1, n)
    ref = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    for call in range(4):
        J.execute(J.SpMVOp, A, dev(x), y)
        assert_within(host(y), ref, absref, np.float64, f"COO call {call}")
    assert len(cache.info()) == 1


@pytest.mark.parametrize("b1,b2,dtype", [(4, 3, np.float64), (16, 16, np.float32)])
def test_bsr_plain_calls_switch_to_a_plan(J, O, cache, b1, b2, dtype):
    """BSR SpMV plain calls: the third on a matrix builds its segment table
    once (a BSR SpMV plan, jlust_hip_bsr_spmv_plan_*); every product matches
    the oracle before and after the switch; values written in place are seen;
    a block column written in place drops the plan."""
    import torch
    mb, nb = 300, 200
    rng = np.random.default_rng(102 + b1)
    lens = np.minimum((rng.pareto(1.3, mb) + 1) * 2, nb).astype(np.int64)
    lens[::7] = 0
    lens[5] = 120                                        # several segments of 32 blocks
    bcols = [np.sort(rng.choice(nb, int(n), replace=False)) for n in lens]
    bp = (np.r_[0, np.cumsum(lens)] + 1).astype(np.int32)
    bc = (np.concatenate(bcols) + 1).astype(np.int32)
    flat = rng.standard_normal(bc.size * b1 * b2).astype(dtype)
    A = J.bsr_tensor(dev(bp), dev(bc), dev(flat), (mb * b1, nb * b2), (b1, b2), True, J.OneBased())

    def check(vals, bcv, what):
        rp, ci, v = O.bsr_to_csr(bp, bcv, vals, b1, 1, True, b2)
        x = rng.uniform(-1, 1, nb * b2).astype(dtype)
        y0 = rng.uniform(-1, 1, mb * b1).astype(dtype)
        y = dev(y0.copy())
        J.execute(J.SpMVOp, A, dev(x), y, alpha=1.5, beta=-0.5)
        ref = O.csr_spmv(rp, ci, v, x, 1.5, -0.5, y0)
        absref = O.csr_spmv_absref(rp, ci, v, x, 1.5, -0.5, y0)
        assert_within(host(y), ref, absref, dtype, f"bsr {b1}x{b2} {what}")

    for call in range(4):
        check(flat, bc, f"call {call}")
        assert len(cache.info()) == (1 if call >= 2 else 0), (call, cache.info())
    assert cache.info()[0]["kernel"] == "bsr_segments"
    A.val.mul_(-2.0)                                     # in place: the plan reads the values at the call
    check(flat * -2, bc, "values scaled in place")
    assert len(cache.info()) == 1
    bc2 = bc.copy()                                      # a block column moved within its row's range
    r = int(np.flatnonzero(lens > 0)[0])
    lo, hi = bp[r] - 1, bp[r + 1] - 1
    free = np.setdiff1d(np.arange(1, nb + 1), bc[lo:hi])
    bc2[lo] = free[0]
    bc2[lo:hi] = np.sort(bc2[lo:hi])
    A.crd_buffers[1].copy_(dev(bc2))
    check(flat * -2, bc2, "block column written in place")
    assert cache.info() == []
    torch.cuda.synchronize()


@pytest.mark.parametrize("fmt", ["coo", "csc"])
def test_coo_csc_spmm_plain_calls_switch_to_a_plan(J, O, cache, fmt):
    """Plain SpMM calls with a COO (entries shuffled) or CSC A: the third on a
    matrix and column count builds a COO/CSC SpMM plan (the entries put in row
    order once); every product matches the oracle; values written in place
    are gathered again; another column count is another plan; an index
    tensor written in place drops the plan."""
    m, n, k = 3000, 2500, 24
    rowptr, colind, val = _powerlaw(m, n, 103)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    rng = np.random.default_rng(104)
    if fmt == "coo":
        p = rng.permutation(rows.size)
        A = J.coo_tensor(dev(rows[p]), dev(colind[p]), dev(val[p]), (m, n))
    else:
        o = np.lexsort((rows, colind))                   # by column, rows ascending within one
        colptr = (np.r_[0, np.cumsum(np.bincount(colind - 1, minlength=n))] + 1).astype(np.int32)
        A = J.csc_tensor(dev(colptr), dev(rows[o]), dev(val[o]), (m, n))

    def check(v, what, kk=k):
        B = np.asfortranarray(rng.standard_normal((n, kk)))
        C0 = np.asfortranarray(rng.standard_normal((m, kk)))
        C = dev(C0)
        J.execute(J.SpMMOp, A, dev(B), C, alpha=1.25, beta=-0.5)
        ref, _ = O.csr_spmm(rowptr, colind, v, B, 1.25, -0.5, C0)
        absref = O.csr_spmm_absref(rowptr, colind, v, B, 1.25, -0.5, C0)
        assert_within(host(C), ref, absref, np.float64, f"{fmt} SpMM {what}")

    for call in range(4):
        check(val, f"call {call}")
        assert len(cache.info()) == (1 if call >= 2 else 0), (call, cache.info())
    assert cache.info()[0]["kernel"] == f"{fmt}_spmm"
    J.nonzeros(A).mul_(-2.0)                             # in place: gathered again in row order
    check(-2.0 * val, "values scaled in place")
    for call in range(3):
        check(-2.0 * val, f"k=40 call {call}", kk=40)
    assert len(cache.info()) == 2                        # one plan per column count
    A.crd_buffers[1].add_(0)                             # an index tensor written in place
    check(-2.0 * val, "after an index write")
    assert len(cache.info()) == 1                        # the k=24 plan is gone


def test_csc_spmv_plain_calls_switch_to_a_plan(J, O, cache):
    """Plain CSC SpMV calls: the third on a matrix builds a plan (CSC planned
    as COO, each entry's column expanded from colptr); values written in place
    are gathered again.  A square CSR matrix on the very same three tensors
    is the CSC one's transpose: the two get plans of their own."""
    import torch
    n = 20000
    rowptr, colind, val = _powerlaw(n, n, 105)
    p, i, v = dev(rowptr), dev(colind), dev(val)
    A_csr = J.csr_tensor(p, i, v, (n, n))
    A_csc = J.csc_tensor(p, i, v, (n, n))               # the transpose of A_csr
    rows = np.repeat(np.arange(1, n + 1, dtype=np.int32), np.diff(rowptr))
    # A_csc as CSR: entry (colind, row) of A_csr is (row, col) of A_csc
    t_order = np.lexsort((rows, colind))
    t_rowptr = (np.r_[0, np.cumsum(np.bincount(colind - 1, minlength=n))] + 1).astype(np.int32)
    t_cols, t_val = rows[t_order], val[t_order]
    x = np.random.default_rng(106).uniform(-1, 1, n)
    xd = dev(x)
    y = torch.empty(n, dtype=torch.float64, device="cuda")

    def check(A, scale, what):
        J.execute(J.SpMVOp, A, xd, y)
        if A is A_csr:
            ref = O.csr_spmv(rowptr, colind, scale * val, x)
            absref = O.csr_spmv_absref(rowptr, colind, scale * val, x)
        else:
            ref = O.csr_spmv(t_rowptr, t_cols, scale * t_val, x)
            absref = O.csr_spmv_absref(t_rowptr, t_cols, scale * t_val, x)
        assert_within(host(y), ref, absref, np.float64, what)

    for call in range(4):
        check(A_csc, 1.0, f"CSC call {call}")
        check(A_csr, 1.0, f"CSR call {call}")
    assert len(cache.info()) == 2
    v.mul_(3.0)                                          # in place: both plans see it
    check(A_csc, 3.0, "CSC values scaled in place")
    check(A_csr, 3.0, "CSR values scaled in place")
