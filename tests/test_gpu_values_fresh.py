"""Prepared SpMV plans read A's values as they are at each call.

execute(h, A, x, y) takes A at every call (EmitterSpMVHandle, ext/
KernelAbstractionsExt/ops/spmv.jl:531-544), and the cuSPARSE-style
execute(h, x, y) reads the buffer its descriptor points at (ext/CUDAExt/ops/
spmv.jl:40-43,63-78).  Plans that hold a permuted copy of the values (sliced,
binned, reordered COO) must therefore gather values written in place before
the product.  Every plan kind is checked against the oracle after an in-place
write with no update_values_, in both forms, and a captured graph is checked
after its value buffer is replaced.
"""
import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr

pytestmark = pytest.mark.gpu

# (plan kind, JLUST_HIP_SPMV_SLICE, JLUST_HIP_SPMV_VECTOR, lengths of rows)
KINDS = [
    ("merge", "0", "0", None),
    ("vector", "0", None, None),
    ("sliced", "1", "0", None),
    ("binned", "2", None, None),
]


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


def _env(monkeypatch, slice_, vector):
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", slice_)
    if vector is None:
        monkeypatch.delenv("JLUST_HIP_SPMV_VECTOR", raising=False)
    else:
        monkeypatch.setenv("JLUST_HIP_SPMV_VECTOR", vector)


def _check(O, rowptr, colind, val, x, y, dtype, what, alpha=1.0, beta=0.0, y0=None):
    ref = O.csr_spmv(rowptr, colind, val, x, alpha, beta, y0)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, alpha, beta, y0)
    assert_within(host(y), ref, absref, dtype, what)


@pytest.mark.parametrize("kind,slice_,vector,_", KINDS, ids=[k[0] for k in KINDS])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csr_plan_sees_in_place_writes(J, O, kind, slice_, vector, _, dtype, monkeypatch):
    import torch
    _env(monkeypatch, slice_, vector)
    m, n = 3000, 5000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(7).integers(0, 24, m),
                                     seed=11, dtype=dtype)
    x = np.random.default_rng(3).uniform(-1, 1, n).astype(dtype)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() == kind
    xd = dev(x)
    y = torch.empty(m, dtype=A.dtype, device="cuda")
    J.execute(h, A, xd, y)
    _check(O, rowptr, colind, val, x, y, dtype, f"{kind}: first product")

    # In place, no update_values_: the three-argument form.
    val2 = np.random.default_rng(5).uniform(-2, 2, val.size).astype(dtype)
    J.nonzeros(A).copy_(dev(val2))
    J.execute(h, A, xd, y)
    _check(O, rowptr, colind, val2, x, y, dtype, f"{kind}: execute(h, A, x, y) after copy_")

    # In place again, then the two-argument (raw) and USTensor forms.
    J.nonzeros(A).mul_(-0.5)
    val3 = (val2 * dtype(-0.5)).astype(dtype)
    J.execute(h, xd, y)
    _check(O, rowptr, colind, val3, x, y, dtype, f"{kind}: execute(h, x, y) after mul_")
    y0 = np.random.default_rng(9).uniform(-1, 1, m).astype(dtype)
    yd = dev(y0)
    J.execute(h, J.ust(xd), J.ust(yd), alpha=1.5, beta=-0.25)
    _check(O, rowptr, colind, val3, x, yd, dtype, f"{kind}: execute(h, ux, uy) beta",
           alpha=1.5, beta=-0.25, y0=y0)

    # A different value tensor given at the call becomes the plan's values.
    val4 = np.random.default_rng(6).uniform(-1, 1, val.size).astype(dtype)
    A4 = J.csr_tensor(J.positions(A, 2), J.coordinates(A, 2), dev(val4), (m, n))
    J.execute(h, A4, xd, y)
    _check(O, rowptr, colind, val4, x, y, dtype, f"{kind}: execute(h, A4, x, y)")
    J.execute(h, xd, y)
    _check(O, rowptr, colind, val4, x, y, dtype, f"{kind}: execute(h, x, y) after A4")


@pytest.mark.parametrize("unsorted", [False, True])
@pytest.mark.parametrize("slice_", ["0", "2"])
def test_coo_plan_sees_in_place_writes(J, O, unsorted, slice_, monkeypatch):
    import torch
    _env(monkeypatch, slice_, None)
    m, n, nnz = 2000, 3000, 30000
    rng = np.random.default_rng(21)
    rows = rng.integers(0, m, nnz)
    cols = rng.integers(0, n, nnz)
    if not unsorted:
        o = np.lexsort((cols, rows))
        rows, cols = rows[o], cols[o]
    val = rng.uniform(-1, 1, nnz)
    x = rng.uniform(-1, 1, n)
    A = J.coo_tensor(dev((rows + 1).astype(np.int32)), dev((cols + 1).astype(np.int32)),
                     dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    xd = dev(x)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    for step in range(3):
        v = rng.uniform(-1, 1, nnz)
        J.nonzeros(A).copy_(dev(v))
        if step % 2:
            J.execute(h, xd, y)
        else:
            J.execute(h, A, xd, y)
        ref = O.coo_spmv(rows + 1, cols + 1, v, x, m)
        absref = O.coo_spmv(rows + 1, cols + 1, np.abs(v), np.abs(x), m)
        assert_within(host(y), ref, absref, np.float64, f"coo unsorted={unsorted} step {step}")


@pytest.mark.parametrize("kind,slice_,vector,_", KINDS, ids=[k[0] for k in KINDS])
def test_graph_follows_value_buffer(J, O, kind, slice_, vector, _, monkeypatch):
    """A captured plan replays with the handle's current values: a replaced
    value tensor (update_values_ with another buffer) is captured again on a
    merge or vector plan; an in-place write is gathered on a copying plan."""
    import torch
    _env(monkeypatch, slice_, vector)
    m, n = 2500, 4000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(1).integers(1, 20, m),
                                     seed=4)
    x = np.random.default_rng(2).uniform(-1, 1, n)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() == kind
    xd = dev(x)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    g = h.capture(xd, y)
    assert g.launch()
    _check(O, rowptr, colind, val, x, y, np.float64, f"{kind}: first replay")

    val2 = np.random.default_rng(8).uniform(-1, 1, val.size)
    A2 = J.csr_tensor(J.positions(A, 2), J.coordinates(A, 2), dev(val2), (m, n))
    J.update_values_(h, A2)
    del A2
    torch.cuda.empty_cache()
    junk = torch.full((val.size * 4,), float("nan"), dtype=torch.float64, device="cuda")
    assert g.launch()
    _check(O, rowptr, colind, val2, x, y, np.float64, f"{kind}: replay after update_values_")

    J.nonzeros(h.u_A).mul_(3.0)
    assert g.launch()
    _check(O, rowptr, colind, val2 * 3.0, x, y, np.float64, f"{kind}: replay after mul_")
    del junk
