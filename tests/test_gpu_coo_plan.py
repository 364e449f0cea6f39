"""Prepared COO SpMV (jlust_hip_coo_spmv_plan_create: entries put in row order
once, products in the CSR plan) against the oracle's COO SpMV
(oracle/jlust_cpu.c, ext/KernelAbstractionsExt/ops/spmv.jl:407-448):
sorted and unsorted rows, duplicates, both origins, f32/f64, alpha/beta,
update_values in the caller's order, a column-sliced plan, run-to-run
identical results, and bad row indices rejected."""
import numpy as np
import pytest

from tests._util import assert_within, dev, host

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


def random_coo(m, n, nnz, seed, origin, dtype, sort=False):
    rng = np.random.default_rng(seed)
    rows = rng.integers(0, m, nnz)
    cols = rng.integers(0, n, nnz)
    if sort:
        o = np.argsort(rows, kind="stable")
        rows, cols = rows[o], cols[o]
    val = rng.uniform(-1, 1, nnz).astype(dtype)
    return (rows + origin).astype(np.int32), (cols + origin).astype(np.int32), val


def absref(rows, cols, val, x, m, alpha, beta, y0, origin):
    a = np.zeros(m)
    np.add.at(a, rows - origin, np.abs(val.astype(np.float64)) * np.abs(x[cols - origin].astype(np.float64)))
    return abs(alpha) * a + abs(beta) * np.abs(y0.astype(np.float64))


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [0, 1])
@pytest.mark.parametrize("sort", [True, False])
def test_plan_matches_oracle(J, O, dtype, origin, sort):
    import torch
    m, n, nnz = 900, 700, 6000          # duplicates and empty rows both occur
    rows, cols, val = random_coo(m, n, nnz, 3 + origin + 2 * sort, origin, dtype, sort)
    A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n),
                     origin=J.OneBased() if origin else J.ZeroBased())
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert isinstance(h, J.hip_backend.HIPSpMVHandle)
    rng = np.random.default_rng(5)
    xs = rng.uniform(-1, 1, n).astype(dtype)
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    y = dev(y0)
    J.execute(h, dev(xs), y, alpha=1.5, beta=-0.25)
    ref = O.coo_spmv(rows, cols, val, xs, m, 1.5, -0.25, y0, origin)
    assert_within(host(y), ref, absref(rows, cols, val, xs, m, 1.5, -0.25, y0, origin), dtype,
                  "COO plan")
    y2 = dev(y0)
    J.execute(h, dev(xs), y2, alpha=1.5, beta=-0.25)
    assert torch.equal(y, y2)                         # no atomics: identical run to run
    # new values in the caller's order
    val2 = rng.uniform(-1, 1, nnz).astype(dtype)
    J.update_values_(h, J.coo_tensor(dev(rows), dev(cols), dev(val2), (m, n),
                                     origin=J.OneBased() if origin else J.ZeroBased()))
    y3 = dev(np.zeros(m, dtype))
    J.execute(h, dev(xs), y3)
    ref3 = O.coo_spmv(rows, cols, val2, xs, m, 1.0, 0.0, None, origin)
    assert_within(host(y3), ref3, absref(rows, cols, val2, xs, m, 1.0, 0.0, np.zeros(m), origin),
                  dtype, "COO plan after update_values")


@pytest.mark.parametrize("layout", ["1", "2"], ids=["sliced", "binned"])
def test_sliced_plan_unsorted(J, O, monkeypatch, layout):
    """x of 5 MB with random columns, slices (1) or LDS bins (2) forced: the
    CSR plan under the COO plan re-lays A out (its 400k entries are below the
    automatic thresholds)."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", layout)
    m, n, nnz = 50_000, 640_000, 400_000
    rows, cols, val = random_coo(m, n, nnz, 8, 1, np.float64)
    A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    xs = np.random.default_rng(9).uniform(-1, 1, n)
    y = dev(np.zeros(m))
    J.execute(h, dev(xs), y)
    ref = O.coo_spmv(rows, cols, val, xs, m)
    bound = absref(rows, cols, val, xs, m, 1.0, 0.0, np.zeros(m), 1)
    assert_within(host(y), ref, bound, np.float64, "sliced COO plan")
    val2 = -2.0 * val
    J.update_values_(h, J.coo_tensor(dev(rows), dev(cols), dev(val2), (m, n)))
    J.execute(h, dev(xs), y)
    assert_within(host(y), -2.0 * ref, 2 * bound, np.float64, "sliced COO plan after update")


def test_empty_and_errors(J):
    A = J.coo_tensor(dev(np.zeros(0, np.int32)), dev(np.zeros(0, np.int32)), dev(np.zeros(0)), (5, 4))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    y = dev(np.full(5, 3.0))
    J.execute(h, dev(np.ones(4)), y, beta=2.0)
    assert host(y).tolist() == [6.0] * 5
    bad = J.coo_tensor(dev(np.int32([1, 7])), dev(np.int32([1, 1])), dev(np.ones(2)), (5, 4))
    with pytest.raises(J.NonCanonicalStorage):
        J.prepare(J.HIPBackend(), J.SpMVOp, bad)
    with pytest.raises(J.UnsupportedFormat, match="output_fn"):
        J.prepare(J.HIPBackend(), J.SpMVOp, A, output_fn=J.abs_fn)


@pytest.mark.parametrize("kind", ["rows", "sliced", "binned"])
def test_coo_plan_capture(J, O, monkeypatch, kind):
    """A COO plan recorded as a HIP graph (jlust_hip_csr_spmv_plan_capture_*)
    and launched: each launch equals execute(h, x, y) bit for bit, also after
    update_values! (new values in caller order, scattered into the plan's own
    row-ordered copy, which the graph reads, and from there into the sliced or
    binned layout), and matches the oracle."""
    import torch
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", {"rows": "0", "sliced": "1", "binned": "2"}[kind])
    m, n, nnz = 20_000, (30_000 if kind == "rows" else 640_000), 160_000
    rows, cols, val = random_coo(m, n, nnz, 12, 1, np.float64)
    A = J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    if kind == "rows":
        assert h.kernel() in ("merge", "vector")
    else:
        assert h.kernel() == kind
    x = torch.empty(n, dtype=torch.float64, device="cuda")
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    ye = torch.empty(m, dtype=torch.float64, device="cuda")
    y0 = np.random.default_rng(13).uniform(-1, 1, m)
    g = h.capture(x, y, alpha=1.25, beta=-1.0)
    for rep in range(3):
        if rep == 2:
            val = -0.5 * val
            J.update_values_(h, J.coo_tensor(dev(rows), dev(cols), dev(val), (m, n)))
        xs = np.random.default_rng(20 + rep).uniform(-1, 1, n)
        x.copy_(torch.from_numpy(xs))
        y.copy_(torch.from_numpy(y0))
        assert g.launch()
        ye.copy_(torch.from_numpy(y0))
        J.execute(h, x, ye, alpha=1.25, beta=-1.0)
        torch.cuda.synchronize()
        got = host(y).copy()
        np.testing.assert_array_equal(got, host(ye), err_msg=f"launch {rep}")
        ref = 1.25 * O.coo_spmv(rows, cols, val, xs, m) - y0
        assert_within(got, ref, absref(rows, cols, val, xs, m, 1.25, -1.0, y0, 1), np.float64,
                      f"captured COO plan, launch {rep}")
    del g
    torch.cuda.synchronize()
