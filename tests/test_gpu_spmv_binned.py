"""GPU parity of the LDS-binned SpMV plan (x in column slices held in LDS by
a slice pass, partial sums added per row bin in LDS by a bin pass) against
the CPU oracle.

JLUST_HIP_SPMV_SLICE=2 asks a plan for the binned layout wherever it fits
(nnz >= 1, at most 1024 slices).  Bar: |y - y_ref| <= 1e-12 (fp64) / 1e-5
(fp32) x (|alpha||A||x| + |beta||y0|) elementwise; the binned sums associate
per slice, so they are not bit-identical to the sequential oracle, but they
are deterministic run to run (checked bit for bit).
"""
import zlib

import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr
from tests.test_gpu_spmv import SHAPES

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


def run_binned(J, rowptr, colind, val, x, m, n, origin=1, alpha=1.0, beta=0.0, y0=None):
    import torch
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n),
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    y = dev(y0) if y0 is not None else torch.full((m,), float("nan"), dtype=A.dtype,
                                                   device="cuda")
    J.execute(h, dev(x), y, alpha=alpha, beta=beta)
    return host(y), h, A


def check(J, O, rowptr, colind, val, x, m, n, dtype, what, origin=1, alpha=1.0, beta=0.0,
          y0=None):
    y, h, A = run_binned(J, rowptr, colind, val, x, m, n, origin, alpha, beta, y0)
    if colind.size:
        assert h.kernel() == "binned", what
    ref = O.csr_spmv(rowptr, colind, val, x, alpha, beta, y0, origin=origin)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, alpha, beta, y0, origin=origin)
    assert_within(y, ref, absref, dtype, what)
    return y, h, A


@pytest.mark.parametrize("name,kw", SHAPES, ids=[s[0] for s in SHAPES])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [1, 0])
def test_binned_shapes(J, O, name, kw, dtype, origin, monkeypatch):
    """Tiny, empty-row, one 250k-entry row (one partial per slice spans a whole
    chunk), long rows among short ones, no entries (another plan kind), dense
    rows, uniform rows."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m, n = kw["m"], kw["n"]
    rowptr, colind, val = random_csr(m, n, density=kw.get("density"), lengths=kw.get("lengths"),
                                     seed=zlib.crc32(name.encode()) % 1000 + 11, origin=origin,
                                     dtype=dtype)
    x = np.random.default_rng(5).uniform(-1, 1, n).astype(dtype)
    y0 = np.random.default_rng(6).uniform(-1, 1, m).astype(dtype)
    check(J, O, rowptr, colind, val, x, m, n, dtype, f"binned {name}", origin=origin,
          alpha=-0.75, beta=1.25, y0=y0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_binned_long_runs(J, O, dtype, monkeypatch):
    """One slice (n = 64) and 600k rows: every bin's single run holds more
    partials than the bin pass's pipelined slots (2 x 1024), so the rest of the
    run goes through its unpipelined loop; every 7th row is empty."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m, n = 600_000, 64
    rng = np.random.default_rng(21)
    lens = np.ones(m, np.int64)
    lens[::7] = 0
    lens[::13] = 5
    # Five distinct sorted columns per long row: the first five of a random
    # permutation of the 64 columns.
    five = np.sort(np.argsort(rng.random((m, n)), axis=1)[:, :5], axis=1)
    one = rng.integers(0, n, (m, 1))
    cols = [five[i] if lens[i] == 5 else one[i, :lens[i]] for i in range(m)]
    colind = (np.concatenate(cols) + 1).astype(np.int32)
    rowptr = (np.r_[0, np.cumsum(lens)] + 1).astype(np.int32)
    val = rng.uniform(-1, 1, colind.size).astype(dtype)
    x = np.random.default_rng(7).uniform(-1, 1, n).astype(dtype)
    check(J, O, rowptr, colind, val, x, m, n, dtype, "binned long runs")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("n", [300_000, 1_100_000])
def test_binned_wide_slices(J, O, dtype, n, monkeypatch):
    """x small enough for at most 128 slices of 128 KB: slices as wide as LDS
    allows, several workgroups per slice (f64 n = 300k: 19 slices of 15,808
    columns, 13 workgroups each; f32: 10 slices, 25 workgroups; n = 1.1M f64:
    68 slices, 3 workgroups; f32: 34 slices, 7 workgroups).  Rows of 0-40
    entries, alpha/beta, bit-identical on a second execute."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m = 250_000
    lens = np.random.default_rng(n % 97).integers(0, 41, m)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=n % 89, dtype=dtype)
    x = np.random.default_rng(41).uniform(-1, 1, n).astype(dtype)
    y0 = np.random.default_rng(42).uniform(-1, 1, m).astype(dtype)
    y, h, A = check(J, O, rowptr, colind, val, x, m, n, dtype, f"binned wide n={n}",
                    alpha=0.5, beta=-2.0, y0=y0)
    y2 = dev(y0)
    J.execute(h, dev(x), y2, alpha=0.5, beta=-2.0)
    np.testing.assert_array_equal(host(y2), y)


@pytest.mark.parametrize("dtype,n", [(np.float64, 2_097_152), (np.float64, 2_097_153),
                                     (np.float32, 4_194_304), (np.float32, 4_194_305)],
                         ids=["f64-128-wide", "f64-per-cu", "f32-128-wide", "f32-per-cu"])
def test_binned_geometry_switch(J, O, dtype, n, monkeypatch):
    """Both sides of the switch between wide slices and one slice per CU on a
    256-CU device: 128 slices of 128 KB (two workgroups each) at n = 2^21
    (f64) / 2^22 (f32); one column more needs 129 wide slices, more than half
    the CUs, and the plan takes ~n/256-column slices instead.  Rows of 0-40
    entries, 0-based, alpha/beta."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m = 30_000
    lens = np.random.default_rng(n % 101).integers(0, 41, m)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=n % 83, origin=0, dtype=dtype)
    x = np.random.default_rng(43).uniform(-1, 1, n).astype(dtype)
    y0 = np.random.default_rng(44).uniform(-1, 1, m).astype(dtype)
    check(J, O, rowptr, colind, val, x, m, n, dtype, f"binned geometry n={n}", origin=0,
          alpha=1.5, beta=0.25, y0=y0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_binned_many_slices_few_rows(J, O, dtype, monkeypatch):
    """300 rows over 4M columns: 256 slices, one workgroup per slice, one
    bin."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m, n = 300, 4_000_000
    lens = np.random.default_rng(8).integers(0, 3000, m)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=22, dtype=dtype)
    x = np.random.default_rng(9).uniform(-1, 1, n).astype(dtype)
    check(J, O, rowptr, colind, val, x, m, n, dtype, "binned many slices")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_binned_powerlaw_update_deterministic(J, O, dtype, monkeypatch):
    """Config 2's power-law rows at 1M x 1M: alpha/beta, bit-identical repeat,
    update_values with new values in the caller's order."""
    import torch
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    from jlust_amd import workloads as W
    cfg = W.make(2, scale=4)
    m, n = cfg["m"], cfg["n"]
    val = cfg["val"].astype(dtype)
    x = cfg["x"].astype(dtype)
    y0 = np.random.default_rng(3).uniform(-1, 1, m).astype(dtype)
    y, h, A = check(J, O, cfg["rowptr"], cfg["colind"], val, x, m, n, dtype, "binned power law",
                    alpha=1.5, beta=-0.5, y0=y0)
    y2 = dev(y0)
    J.execute(h, dev(x), y2, alpha=1.5, beta=-0.5)
    np.testing.assert_array_equal(host(y2), y)
    val2 = (val * -3.0).astype(dtype)
    J.update_values_(h, J.csr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(val2), (m, n)))
    yt = torch.empty(m, dtype=A.dtype, device="cuda")
    J.execute(h, dev(x), yt)
    ref2 = O.csr_spmv(cfg["rowptr"], cfg["colind"], val2, x)
    absref2 = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], val2, x)
    assert_within(host(yt), ref2, absref2, dtype, "binned after update_values!")


def test_binned_full_config2(J, O, monkeypatch):
    """BASELINE config 2 (4M x 4M, 64M entries, Pareto rows) through the binned
    plan, against the oracle, and bit-identical on a second execute."""
    import torch
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    from jlust_amd import workloads as W
    cfg = W.make(2)
    y, h, _ = check(J, O, cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"], cfg["m"], cfg["n"],
                    np.float64, "binned full config 2")
    y2 = torch.empty(cfg["m"], dtype=torch.float64, device="cuda")
    J.execute(h, dev(cfg["x"]), y2)
    np.testing.assert_array_equal(host(y2), y)


@pytest.mark.parametrize("dtype,n,fits", [(np.float64, 16_000_000, True),
                                          (np.float32, 33_000_000, True),
                                          (np.float64, 17_000_000, False)],
                         ids=["f64-977-slices", "f32-1008-slices", "f64-past-1024-slices"])
def test_binned_slice_count_limit(J, O, dtype, n, fits, monkeypatch):
    """Slices of at most 128 KB of x and at most 1024 of them (the bin pass
    keeps two run bounds per slice in LDS): n = 16M f64 / 33M f32 run binned
    with close to 1024 slices; n = 17M f64 needs more, and the forced request
    falls back to another layout with the same results."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m = 2000
    lens = np.random.default_rng(31).integers(0, 300, m)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=32, dtype=dtype)
    x = np.random.default_rng(33).uniform(-1, 1, n).astype(dtype)
    y, h, _ = run_binned(J, rowptr, colind, val, x, m, n)
    assert (h.kernel() == "binned") == fits, h.kernel()
    ref = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    assert_within(y, ref, absref, dtype, f"slice limit n={n}")


@pytest.mark.parametrize("mode", ["2", "1"])
def test_copied_layout_falls_back_to_merge_when_over_budget(J, O, mode, monkeypatch):
    """A plan whose copied layout (binned "2", sliced "1") with its build
    temporaries would exceed JLUST_HIP_PLAN_MAX_BYTES -- the path an
    allocation failure takes -- is built on the merge/vector kernels over the
    caller's arrays instead, with no error, and computes the same product; the
    layout is taken again once the budget allows it."""
    import torch
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", mode)
    m, n = 120000, 900000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(3).integers(4, 30, m), seed=4)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    x = np.random.default_rng(5).uniform(-1, 1, n)
    ref = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    monkeypatch.setenv("JLUST_HIP_PLAN_MAX_BYTES", str(4 << 20))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() in ("merge", "vector")
    assert h.device_bytes() < (4 << 20)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    J.execute(h, dev(x), y)
    assert_within(host(y), ref, absref, np.float64, "fallback plan")
    monkeypatch.delenv("JLUST_HIP_PLAN_MAX_BYTES")
    h2 = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h2.kernel() == {"2": "binned", "1": "sliced"}[mode]
    assert h2.device_bytes() > 12 * rowptr[-1]
    J.execute(h2, dev(x), y)
    assert_within(host(y), ref, absref, np.float64, "layout plan")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_binned_refresh_uneven_bins(J, O, dtype, monkeypatch):
    """update_values on a binned plan re-gathers the values chunk by chunk of
    consecutive CSR entries (8,192 f64 / 16,384 f32 per chunk): a bin holding
    one 300,000-entry row spans dozens of chunks, runs of empty rows leave
    bins without entries.  After the update the plan's product is
    bit-identical to a plan built on the new values (the same layout and sums)
    and within the bar of the oracle."""
    import torch
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m, n = 600_000, 2_000_000
    rng = np.random.default_rng(41)
    lens = rng.integers(0, 12, m)
    lens[100_000:260_000] = 0                     # empty bins
    lens[400_123] = 300_000                       # one bin of many chunks
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=42, dtype=dtype)
    x = rng.uniform(-1, 1, n).astype(dtype)
    y, h, A = check(J, O, rowptr, colind, val, x, m, n, dtype, "binned uneven bins")
    val2 = rng.uniform(-2, 2, val.size).astype(dtype)
    J.update_values_(h, J.csr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(val2), (m, n)))
    yt = torch.full((m,), float("nan"), dtype=A.dtype, device="cuda")
    J.execute(h, dev(x), yt)
    fresh, hf, _ = run_binned(J, rowptr, colind, val2, x, m, n)
    assert hf.kernel() == "binned"
    np.testing.assert_array_equal(host(yt), fresh)
    ref2 = O.csr_spmv(rowptr, colind, val2, x)
    absref2 = O.csr_spmv_absref(rowptr, colind, val2, x)
    assert_within(host(yt), ref2, absref2, dtype, "binned uneven bins after update_values!")
