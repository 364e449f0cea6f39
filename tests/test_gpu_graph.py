"""HIP graph capture of the prepared and plain products: a caller may
capture execute(h, x, y) (or the plain SpMV/SpMM calls) in a torch HIP graph
and replay it.  Each graph is replayed several times with eager work and a
synchronisation between replays (inputs refilled, outputs reset), and every
replay is compared with the eager result bit for bit (the kernels are
deterministic).  The plain calls use the library's per-stream scratch buffer,
so they are warmed up on the capturing stream first (no allocation may happen
inside a capture)."""
import numpy as np
import pytest

from tests._util import dev, host, random_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


def check_replays(run, inp, out, out0, nrep=4):
    """Warm run() up on a side stream, capture it there, then replay nrep
    times; before each replay inp gets new values and out its start values;
    each replay's out must equal an eager run's."""
    import torch
    s = torch.cuda.Stream()                       # default priority
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.synchronize()
    for rep in range(nrep):
        inp.uniform_(-1.0, 1.0)
        out.copy_(out0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = host(out).copy()
        out.copy_(out0)
        run()                                     # eager, on the current stream
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, host(out), err_msg=f"replay {rep}")


@pytest.mark.parametrize("kind", ["merge", "vector", "sliced", "binned"])
def test_graph_spmv_plan(J, kind, monkeypatch):
    import torch
    if kind == "vector":
        m, n, lens = 30_000, 20_000, np.full(30_000, 12)
    else:
        m, n, lens = 30_000, 700_000, np.random.default_rng(1).integers(0, 90, 30_000)
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", {"sliced": "1", "binned": "2"}.get(kind, "0"))
    if kind == "merge":
        monkeypatch.setenv("JLUST_HIP_SPMV_VECTOR", "0")
    else:
        monkeypatch.delenv("JLUST_HIP_SPMV_VECTOR", raising=False)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=5)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() == kind
    x = torch.zeros(n, dtype=torch.float64, device="cuda")
    y = torch.zeros(m, dtype=torch.float64, device="cuda")
    y0 = dev(np.random.default_rng(2).uniform(-1, 1, m))
    check_replays(lambda: J.execute(h, x, y, alpha=1.5, beta=-0.5), x, y, y0)


@pytest.fixture()
def no_plan_cache():
    """The plain kernels themselves (repeated plain SpMV calls would switch to
    a cached plan, whose sums may differ in the last bits)."""
    from jlust_amd import hip_backend as HB
    was = HB.PLAN_CACHE.enabled
    HB.PLAN_CACHE.enabled = False
    yield
    HB.PLAN_CACHE.enabled = was


def test_graph_plain_spmv_cached_plan(J):
    """Plain SpMV calls that the plan cache has switched to a plan (three
    calls on the capturing stream first) are captured and replayed; every
    replay equals an eager call on the same stream, which runs the same
    cached plan."""
    import torch
    from jlust_amd import hip_backend as HB
    HB.PLAN_CACHE.clear()
    m, n = 20000, 300000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(8).integers(0, 60, m), seed=9)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    x = torch.zeros(n, dtype=torch.float64, device="cuda")
    y = torch.zeros(m, dtype=torch.float64, device="cuda")
    y0 = dev(np.random.default_rng(10).uniform(-1, 1, m))
    s = torch.cuda.Stream()
    run = lambda: J.execute(J.SpMVOp, A, x, y, alpha=0.5, beta=2.0)  # noqa: E731
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(4):
            run()
    torch.cuda.synchronize()
    assert len(HB.PLAN_CACHE.info()) == 1
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.synchronize()
    for rep in range(4):
        x.uniform_(-1.0, 1.0)
        y.copy_(y0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = host(y).copy()
        y.copy_(y0)
        with torch.cuda.stream(s):
            run()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, host(y), err_msg=f"replay {rep}")
    HB.PLAN_CACHE.clear()


def test_graph_plain_spmv_and_spmm(J, no_plan_cache):
    import torch
    m, n, k = 5000, 4000, 24
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(3).integers(0, 40, m),
                                     seed=6, dtype=np.float32)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    x = torch.zeros(n, dtype=torch.float32, device="cuda")
    y = torch.zeros(m, dtype=torch.float32, device="cuda")
    check_replays(lambda: J.execute(J.SpMVOp, A, x, y), x, y, torch.zeros_like(y))
    B = J.dense_matrix(n, k, dtype=torch.float32)
    C = J.dense_matrix(m, k, dtype=torch.float32)
    C0 = torch.randn(k, m, device="cuda").t()
    check_replays(lambda: J.execute(J.SpMMOp, A, B, C, alpha=2.0, beta=0.5), B, C, C0)


@pytest.mark.parametrize("kind", ["merge", "vector", "sliced", "binned"])
def test_plan_capture_launch(J, kind, monkeypatch):
    """jlust_hip_csr_spmv_plan_capture_* / spmv_graph_launch: each launch
    equals execute(h, x, y) bit for bit with the inputs as they are at launch
    (new x, y read through beta, new values stored in place); a launch onto a
    stream that is itself being captured launches nothing and reports it."""
    import torch
    if kind == "vector":
        m, n, lens = 20_000, 15_000, np.full(20_000, 10)
    else:
        m, n, lens = 20_000, 700_000, np.random.default_rng(7).integers(0, 80, 20_000)
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", {"sliced": "1", "binned": "2"}.get(kind, "0"))
    if kind == "merge":
        monkeypatch.setenv("JLUST_HIP_SPMV_VECTOR", "0")
    else:
        monkeypatch.delenv("JLUST_HIP_SPMV_VECTOR", raising=False)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=8)
    v = dev(val)
    A = J.csr_tensor(dev(rowptr), dev(colind), v, (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() == kind
    x = torch.empty(n, dtype=torch.float64, device="cuda")
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    ye = torch.empty(m, dtype=torch.float64, device="cuda")
    y0 = dev(np.random.default_rng(9).uniform(-1, 1, m))
    g = h.capture(x, y, alpha=-2.0, beta=0.75)
    for rep in range(4):
        x.uniform_(-1.0, 1.0)
        if rep == 2:                        # new values in the same buffer
            v.copy_(dev(np.random.default_rng(10).uniform(-1, 1, v.numel())))
            J.update_values_(h, A)
        y.copy_(y0)
        assert g.launch()
        ye.copy_(y0)
        J.execute(h, x, ye, alpha=-2.0, beta=0.75)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(y), host(ye), err_msg=f"launch {rep}")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    outer = torch.cuda.CUDAGraph()
    with torch.cuda.graph(outer, stream=s):
        launched = g.launch()
    assert launched is False
    with pytest.raises(J.IncompatibleExtents):
        h.capture(x[:-1], y)
    del g
    torch.cuda.synchronize()


def test_graph_spmm_plan_with_split_rows(J):
    """The prepared CSR SpMM plan (rows longer than 1024 entries split into
    segments, their partial rows reduced by a third kernel) captured and
    replayed: the plan's execute allocates nothing and synchronises nothing."""
    import torch
    m, n, k = 3000, 6000, 24
    lens = np.random.default_rng(11).integers(0, 30, m)
    lens[[5, 777, 2999]] = [5000, 2500, 1100]
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=12)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    assert h.info()["split_rows"] == 3
    B = J.dense_matrix(n, k, dtype=torch.float64)
    C = J.dense_matrix(m, k, dtype=torch.float64)
    C0 = torch.randn(k, m, dtype=torch.float64, device="cuda").t()
    check_replays(lambda: J.execute(J.SpMMOp, h, B, C, alpha=1.25, beta=-0.5), B, C, C0)


@pytest.mark.parametrize("mask", ["csr", "coo_unsorted"])
def test_graph_sddmm_plan(J, mask):
    import torch
    m, n, K = 2000, 1500, 40
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(13).integers(0, 25, m),
                                     seed=14, dtype=np.float32)
    out = dev(val.copy())
    if mask == "csr":
        Cs = J.csr_tensor(dev(rowptr), dev(colind), out, (m, n))
    else:
        rows = np.repeat(np.arange(m, dtype=np.int32), np.diff(rowptr)) + 1
        perm = np.random.default_rng(15).permutation(rows.size)
        out = dev(val[perm].copy())
        Cs = J.coo_tensor(dev(rows[perm]), dev(colind[perm]), out, (m, n))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
    A = torch.zeros(K, m, dtype=torch.float32, device="cuda").t()
    Bm = torch.randn(n, K, dtype=torch.float32, device="cuda").t()
    c0 = out.clone()
    check_replays(lambda: J.execute(J.SDDMMOp, h, A, Bm, Cs, alpha=0.5, beta=2.0), A, out, c0)


@pytest.mark.parametrize("b1,b2,dtype", [(16, 16, np.float32), (4, 8, np.float64)])
def test_graph_bsr_plan(J, b1, b2, dtype):
    """The prepared BSR SpMM plan on both of its paths (MFMA kernels; CSR
    expansion + CSR SpMM plan) captured and replayed."""
    import torch
    mb, nb, k = 60, 50, 32
    rng = np.random.default_rng(16)
    counts = rng.integers(0, 6, mb)
    bcols = [np.sort(rng.choice(nb, c, replace=False)) for c in counts]
    bp = (np.r_[0, np.cumsum(counts)] + 1).astype(np.int32)
    bc = (np.concatenate(bcols) + 1).astype(np.int32)
    vals = rng.standard_normal(bc.size * b1 * b2).astype(dtype)
    A = J.bsr_tensor(dev(bp), dev(bc), dev(vals), (mb * b1, nb * b2), (b1, b2))
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    assert h.info()["path"] == ("mfma" if b1 == 16 and dtype == np.float32 else "csr_expansion")
    tdt = torch.float64 if dtype == np.float64 else torch.float32
    B = J.dense_matrix(nb * b2, k, dtype=tdt)
    C = J.dense_matrix(mb * b1, k, dtype=tdt)
    C0 = torch.randn(k, mb * b1, dtype=tdt, device="cuda").t()
    check_replays(lambda: J.execute(J.SpMMOp, h, B, C, alpha=0.75, beta=1.5), B, C, C0)
