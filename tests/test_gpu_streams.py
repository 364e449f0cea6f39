"""Plain calls on two streams at once.

The plain SpMV call keeps its block carries, and the plain SpMM call its
row-major copy of B, in library scratch held per (device, stream).  Two
streams of default priority each get a queue of calls on their own operands,
enqueued alternately so the kernels overlap on the device.  Every result is
checked against the oracle."""
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


def _matrix(seed, m, n):
    rng = np.random.default_rng(seed)
    lens = np.minimum((rng.pareto(1.6, m) + 1) * 4, n).astype(np.int64)
    return random_csr(m, n, lengths=lens, seed=seed)


def test_spmv_two_streams(J, O):
    import torch
    mats = [_matrix(70, 120000, 90000), _matrix(71, 80000, 150000)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]        # default priority
    rng = np.random.default_rng(72)
    A, xs, ys, refs = [], [], [], []
    for (rowptr, colind, val), (m, n) in zip(mats, [(120000, 90000), (80000, 150000)]):
        A.append(J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n)))
        x = [rng.uniform(-1, 1, n) for _ in range(6)]
        xs.append([dev(v) for v in x])
        ys.append([torch.full((m,), float("nan"), dtype=torch.float64, device="cuda") for _ in x])
        refs.append([(O.csr_spmv(rowptr, colind, val, v), O.csr_spmv_absref(rowptr, colind, val, v))
                     for v in x])
    torch.cuda.synchronize()
    for i in range(6):
        for s in range(2):
            with torch.cuda.stream(streams[s]):
                J.execute(J.SpMVOp, A[s], xs[s][i], ys[s][i])
    torch.cuda.synchronize()
    for s in range(2):
        for i in range(6):
            ref, absref = refs[s][i]
            assert_within(host(ys[s][i]), ref, absref, np.float64, f"stream {s} call {i}")


def test_spmm_two_streams(J, O):
    import torch
    mats = [_matrix(73, 60000, 50000), _matrix(74, 40000, 70000)]
    dims = [(60000, 50000, 48), (40000, 70000, 96)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    rng = np.random.default_rng(75)
    A, Bs, Cs, refs = [], [], [], []
    for (rowptr, colind, val), (m, n, k) in zip(mats, dims):
        A.append(J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n)))
        B = [np.asfortranarray(rng.uniform(-1, 1, (n, k))) for _ in range(3)]
        Bs.append([dev(b) for b in B])
        Cs.append([J.dense_matrix(m, k, fill=float("nan")) for _ in B])
        refs.append([(O.csr_spmm(rowptr, colind, val, b)[0], O.csr_spmm_absref(rowptr, colind, val, b))
                     for b in B])
    torch.cuda.synchronize()
    for i in range(3):
        for s in range(2):
            with torch.cuda.stream(streams[s]):
                J.execute(J.SpMMOp, A[s], Bs[s][i], Cs[s][i])
    torch.cuda.synchronize()
    for s in range(2):
        for i in range(3):
            ref, absref = refs[s][i]
            assert_within(host(Cs[s][i]), ref, absref, np.float64, f"stream {s} call {i}")


@pytest.mark.parametrize("kind", ["binned", "coo"])
def test_update_values_is_stream_ordered(J, O, kind, monkeypatch):
    """update_values_ on a plan that copies its values (the LDS-binned layout;
    a COO plan whose entries were reordered) is enqueued on the caller's
    stream (jlust_hip_csr_spmv_plan_update_values takes the stream): it returns
    at once and its work, and a product after it, complete while long work
    queued before it on another stream is still running.  The product then
    sees the new values (parity against the oracle)."""
    import time

    import torch
    if kind == "binned":
        monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "2")
    m, n = 200000, 150000
    rowptr, colind, val = random_csr(m, n, lengths=np.full(m, 12), seed=76)
    if kind == "coo":
        rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
        p = np.random.default_rng(77).permutation(rows.size)
        rows, cols, v0 = rows[p], colind[p], val[p]
        A = J.coo_tensor(dev(rows), dev(cols), dev(v0), (m, n))
    else:
        A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    if kind == "binned":
        assert h.kernel() == "binned"
    rng = np.random.default_rng(78)
    x = rng.uniform(-1, 1, n)
    newval = rng.uniform(-1, 1, val.size)
    A2 = J.USTensor(A.extents, A.format, A.pos_buffers, A.crd_buffers, dev(newval), None, A.origin)
    xd = dev(x)
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda")
    big = torch.randn(8192, 8192, device="cuda")
    out = torch.empty_like(big)
    sA, sB = torch.cuda.Stream(), torch.cuda.Stream()        # default priority
    torch.cuda.synchronize()
    with torch.cuda.stream(sB):
        for _ in range(60):
            torch.mm(big, big, out=out)
    t0 = time.perf_counter()
    with torch.cuda.stream(sA):
        J.update_values_(h, A2)
        J.execute(h, xd, y)
        done = torch.cuda.Event()
        done.record(sA)
    host_s = time.perf_counter() - t0
    done.synchronize()
    b_running = not sB.query()
    torch.cuda.synchronize()
    assert b_running, "the update and product waited for the other stream's queued work"
    assert host_s < 0.05, f"update_values_ + execute took {host_s * 1e3:.1f} ms on the host"
    if kind == "coo":
        r0 = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))[p]
        ref = O.coo_spmv(r0, cols, newval, x, m)
        absref = O.csr_spmv_absref(rowptr, colind, np.abs(newval[np.argsort(p)]), np.abs(x))
    else:
        ref = O.csr_spmv(rowptr, colind, newval, x)
        absref = O.csr_spmv_absref(rowptr, colind, newval, x)
    assert_within(host(y), ref, absref, np.float64, f"{kind} plan after a stream-ordered update")
