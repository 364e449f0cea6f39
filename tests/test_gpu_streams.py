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
