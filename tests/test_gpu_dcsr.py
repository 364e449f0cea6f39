"""DCSR SpMV and SpMM on the GPU (the CSR kernels over the stored rows plus
row gathers/scatters, jlust_amd/csrc/dcsr.hip) against the oracle: the
reference's fixtures (test/test_emitter.jl:127-157, 230-260), rows that are
not stored left untouched for any beta, both origins, f32/f64."""
import json
import os

import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr

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
def O():
    from oracle import oracle
    return oracle


def test_reference_fixtures(J):
    c = next(c for c in GOLDEN["spmv"] if c["format"] == "DCSR")
    A = J.dcsr_tensor(dev(np.int32(c["outer_crd"])), dev(np.int32(c["inner_pos"])),
                      dev(np.int32(c["inner_crd"])), dev(np.float64(c["val"])), (c["m"], c["n"]))
    y = dev(np.zeros(3))
    J.mul_(y, A, dev(np.float64(c["x"])))
    assert host(y).tolist() == c["y"]
    s = next(c for c in GOLDEN["spmm"] if c["format"] == "DCSR")
    A = J.dcsr_tensor(dev(np.int32(s["outer_crd"])), dev(np.int32(s["inner_pos"])),
                      dev(np.int32(s["inner_crd"])), dev(np.float64(s["val"])), (s["m"], s["n"]))
    C = J.dense_matrix(3, 2, fill=0.0)
    J.mul_(C, A, dev(np.asfortranarray(np.float64(s["B"]))))
    assert host(C).tolist() == s["C"]


def random_dcsr(m, n, seed, origin, dtype):
    rng = np.random.default_rng(seed)
    lens = np.where(rng.random(m) < 0.4, 0, rng.integers(1, 12, m))
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=seed, origin=origin, dtype=dtype)
    stored = np.flatnonzero(lens)
    pos = np.concatenate([[0], np.cumsum(lens[stored])]) + origin
    return (stored + origin).astype(np.int32), pos.astype(np.int32), colind, val, rowptr


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [0, 1])
@pytest.mark.parametrize("beta", [0.0, 0.75])
def test_spmv_random(J, O, dtype, origin, beta):
    m, n = 700, 333
    outer, pos, cols, val, rowptr = random_dcsr(m, n, 5 + origin, origin, dtype)
    A = J.dcsr_tensor(dev(outer), dev(pos), dev(cols), dev(val), (m, n),
                      origin=J.OneBased() if origin else J.ZeroBased())
    rng = np.random.default_rng(9)
    xs = rng.uniform(-1, 1, n).astype(dtype)
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    y = dev(y0)
    J.execute(J.SpMVOp, A, dev(xs), y, alpha=-1.25, beta=beta)
    ref = O.dcsr_spmv(outer, pos, cols, val, xs, m, -1.25, beta, y0, origin)
    absref = O.csr_spmv_absref(rowptr, cols, val, xs, -1.25, beta, y0, origin)
    got = host(y)
    absent = np.setdiff1d(np.arange(m), outer - origin)
    assert np.array_equal(got[absent], y0[absent])               # untouched, bit for bit
    assert_within(got, ref, absref, dtype, "DCSR SpMV")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_random(J, O, dtype):
    m, n, k = 500, 260, 7
    outer, pos, cols, val, rowptr = random_dcsr(m, n, 11, 1, dtype)
    A = J.dcsr_tensor(dev(outer), dev(pos), dev(cols), dev(val), (m, n))
    rng = np.random.default_rng(12)
    B = np.asfortranarray(rng.uniform(-1, 1, (n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.uniform(-1, 1, (m, k)).astype(dtype))
    C = dev(C0)
    J.execute(J.SpMMOp, A, dev(B), C, alpha=0.5, beta=2.0)
    ref = O.dcsr_spmm(outer, pos, cols, val, B, m, 0.5, 2.0, C0, 1)
    absref = O.csr_spmm_absref(rowptr, cols, val, B, 0.5, 2.0, C0, 1)
    got = host(C)
    absent = np.setdiff1d(np.arange(m), outer - 1)
    assert np.array_equal(got[absent], C0[absent])
    assert_within(got, ref, absref, dtype, "DCSR SpMM")


def test_empty_and_prepared(J, O):
    A = J.dcsr_tensor(dev(np.zeros(0, np.int32)), dev(np.int32([1])), dev(np.zeros(0, np.int32)),
                      dev(np.zeros(0)), (4, 3))
    y = dev(np.float64([1.0, 2.0, 3.0, 4.0]))
    J.mul_(y, A, dev(np.ones(3)))
    assert host(y).tolist() == [1.0, 2.0, 3.0, 4.0]
    outer, pos, cols, val, rowptr = random_dcsr(50, 40, 3, 1, np.float64)
    A = J.dcsr_tensor(dev(outer), dev(pos), dev(cols), dev(val), (50, 40))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    xs = np.random.default_rng(1).uniform(-1, 1, 40)
    y = dev(np.zeros(50))
    J.execute(h, dev(xs), y)
    ref = O.dcsr_spmv(outer, pos, cols, val, xs, 50)
    assert_within(host(y), ref, O.csr_spmv_absref(rowptr, cols, val, xs), np.float64, "prepared")
