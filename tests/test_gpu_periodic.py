"""PeriodicCSR (src/named_formats.jl:63-88, periodic_csr_tensor src/interop.jl:
183-212): SpMV of kron(I(T), block) on the GPU (one CSR SpMM of the block
over the T column blocks of x) against the oracle's CSR SpMV of the
explicitly replicated matrix."""
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


def replicate(rowptr, colind, val, br, nc, T, origin):
    """kron(I(T), block) as a CSR with the same origin."""
    nnz = val.size
    rp = (rowptr - origin).astype(np.int64)
    out_rp = np.concatenate([[0]] + [rp[1:] + t * nnz for t in range(T)]) + origin
    out_ci = np.concatenate([colind + t * nc for t in range(T)])
    return out_rp.astype(np.int32), out_ci.astype(np.int32), np.tile(val, T)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("T", [1, 5, 24, 40])
@pytest.mark.parametrize("origin", [0, 1])
def test_periodic_spmv(J, O, dtype, T, origin):
    br, nc = 37, 29
    rowptr, colind, val = random_csr(br, nc, density=0.2, seed=T + origin, origin=origin, dtype=dtype)
    blk = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (br, nc),
                       origin=J.OneBased() if origin else J.ZeroBased())
    P = J.periodic_csr_tensor(blk, T)
    assert J.size(P) == (T * br, T * nc) and J.nnz(P) == val.size
    rng = np.random.default_rng(T)
    xs = rng.uniform(-1, 1, T * nc).astype(dtype)
    y0 = rng.uniform(-1, 1, T * br).astype(dtype)
    y = dev(y0)
    J.mul_(y, P, dev(xs), 0.5, 2.0)
    rp, ci, v = replicate(rowptr, colind, val, br, nc, T, origin)
    ref = O.csr_spmv(rp, ci, v, xs, 0.5, 2.0, y0, origin)
    absref = O.csr_spmv_absref(rp, ci, v, xs, 0.5, 2.0, y0, origin)
    assert_within(host(y), ref, absref, dtype, f"PeriodicCSR T={T}")
    assert host(J.matmul(P, dev(xs))).shape == (T * br,)


def test_periodic_requires_csr(J):
    import torch
    coo = J.coo_tensor(dev(np.int32([1])), dev(np.int32([1])), dev(np.ones(1)), (2, 2))
    with pytest.raises(J.UnsupportedFormat):
        J.periodic_csr_tensor(coo, 3)
    d1 = J.Formats.DensedRight(1)
    assert J.supports_backend(J.HIPBackend(), J.SpMVOp(J.Formats.PeriodicCSR(3, 2, 2), d1, d1))
    assert J.Formats.PeriodicCSR(3, 2, 2) == J.Formats.PeriodicCSR(3, 2, 2)
    assert J.Formats.PeriodicCSR(3, 2, 2) != J.Formats.PeriodicCSR(4, 2, 2)
    del torch
