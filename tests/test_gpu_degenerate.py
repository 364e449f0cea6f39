"""Degenerate shapes through the operator API: no columns (SpMM k = 0, SDDMM
K = 0: the dot products are empty sums), no rows, and a matrix without
entries.  Each follows the definition: an empty sum is 0, so the output is
beta*C (or untouched when there is nothing to write)."""
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


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_k0_is_beta_c(J, dtype):
    import torch
    m, n = 300, 200
    rowptr, colind, _ = random_csr(m, n, density=0.05, seed=1, dtype=dtype)
    c0 = np.random.default_rng(2).standard_normal(colind.size).astype(dtype)
    out = dev(c0)
    Cs = J.csr_tensor(dev(rowptr), dev(colind), out, (m, n))
    A = torch.empty((0, m), dtype=out.dtype, device="cuda").t()    # m x 0
    B = torch.empty((n, 0), dtype=out.dtype, device="cuda").t()    # 0 x n
    J.execute(J.SDDMMOp, A, B, Cs, alpha=3.0, beta=0.5)
    np.testing.assert_array_equal(host(out), (dtype(0.5) * c0).astype(dtype))


def test_spmm_k0_and_empty_rows(J):
    import torch
    m, n = 300, 200
    rowptr, colind, val = random_csr(m, n, density=0.05, seed=3)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    B = J.dense_matrix(n, 0)
    C = J.dense_matrix(m, 0)
    J.execute(J.SpMMOp, A, B, C)                                   # nothing to write
    assert C.shape == (m, 0)
    E = J.csr_tensor(dev(np.ones(m + 1, np.int32)), dev(np.zeros(0, np.int32)),
                     dev(np.zeros(0)), (m, n))                       # no entries
    B = J.dense_matrix(n, 5, fill=1.0)
    C0 = np.asfortranarray(np.random.default_rng(4).standard_normal((m, 5)))
    C = dev(C0)
    J.execute(J.SpMMOp, E, B, C, alpha=2.0, beta=-1.0)
    np.testing.assert_array_equal(host(C), -C0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmv_no_columns_and_no_entries(J, dtype):
    import torch
    m = 257
    y0 = np.random.default_rng(5).standard_normal(m).astype(dtype)
    E = J.csr_tensor(dev(np.ones(m + 1, np.int32)), dev(np.zeros(0, np.int32)),
                     dev(np.zeros(0, dtype)), (m, 0))                # m x 0
    y = dev(y0)
    J.execute(J.SpMVOp, E, torch.empty(0, dtype=y.dtype, device="cuda"), y, beta=2.0)
    np.testing.assert_array_equal(host(y), (dtype(2) * y0).astype(dtype))
    y = dev(y0)
    J.execute(J.SpMVOp, E, torch.empty(0, dtype=y.dtype, device="cuda"), y)
    np.testing.assert_array_equal(host(y), np.zeros(m, dtype))
    Z = J.csr_tensor(dev(np.ones(1, np.int32)), dev(np.zeros(0, np.int32)),
                     dev(np.zeros(0, dtype)), (0, 10))               # 0 x 10
    J.execute(J.SpMVOp, Z, dev(np.ones(10, dtype)), torch.empty(0, dtype=y.dtype, device="cuda"))
