"""jlust_hip_csr_spmv_f64_i32_noalloc: the plain CSR SpMV call with its carry
slots in the library's static device array instead of the per-stream scratch
buffer.  Called through the C ABI and compared with jlust_hip_csr_spmv_f64_i32
(same kernels and grid, so bit for bit) and with the oracle (1e-12 *
|alpha||A||x| + |beta||y0|), on two calls in a row, the second smaller, so
the second reads nothing the first left in the shared array."""
import ctypes

import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from jlust_amd import _lib
    return _lib.lib()


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def _call(L, entry, m, n, rowptr, colind, val, x, y, alpha, beta):
    import torch
    from jlust_amd import _lib
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = getattr(L, entry)(m, n, colind.numel(), 1, rowptr.data_ptr(),
                           colind.data_ptr() if colind.numel() else None,
                           val.data_ptr() if val.numel() else None, alpha, x.data_ptr(), beta,
                           y.data_ptr(), s)
    assert st == 0, f"{entry}: status {st}: {_lib.last_error()}"


def _case(L, O, m, n, lengths, seed, alpha, beta):
    import torch
    rowptr, colind, val = random_csr(m, n, lengths=lengths, seed=seed)
    rng = np.random.default_rng(seed + 1)
    x = rng.uniform(-1, 1, n)
    y0 = rng.uniform(-1, 1, m)
    rp, ci, va, xd = dev(rowptr), dev(colind), dev(val), dev(x)
    y_ref = dev(y0)
    y_new = dev(y0)
    _call(L, "jlust_hip_csr_spmv_f64_i32", m, n, rp, ci, va, xd, y_ref, alpha, beta)
    _call(L, "jlust_hip_csr_spmv_f64_i32_noalloc", m, n, rp, ci, va, xd, y_new, alpha, beta)
    torch.cuda.synchronize()
    got, want = host(y_new), host(y_ref)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), \
        f"m={m}: noalloc differs from the plain entry point"
    ref = O.csr_spmv(rowptr, colind, val, x, alpha, beta, y0)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, alpha, beta, y0)
    assert_within(got, ref, absref, np.float64, f"noalloc m={m}")


def test_noalloc_matches_plain_call_twice(L, O):
    rng = np.random.default_rng(0)
    # First call: many blocks (long rows mixed with empty ones); second: smaller.
    big = rng.integers(0, 40, 60000)
    big[::997] = 3000
    print("noalloc case 1: m=60000", flush=True)
    _case(L, O, 60000, 80000, big, 1, 1.25, 0.0)
    print("noalloc case 2: m=700", flush=True)
    _case(L, O, 700, 900, rng.integers(0, 12, 700), 2, -0.5, 0.75)


def test_noalloc_power_law_rows(L, O):
    rng = np.random.default_rng(3)
    lens = np.minimum((rng.pareto(1.8, 200000) + 1) * 6, 20000).astype(np.int64)
    print("noalloc case 3: power-law m=200000", flush=True)
    _case(L, O, 200000, 200000, lens, 4, 1.0, 0.0)
    print("noalloc case 4: m=5", flush=True)
    _case(L, O, 5, 7, np.array([0, 3, 7, 1, 0]), 5, 2.0, -1.0)


def test_noalloc_rejects_bad_arguments(L):
    import torch
    from jlust_amd import _lib
    y = torch.zeros(4, dtype=torch.float64, device="cuda")
    st = L.jlust_hip_csr_spmv_f64_i32_noalloc(4, 4, 0, 2, y.data_ptr(), None, None, 1.0,
                                              y.data_ptr(), 0.0, y.data_ptr(), None)
    assert st == 5, _lib.last_error()            # origin 2
    st = L.jlust_hip_csr_spmv_f64_i32_noalloc(-1, 4, 0, 1, y.data_ptr(), None, None, 1.0,
                                              y.data_ptr(), 0.0, y.data_ptr(), None)
    assert st == 1, _lib.last_error()
