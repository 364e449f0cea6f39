"""Prepared plans give their device memory back.

Every plan kind (the SpMV layouts -- row order, XCD slices, LDS bins, COO --
and the SpMM, SDDMM and BSR plans) owns device allocations made with the HIP
runtime, outside torch's caching allocator.  Creating, executing and dropping
each of them 20 times must leave the device's free memory where it was after
the first round (the first round may grow the library's per-stream scratch,
which it keeps by design)."""
import gc

import numpy as np
import pytest

from tests._util import dev, random_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


def _free_bytes():
    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.cuda.mem_get_info()[0]


def test_plans_release_their_memory(J, monkeypatch):
    import torch
    m, n, k, K = 300000, 250000, 32, 16
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(80).integers(0, 20, m), seed=81)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    Ac = J.coo_tensor(dev(rows[::-1].copy()), dev(colind[::-1].copy()), dev(val[::-1].copy()), (m, n))
    x = torch.rand(n, dtype=torch.float64, device="cuda")
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    B = J.dense_matrix(n, k, fill=1.0)
    C = J.dense_matrix(m, k)
    Am, Bm = J.dense_matrix(m, K, fill=0.5), J.dense_matrix(K, n, fill=0.25)
    cv = torch.zeros(colind.size, dtype=torch.float64, device="cuda")
    Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n))
    mb, nb = 2000, 2000
    bp = (np.arange(mb + 1) * 4 + 1).astype(np.int32)
    bc = (np.tile(np.arange(4), mb) + np.repeat(np.arange(mb) // 2, 4)).astype(np.int32) % nb + 1
    bc = np.sort(bc.reshape(mb, 4), axis=1).reshape(-1)
    Ab = J.bsr_tensor(dev(bp), dev(bc), torch.rand(bc.size * 256, device="cuda"), (mb * 16, nb * 16))
    Bb, Cb = J.dense_matrix(nb * 16, k, dtype=torch.float32, fill=1.0), J.dense_matrix(mb * 16, k, dtype=torch.float32)

    def one_round():
        for layout in ("0", "1", "2"):
            monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", layout)
            h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
            J.execute(h, x, y)
            del h
        monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)
        h = J.prepare(J.HIPBackend(), J.SpMVOp, Ac)
        J.execute(h, x, y)
        h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
        J.execute(h, B, C)
        h = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
        J.execute(J.SDDMMOp, h, Am, Bm, Cs)
        h = J.prepare(J.HIPBackend(), J.SpMMOp, Ab, n_cols=k)
        J.execute(h, Bb, Cb)
        del h

    one_round()
    base = _free_bytes()
    for _ in range(20):
        one_round()
    after = _free_bytes()
    # Allocation granularity and driver bookkeeping allow a little drift; one
    # leaked binned plan alone would hold tens of MB here.
    assert base - after < 16 * 2**20, f"free device memory fell by {(base - after) / 2**20:.1f} MiB"
