"""Full-size parity of BASELINE configs 1, 3, 4 and 5 on the paths bench.py
times, against the CPU oracle on the same seeded inputs.

- Config 1: the prepared plan (bench.py's step, execute(h, x, y)), whose
  choice at this shape is the vector kernel with computed row bounds; every
  row.
- Config 3: the plain SpMM call (bench.py's step), every output (all rows,
  all 128 columns), plus the prepared plan bit for bit against the plain
  call.
- Config 4: every one of the 16M masked outputs.
- Config 5: every output (all rows, all 256 columns, in chunks of 32).
(Config 2 is checked on every row through the plain call and the binned plan
in test_gpu_spmv.py / test_gpu_spmv_binned.py.)

Bar: |out - ref| <= 1e-12 (fp64) / 1e-5 (fp32) x (|A| |B|) elementwise.
"""
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


@pytest.fixture(scope="module")
def W():
    from jlust_amd import workloads
    return workloads


def test_config1_full_through_prepared_plan(J, O, W):
    import torch
    cfg = W.make(1)
    m, n = cfg["m"], cfg["n"]
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert h.kernel() == "vector"
    y = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda")
    J.execute(h, dev(cfg["x"]), y)
    ref = O.csr_spmv(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    absref = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    assert_within(host(y), ref, absref, np.float64, cfg["name"] + " (plan, every row)")


def test_config3_every_output(J, O, W):
    import torch
    cfg = W.make(3)
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
    B = dev(cfg["B"])
    C = J.dense_matrix(m, k, dtype=torch.float32, fill=float("nan"))
    J.execute(J.SpMMOp, A, B, C)
    got = host(C)
    ref, _ = O.csr_spmm(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"])
    absref = O.csr_spmm_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"])
    assert_within(got, ref, absref, np.float32, cfg["name"] + " (every output)")
    del ref, absref
    # The prepared plan runs the same kernels here (no row is long): all of C
    # bit for bit.
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    assert h.info()["split_rows"] == 0
    C2 = J.dense_matrix(m, k, dtype=torch.float32, fill=float("nan"))
    J.execute(h, B, C2)
    assert np.array_equal(host(C2).view(np.uint32), got.view(np.uint32))


def test_config4_every_output(J, O, W):
    import torch
    cfg = W.make(4)
    m, n = cfg["m"], cfg["n"]
    S = dev(cfg["mask"])
    out = torch.full_like(S, float("nan"))
    Cs = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), out, (m, n))
    J.execute(J.SDDMMOp, dev(cfg["A"]), dev(cfg["B"]), Cs, mask=S)
    ref = O.csr_sddmm(cfg["rowptr"], cfg["colind"], cfg["A"], cfg["B"], mask=cfg["mask"])
    absref = O.csr_sddmm_absref(cfg["rowptr"], cfg["colind"], cfg["A"], cfg["B"], mask=cfg["mask"])
    assert_within(host(out), ref, absref, np.float32, cfg["name"] + " (every output)")


def test_config5_every_output(J, O, W):
    """Config 5 on every output: all 1M rows and all 256 columns, checked in
    column chunks of 32 against the oracle's CSR expansion of the blocks
    (computed once) and its CSR SpMM, to bound host memory."""
    import torch
    cfg = W.make(5)
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    A = J.bsr_tensor(dev(cfg["browptr"]), dev(cfg["bcolind"]), dev(cfg["val"]), (m, n))
    C = J.dense_matrix(m, k, dtype=torch.float32, fill=float("nan"))
    J.execute(J.SpMMOp, A, dev(cfg["B"]), C)
    got = host(C)
    del C
    assert np.isfinite(got).all()
    rp, ci, v = O.bsr_to_csr(cfg["browptr"], cfg["bcolind"], cfg["val"], 16)
    for c0 in range(0, k, 32):
        Bs = np.asfortranarray(cfg["B"][:, c0:c0 + 32])
        ref, _ = O.csr_spmm(rp, ci, v, Bs)
        absref = O.csr_spmm_absref(rp, ci, v, Bs)
        assert_within(got[:, c0:c0 + 32], ref, absref, np.float32,
                      cfg["name"] + f" (every row, columns {c0}..{c0 + 31})")
        del ref, absref
