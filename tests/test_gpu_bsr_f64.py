"""GPU parity of the fp64 16 x 16 BSR SpMM (v_mfma_f64_16x16x4_f64 kernel,
jlust_hip_bsr_spmm_f64_i32) against the CPU oracle, which expands the BSR
matrix to CSR bit-exactly and runs the CSR SpMM.  Bar: |C - C_ref| <=
1e-12 x (|alpha||A||B| + |beta||C0|) elementwise; integer-valued cases are
compared bit for bit."""
import numpy as np
import pytest

from tests._util import assert_within, dev, host
from tests.test_gpu_bsr import dense_of_bsr, random_bsr

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


def _bsr64(J, browptr, bcolind, val, mb, nb, origin=1, row_major=True):
    return J.bsr_tensor(dev(browptr), dev(bcolind), dev(val), (mb * 16, nb * 16), (16, 16),
                        row_major_blocks=row_major,
                        origin=J.OneBased() if origin == 1 else J.ZeroBased())


def _run(J, A, B, C0=None, alpha=1.0, beta=0.0):
    import torch
    k = B.shape[1]
    if C0 is None:
        C = J.dense_matrix(A.extents[0], k, dtype=torch.float64, fill=float("nan"))
    else:
        C = dev(np.asfortranarray(C0))
    J.execute(J.SpMMOp, A, dev(np.asfortranarray(B)), C, alpha=alpha, beta=beta)
    return host(C)


def _check(O, C, browptr, bcolind, val, B, alpha, beta, C0, what, origin=1, row_major=True):
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, alpha, beta, C0, origin=origin,
                     row_major_blocks=row_major)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16, origin=origin, row_major_blocks=row_major)
    absref = O.csr_spmm_absref(rp, ci, v, B, alpha, beta, C0, origin=origin)
    assert_within(C, ref, absref, np.float64, what)


@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_f64_single_block_exact_layout(J, row_major):
    """One block whose entries make any operand-layout mix-up (row/column
    swap, contraction-group order, output row groups) change the result;
    small integers, so every product and sum is exact."""
    browptr = np.array([1, 2], np.int32)
    bcolind = np.array([1], np.int32)
    blk = (np.arange(256) % 7 - 3).astype(np.float64)          # V[r][s] = blk[16r+s]
    val = blk if row_major else blk.reshape(16, 16).T.reshape(-1).copy()
    B = np.asfortranarray((np.arange(16 * 48) % 5 - 2).astype(np.float64).reshape(16, 48))
    C = _run(J, _bsr64(J, browptr, bcolind, val, 1, 1, row_major=row_major), B)
    np.testing.assert_array_equal(C, blk.reshape(16, 16) @ B)


@pytest.mark.parametrize("k", [1, 16, 40, 256, 300])
@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_f64_random(J, O, k, row_major):
    """Random blocks, k across the 16-column tiles and the 256-column passes,
    alpha/beta; also against the dense product."""
    mb, nb = 37, 29
    browptr, bcolind, val32 = random_bsr(mb, nb, 5, seed=k + 7)
    val = val32.astype(np.float64)
    rng = np.random.default_rng(k)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k)))
    C = _run(J, _bsr64(J, browptr, bcolind, val, mb, nb, row_major=row_major), B, C0, 1.25, -0.5)
    _check(O, C, browptr, bcolind, val, B, 1.25, -0.5, C0, f"bsr f64 k={k}", row_major=row_major)
    D = dense_of_bsr(browptr, bcolind, val, mb, nb, row_major=row_major)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16, row_major_blocks=row_major)
    absref = O.csr_spmm_absref(rp, ci, v, B, 1.25, -0.5, C0)
    assert_within(C, 1.25 * (D @ B) - 0.5 * C0, absref, np.float64, "bsr f64 vs dense")


def test_bsr_f64_zero_based_long_and_empty_rows(J, O):
    """ZeroBased, BSRLeft, block-rows of 0 to 12 blocks (beyond the fp32
    kernels' 8-block register chunk) with empty ones, beta = 0 and beta != 0."""
    mb, nb, k = 40, 40, 48
    rng = np.random.default_rng(3)
    counts = rng.integers(0, 13, mb)
    counts[::5] = 0
    bcols = [np.sort(rng.choice(nb, c, replace=False)) for c in counts]
    browptr = np.r_[0, np.cumsum(counts)].astype(np.int32)
    bcolind = np.concatenate(bcols).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256)
    A = _bsr64(J, browptr, bcolind, val, mb, nb, origin=0, row_major=False)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k)))
    for beta in (0.0, 0.75):
        C = _run(J, A, B, C0 if beta else None, 2.0, beta)
        _check(O, C, browptr, bcolind, val, B, 2.0, beta, C0 if beta else None,
               f"BSRLeft ZeroBased beta={beta}", origin=0, row_major=False)


def test_bsr_f64_unaligned_operands(J, O):
    """ldb and ldc not multiples of 4 and block values at an odd offset (8-byte
    aligned only): the element-access kernel."""
    import torch
    mb, nb, k = 9, 11, 24
    browptr, bcolind, val32 = random_bsr(mb, nb, 3, seed=21)
    val = val32.astype(np.float64)
    vbuf = dev(np.r_[0.0, val])
    vview = vbuf[1:]
    assert vview.data_ptr() % 32 != 0
    A = J.bsr_tensor(dev(browptr), dev(bcolind), vview, (mb * 16, nb * 16), (16, 16))
    Bbig = np.asfortranarray(np.random.default_rng(7).standard_normal((nb * 16 + 1, k)))
    Bd = dev(Bbig)[: nb * 16]
    Cbig = torch.full((k, mb * 16 + 3), float("nan"), dtype=torch.float64, device="cuda").t()
    Cd = Cbig[: mb * 16]
    from jlust_amd.tensor import leading_dim
    assert leading_dim(Bd) == nb * 16 + 1 and leading_dim(Cd) == mb * 16 + 3
    J.execute(J.SpMMOp, A, Bd, Cd)
    _check(O, host(Cd), browptr, bcolind, val, np.asfortranarray(Bbig[: nb * 16]), 1.0, 0.0, None,
           "unaligned f64 operands")


def test_bsr_f64_banded_scaled(J, O):
    """Config 5's banded pattern at 1/32 scale (2,048 block-rows, 8 blocks
    within +-32, k = 256) in Float64."""
    from jlust_amd import workloads as W
    cfg = W.make(5, scale=32)
    val = cfg["val"].astype(np.float64)
    B = np.asfortranarray(cfg["B"].astype(np.float64))
    A = _bsr64(J, cfg["browptr"], cfg["bcolind"], val, cfg["mb"], cfg["nb"])
    C = _run(J, A, B)
    _check(O, C, cfg["browptr"], cfg["bcolind"], val, B, 1.0, 0.0, None, cfg["name"] + " f64 /32")


@pytest.mark.parametrize("beta", [0.0, -0.5])
@pytest.mark.parametrize("strip", ["1", "0"])
def test_bsr_f64_strip_paths(J, O, beta, strip, monkeypatch):
    """Row-major aligned Float64 blocks run the strip kernel (LDS windows of
    B); a strip whose rows hold more than 8 blocks, or whose window spans more
    than 76 block-rows, computes with direct operand loads; a banded strip
    uses the window.  Every kind of strip in one matrix, k not a multiple of
    16, against the oracle; JLUST_HIP_BSR_STRIP=0 runs the per-row kernel on
    the same input."""
    monkeypatch.setenv("JLUST_HIP_BSR_STRIP", strip)
    mb, nb, k = 60, 200, 40
    rng = np.random.default_rng(11)
    bcols = []
    for R in range(mb):
        if R < 12:                                   # long rows: up to 12 blocks
            c = rng.choice(nb, int(rng.integers(6, 13)), replace=False)
        elif R < 24:                                 # a window wider than 76 block-rows
            c = rng.choice(nb, 5, replace=False)
        elif R % 7 == 0:
            c = np.zeros(0, np.int64)                # empty rows inside banded strips
        else:                                        # banded: within +-10 of the diagonal
            lo, hi = max(0, R - 10), min(nb, R + 11)
            c = rng.choice(np.arange(lo, hi), 6, replace=False)
        bcols.append(np.sort(c))
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcols) + 1).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256)
    A = _bsr64(J, browptr, bcolind, val, mb, nb)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k))) if beta else None
    C = _run(J, A, B, C0, 1.5, beta)
    _check(O, C, browptr, bcolind, val, B, 1.5, beta, C0, f"f64 strip paths (strip={strip})")


def test_bsr_f64_banded_quarter_every_output(J, O):
    """Config 5's banded pattern at 1/4 scale (16,384 block-rows, 8 blocks
    within +-32, k = 256) in Float64 through the strip kernel, every output."""
    from jlust_amd import workloads as W
    cfg = W.make(5, scale=4)
    val = cfg["val"].astype(np.float64)
    B = np.asfortranarray(cfg["B"].astype(np.float64))
    A = _bsr64(J, cfg["browptr"], cfg["bcolind"], val, cfg["mb"], cfg["nb"])
    C = _run(J, A, B)
    rp, ci, v = O.bsr_to_csr(cfg["browptr"], cfg["bcolind"], val, 16)
    for c0 in range(0, B.shape[1], 64):
        Bs = np.asfortranarray(B[:, c0:c0 + 64])
        ref, _ = O.csr_spmm(rp, ci, v, Bs)
        absref = O.csr_spmm_absref(rp, ci, v, Bs)
        assert_within(C[:, c0:c0 + 64], ref, absref, np.float64, cfg["name"] + f" f64 /4 cols {c0}..")


@pytest.mark.parametrize("k,beta", [(40, 0.0), (64, 0.0), (100, -0.5), (256, 1.0)])
def test_bsr_f64_persistent_schedule(J, O, k, beta):
    """A matrix of 3,100 block-rows (259 strips of 12): with one workgroup per
    CU each XCD's workgroups take several strips in turn, setting up the next
    strip during a strip's last tiles (4 tiles or more: k = 64, 100, 256) or
    at its start (k = 40); an XCD's last round of one strip is cut into column
    ranges.  Strips of long rows or wide windows (direct operand loads) sit
    between banded ones, some rows are empty and the last strip is partial;
    every output against the oracle."""
    mb = nb = 3100
    rng = np.random.default_rng(k)
    bcols = []
    for R in range(mb):
        s = R // 12
        if s % 17 == 5:                               # long rows: up to 11 blocks
            c = rng.choice(nb, int(rng.integers(9, 12)), replace=False)
        elif s % 23 == 9:                             # a window wider than 128 block-rows
            c = rng.choice(nb, 4, replace=False)
        elif R % 13 == 0:
            c = np.zeros(0, np.int64)
        else:
            lo, hi = max(0, R - 32), min(nb, R + 33)
            c = rng.choice(np.arange(lo, hi), int(rng.integers(1, 9)), replace=False)
        bcols.append(np.sort(c))
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcols) + 1).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256)
    A = _bsr64(J, browptr, bcolind, val, mb, nb)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k))) if beta else None
    C = _run(J, A, B, C0, 0.75, beta)
    _check(O, C, browptr, bcolind, val, B, 0.75, beta, C0, f"f64 persistent k={k} beta={beta}")
