"""GPU parity of the 16x16 BSR SpMM (fp32 MFMA) against its definition:
the oracle expands the BSR matrix to CSR bit-exactly and runs the CSR path
(the reference has no working BSR compute path to compare with)."""
import json
import os

import numpy as np
import pytest

from tests._util import assert_within, dev, host

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


def random_bsr(mb, nb, per_row, seed, origin=1, band=None):
    rng = np.random.default_rng(seed)
    bcols = []
    counts = []
    for R in range(mb):
        lo, hi = (0, nb) if band is None else (max(0, R - band), min(nb, R + band + 1))
        c = np.sort(rng.choice(np.arange(lo, hi), size=min(per_row, hi - lo), replace=False))
        bcols.append(c)
        counts.append(c.size)
    browptr = (np.r_[0, np.cumsum(counts)] + origin).astype(np.int32)
    bcolind = (np.concatenate(bcols) + origin).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256).astype(np.float32)
    return browptr, bcolind, val


def run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=1.0, beta=0.0, C0=None, origin=1,
            row_major=True):
    A = J.bsr_tensor(dev(browptr), dev(bcolind), dev(val), (mb * 16, nb * 16), (16, 16),
                     row_major_blocks=row_major,
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    k = B.shape[1]
    C = J.dense_matrix(mb * 16, k, dtype=A.dtype, fill=float("nan")) if C0 is None else \
        dev(np.asfortranarray(C0))
    J.execute(J.SpMMOp, A, dev(np.asfortranarray(B)), C, alpha=alpha, beta=beta)
    return host(C)


def dense_of_bsr(browptr, bcolind, val, mb, nb, origin=1, row_major=True):
    D = np.zeros((mb * 16, nb * 16), np.float64)
    blocks = val.reshape(-1, 16, 16).astype(np.float64)
    for R in range(mb):
        for q in range(browptr[R] - origin, browptr[R + 1] - origin):
            c = bcolind[q] - origin
            blk = blocks[q] if row_major else blocks[q].T
            D[16 * R:16 * R + 16, 16 * c:16 * c + 16] += blk
    return D


@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_single_blocks_exact_layout(J, row_major):
    """One block with entries chosen so that any mix-up of the MFMA operand
    layout (row/column swap, k-group order) changes the result: small integers,
    so fp32 products and sums are exact."""
    browptr = np.array([1, 2], np.int32)
    bcolind = np.array([1], np.int32)
    blk = (np.arange(256) % 7 - 3).astype(np.float32)          # V[r][s] = blk[16r+s]
    val = blk if row_major else blk.reshape(16, 16).T.reshape(-1).copy()
    B = np.asfortranarray((np.arange(16 * 48) % 5 - 2).astype(np.float32).reshape(16, 48))
    C = run_bsr(J, browptr, bcolind, val, B, 1, 1, row_major=row_major)
    expect = blk.reshape(16, 16).astype(np.float64) @ B.astype(np.float64)
    np.testing.assert_array_equal(C, expect.astype(np.float32))


@pytest.mark.parametrize("k", [16, 40, 256, 300])
def test_bsr_random_vs_dense(J, O, k):
    mb, nb = 37, 29
    browptr, bcolind, val = random_bsr(mb, nb, 5, seed=k)
    B = np.asfortranarray(np.random.default_rng(1).standard_normal((nb * 16, k)).astype(np.float32))
    C0 = np.asfortranarray(np.random.default_rng(2).standard_normal((mb * 16, k)).astype(np.float32))
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=1.25, beta=-0.5, C0=C0)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 1.25, -0.5, C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, B, 1.25, -0.5, C0)
    assert_within(C, ref, absref, np.float32, f"bsr k={k}")
    D = dense_of_bsr(browptr, bcolind, val, mb, nb)
    exact = 1.25 * (D @ B.astype(np.float64)) - 0.5 * C0
    assert_within(C, exact, absref, np.float32, "bsr vs dense")


def test_bsr_left_zero_based(J, O):
    mb, nb, k = 20, 20, 64
    browptr, bcolind, val = random_bsr(mb, nb, 4, seed=3, origin=0)
    B = np.asfortranarray(np.random.default_rng(4).standard_normal((nb * 16, k)).astype(np.float32))
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, origin=0, row_major=False)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, origin=0, row_major_blocks=False)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16, origin=0, row_major_blocks=False)
    absref = O.csr_spmm_absref(rp, ci, v, B, origin=0)
    assert_within(C, ref, absref, np.float32, "BSRLeft, ZeroBased")


def test_bsr_empty_block_rows(J, O):
    mb, nb, k = 10, 10, 32
    browptr = np.array([1, 1, 3, 3, 3, 4, 4, 4, 4, 4, 5], np.int32)
    bcolind = np.array([1, 10, 5, 2], np.int32)
    val = np.random.default_rng(0).standard_normal(4 * 256).astype(np.float32)
    B = np.asfortranarray(np.random.default_rng(1).standard_normal((160, k)).astype(np.float32))
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    assert_within(C, ref, O.csr_spmm_absref(rp, ci, v, B), np.float32, "empty block-rows")


def test_bsr_config5_scaled(J, O):
    from jlust_amd import workloads as W
    cfg = W.make(5, scale=32)
    C = run_bsr(J, cfg["browptr"], cfg["bcolind"], cfg["val"], cfg["B"], cfg["mb"], cfg["nb"])
    ref = O.bsr_spmm(cfg["browptr"], cfg["bcolind"], cfg["val"], 16, cfg["B"])
    rp, ci, v = O.bsr_to_csr(cfg["browptr"], cfg["bcolind"], cfg["val"], 16)
    absref = O.csr_spmm_absref(rp, ci, v, cfg["B"])
    assert_within(C, ref, absref, np.float32, cfg["name"] + " /32")


def test_bsr_config5_full_sampled_block_rows(J, O):
    from jlust_amd import workloads as W
    cfg = W.make(5)
    C = run_bsr(J, cfg["browptr"], cfg["bcolind"], cfg["val"], cfg["B"], cfg["mb"], cfg["nb"])
    assert np.isfinite(C).all()
    rng = np.random.default_rng(2)
    sel = np.sort(rng.choice(cfg["mb"], 64, replace=False))
    bp = cfg["browptr"]
    cnt = bp[sel + 1] - bp[sel]
    sub_bp = (np.r_[0, np.cumsum(cnt)] + 1).astype(np.int32)
    q = np.concatenate([np.arange(bp[s] - 1, bp[s + 1] - 1) for s in sel])
    sub_bc = cfg["bcolind"][q]
    sub_val = cfg["val"].reshape(-1, 256)[q].reshape(-1)
    ref = O.bsr_spmm(sub_bp, sub_bc, sub_val, 16, cfg["B"])
    rp, ci, v = O.bsr_to_csr(sub_bp, sub_bc, sub_val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, cfg["B"])
    rows = (sel[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    assert_within(C[rows], ref, absref, np.float32, cfg["name"])


def test_bsr_unsupported_block_size(J):
    import torch
    A = J.bsr_tensor(dev(np.array([1, 2], np.int32)), dev(np.array([1], np.int32)),
                     dev(np.ones(64, np.float32)), (8, 8), (8, 8))
    with pytest.raises(J.UnsupportedFormat):
        J.execute(J.SpMMOp, A, dev(np.ones((8, 4), np.float32)), J.dense_matrix(8, 4, dtype=torch.float32))


@pytest.mark.parametrize("beta", [0.0, -0.5])
def test_bsr_long_block_rows(J, O, beta):
    """Block-rows with more blocks than one register chunk (8): the partial
    products of later chunks are added onto C."""
    mb, nb, k = 12, 40, 48
    browptr, bcolind, val = random_bsr(mb, nb, 19, seed=11)
    B = np.asfortranarray(np.random.default_rng(5).standard_normal((nb * 16, k)).astype(np.float32))
    C0 = np.asfortranarray(np.random.default_rng(6).standard_normal((mb * 16, k)).astype(np.float32))
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=0.75, beta=beta, C0=C0)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 0.75, beta, C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, B, 0.75, beta, C0)
    assert_within(C, ref, absref, np.float32, f"19 blocks per block-row, beta={beta}")


def test_bsr_empty_block_rows_beta(J, O):
    mb, nb, k = 10, 10, 20
    browptr = np.array([1, 1, 3, 3, 3, 4, 4, 4, 4, 4, 5], np.int32)
    bcolind = np.array([1, 10, 5, 2], np.int32)
    val = np.random.default_rng(0).standard_normal(4 * 256).astype(np.float32)
    B = np.asfortranarray(np.random.default_rng(1).standard_normal((160, k)).astype(np.float32))
    C0 = np.asfortranarray(np.random.default_rng(2).standard_normal((160, k)).astype(np.float32))
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=2.0, beta=3.0, C0=C0)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 2.0, 3.0, C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, B, 2.0, 3.0, C0)
    assert_within(C, ref, absref, np.float32, "empty block-rows, beta=3")


def test_bsr_unaligned_leading_dims(J, O):
    """ldb and ldc not multiples of 4: the scalar-access kernel."""
    import torch
    mb, nb, k = 9, 11, 24
    browptr, bcolind, val = random_bsr(mb, nb, 3, seed=21)
    Bbig = np.asfortranarray(np.random.default_rng(7).standard_normal((nb * 16 + 1, k)).astype(np.float32))
    A = J.bsr_tensor(dev(browptr), dev(bcolind), dev(val), (mb * 16, nb * 16), (16, 16))
    Bd = dev(Bbig)[: nb * 16]
    Cbig = torch.full((k, mb * 16 + 3), float("nan"), dtype=torch.float32, device="cuda").t()
    Cd = Cbig[: mb * 16]
    from jlust_amd.tensor import leading_dim
    assert leading_dim(Bd) == nb * 16 + 1 and leading_dim(Cd) == mb * 16 + 3
    J.execute(J.SpMMOp, A, Bd, Cd)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, np.asfortranarray(Bbig[: nb * 16]))
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, np.asfortranarray(Bbig[: nb * 16]))
    assert_within(host(Cd), ref, absref, np.float32, "unaligned leading dimensions")


@pytest.mark.parametrize("case", ["scattered", "wide_band", "band_tail"])
def test_bsr_block_patterns(J, O, case):
    """Block patterns beside config 5's: blocks scattered over 2000 block
    columns, a band of +-60 block columns, and a narrow band with 12 blocks
    per block-row (more than one register chunk of 8), each for beta = 0 and
    beta != 0."""
    if case == "scattered":
        mb, nb, per_row, band = 48, 2000, 4, None
    elif case == "wide_band":
        mb, nb, per_row, band = 64, 64, 8, 60
    else:
        mb, nb, per_row, band = 40, 40, 12, 10
    k = 40
    browptr, bcolind, val = random_bsr(mb, nb, per_row, seed=31, band=band)
    B = np.asfortranarray(np.random.default_rng(8).standard_normal((nb * 16, k)).astype(np.float32))
    C0 = np.asfortranarray(np.random.default_rng(9).standard_normal((mb * 16, k)).astype(np.float32))
    for beta in (0.0, 0.5):
        C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=1.5, beta=beta, C0=C0)
        ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 1.5, beta, C0)
        rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
        absref = O.csr_spmm_absref(rp, ci, v, B, 1.5, beta, C0)
        assert_within(C, ref, absref, np.float32, f"{case} beta={beta}")
