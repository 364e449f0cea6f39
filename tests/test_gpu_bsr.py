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


@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_bsr_rowwave_kernel(J, O, monkeypatch, beta):
    """JLUST_HIP_BSR_STRIP=0 runs the row-wave kernel, the one taken when B's
    or C's byte offsets reach 2^31: config 5's pattern at 1/32 scale, a
    scattered pattern and long block-rows, against the oracle."""
    from jlust_amd import workloads as W
    monkeypatch.setenv("JLUST_HIP_BSR_STRIP", "0")
    cfg = W.make(5, scale=32)
    cases = [(cfg["browptr"], cfg["bcolind"], cfg["val"], cfg["B"], cfg["mb"], cfg["nb"], "config 5 /32")]
    for per_row, nb, name in ((4, 300, "scattered"), (19, 40, "long block-rows")):
        bp, bc, bv = random_bsr(30, nb, per_row, seed=60 + per_row)
        B = np.asfortranarray(np.random.default_rng(61).standard_normal((nb * 16, 40)).astype(np.float32))
        cases.append((bp, bc, bv, B, 30, nb, name))
    for bp, bc, bv, B, mb, nb, name in cases:
        C0 = np.asfortranarray(np.random.default_rng(62).standard_normal((mb * 16, B.shape[1])).astype(np.float32))
        C = run_bsr(J, bp, bc, bv, B, mb, nb, alpha=1.25, beta=beta, C0=C0 if beta else None)
        ref = O.bsr_spmm(bp, bc, bv, 16, B, 1.25, beta, C0 if beta else None)
        rp, ci, v = O.bsr_to_csr(bp, bc, bv, 16)
        absref = O.csr_spmm_absref(rp, ci, v, B, 1.25, beta, C0 if beta else None)
        assert_within(C, ref, absref, np.float32, f"row-wave kernel, {name}, beta={beta}")


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


def test_bsr_mfma_entry_rejects_other_block_sizes(J):
    """The fp32 MFMA entry point serves 16 x 16 blocks only and says so; the
    host routes other shapes through the CSR expansion (tests below)."""
    import torch
    from jlust_amd import _lib
    bp = dev(np.array([1, 2], np.int32))
    bc = dev(np.array([1], np.int32))
    v = dev(np.ones(64, np.float32))
    B = dev(np.ones((8, 4), np.float32))
    C = J.dense_matrix(8, 4, dtype=torch.float32)
    st = _lib.lib().jlust_hip_bsr_spmm_f32_i32(
        1, 1, 8, 1, 1, bp.data_ptr(), bc.data_ptr(), v.data_ptr(), 1, 4, 1.0, B.data_ptr(), 8, 0.0,
        C.data_ptr(), 8, torch.cuda.current_stream().cuda_stream)
    assert _lib.STATUS[st] == "UNSUPPORTED_FORMAT"


def _random_rect_bsr(mb, nb, b1, b2, per_row, seed, dtype, row_major, origin=1, zeros=True):
    """Random BSR of b1 x b2 blocks; small integers (exact sums) with some
    stored zeros.  Returns browptr, bcolind, the flat values in the block order
    asked for, and the same blocks row-major as (nnzb, b1, b2)."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, per_row + 1, mb)
    bcols = [np.sort(rng.choice(nb, min(c, nb), replace=False)) for c in counts]
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + origin).astype(np.int32)
    bcolind = (np.concatenate(bcols) + origin).astype(np.int32) if bcols else np.zeros(0, np.int32)
    blocks = rng.integers(-4, 5, (bcolind.size, b1, b2)).astype(dtype)
    if zeros:
        blocks[blocks == 4] = 0
    flat = blocks.reshape(-1) if row_major else blocks.transpose(0, 2, 1).reshape(-1)
    return browptr, bcolind, np.ascontiguousarray(flat), blocks


@pytest.mark.parametrize("b1,b2", [(2, 2), (4, 8), (3, 5), (16, 16), (1, 7)])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_any_block_shape_spmm_and_spmv(J, O, b1, b2, dtype, row_major):
    """BSR of any block shape and value type (16 x 16 fp32 excepted, tested
    above): SpMM through the device CSR expansion, or for 16 x 16 fp64 blocks
    the fp64 MFMA kernel, and SpMV through the expansion, against the
    oracle's expansion + CSR path, with alpha/beta; integer data, so the
    results are exact in both precisions."""
    import torch
    if (b1, b2) == (16, 16) and dtype == np.float32:
        pytest.skip("16 x 16 fp32 is the MFMA kernel (tested above)")
    mb, nb, k = 37, 29, 9
    origin = 1 if row_major else 0
    bp, bc, flat, _ = _random_rect_bsr(mb, nb, b1, b2, 5, 100 + b1 * 7 + b2, dtype, row_major, origin)
    A = J.bsr_tensor(dev(bp), dev(bc), dev(flat), (mb * b1, nb * b2), (b1, b2), row_major,
                     J.OneBased() if origin == 1 else J.ZeroBased())
    rng = np.random.default_rng(5)
    B = np.asfortranarray(rng.integers(-3, 4, (nb * b2, k)).astype(dtype))
    C0 = np.asfortranarray(rng.integers(-3, 4, (mb * b1, k)).astype(dtype))
    C = J.dense_matrix(mb * b1, k, dtype=torch.float64 if dtype == np.float64 else torch.float32)
    C.copy_(dev(C0))
    J.execute(J.SpMMOp, A, dev(B), C, alpha=2.0, beta=-1.0)
    ref = O.bsr_spmm(bp, bc, flat, b1, B, 2.0, -1.0, C0, origin=origin, row_major_blocks=row_major, b2=b2)
    np.testing.assert_array_equal(host(C), ref)
    x = rng.integers(-3, 4, nb * b2).astype(dtype)
    y0 = rng.integers(-3, 4, mb * b1).astype(dtype)
    y = dev(y0.copy())
    J.execute(J.SpMVOp, A, dev(x), y, alpha=0.5, beta=2.0)
    rp, ci, v = O.bsr_to_csr(bp, bc, flat, b1, origin, row_major, b2)
    yref = O.csr_spmv(rp, ci, v, x, 0.5, 2.0, y0, origin)
    np.testing.assert_array_equal(host(y), yref)


def test_bsr_expansion_keeps_stored_zeros_and_matches_oracle_arrays(J, O):
    """jlust_hip_bsr_expand_csr_i32 itself: rowptr, colind and values equal
    the oracle's expansion array for array (explicit zeros kept)."""
    from jlust_amd import hip_backend as HB
    b1, b2 = 3, 4
    bp, bc, flat, _ = _random_rect_bsr(11, 13, b1, b2, 4, 77, np.float64, False)
    A = J.bsr_tensor(dev(bp), dev(bc), dev(flat), (11 * b1, 13 * b2), (b1, b2), False)
    E = HB._bsr_as_csr(A)
    rp, ci, v = O.bsr_to_csr(bp, bc, flat, b1, 1, False, b2)
    assert np.array_equal(host(E.pos_buffers[1]), rp)
    assert np.array_equal(host(E.crd_buffers[1]), ci)
    assert np.array_equal(host(J.nonzeros(E)).view(np.uint64), v.view(np.uint64))
    assert (v == 0).any()


def test_bsr_expansion_rejects_bad_browptr(J):
    """The CSR expansion (the SpMM route of 2 x 2 blocks) reads browptr's ends
    back and rejects a pointer array that does not end at nnzb."""
    bp = dev(np.array([1, 2, 5], np.int32))           # ends at 5, but only 2 blocks are stored
    bc = dev(np.array([1, 2], np.int32))
    A = J.bsr_tensor(bp, bc, dev(np.ones(2 * 4, np.float64)), (4, 4), (2, 2))
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(J.SpMMOp, A, dev(np.asfortranarray(np.ones((4, 3)))), J.dense_matrix(4, 3))


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


@pytest.mark.parametrize("b1,b2", [(16, 16), (3, 5), (1, 9), (7, 1)])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_spmv_direct(J, O, b1, b2, dtype, row_major):
    """BSR SpMV (jlust_hip_bsr_spmv_*, one thread per scalar row, no
    expansion): random values, empty block-rows, ZeroBased for BSRLeft,
    alpha/beta, against the oracle's expansion + CSR SpMV."""
    import torch
    mb, nb = 53, 41
    origin = 1 if row_major else 0
    bp, bc, flat, _ = _random_rect_bsr(mb, nb, b1, b2, 6, 500 + b1 * 11 + b2, dtype, row_major, origin)
    rng = np.random.default_rng(b1 + 31 * b2)
    flat = rng.standard_normal(flat.size).astype(dtype)
    A = J.bsr_tensor(dev(bp), dev(bc), dev(flat), (mb * b1, nb * b2), (b1, b2), row_major,
                     J.OneBased() if origin == 1 else J.ZeroBased())
    x = rng.uniform(-1, 1, nb * b2).astype(dtype)
    y0 = rng.uniform(-1, 1, mb * b1).astype(dtype)
    rp, ci, v = O.bsr_to_csr(bp, bc, flat, b1, origin, row_major, b2)
    for alpha, beta in ((1.0, 0.0), (-0.5, 1.5)):
        y = dev(y0.copy()) if beta else torch.full((mb * b1,), float("nan"), dtype=A.dtype, device="cuda")
        J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
        yb = y0 if beta else None
        ref = O.csr_spmv(rp, ci, v, x, alpha, beta, yb, origin)
        absref = O.csr_spmv_absref(rp, ci, v, x, alpha, beta, yb, origin)
        assert_within(host(y), ref, absref, dtype, f"bsr spmv {b1}x{b2} beta={beta}")


def test_bsr_spmv_rejects_bad_browptr(J):
    """BSR SpMV checks browptr (and the block columns) once per version of
    the index buffers: a pointer array that ends past nnzb, or one that does
    not start at the origin, is NonCanonicalStorage, as the CSR expansion
    route reports it; the kernel itself would only clamp it."""
    bc = dev(np.array([1, 2], np.int32))
    x = dev(np.ones(4))
    for bad in ([1, 2, 5], [2, 2, 3], [1, 3, 3 - 1]):
        A = J.bsr_tensor(dev(np.array(bad, np.int32)), bc, dev(np.ones(2 * 4, np.float64)), (4, 4), (2, 2))
        with pytest.raises(J.NonCanonicalStorage):
            J.execute(J.SpMVOp, A, x, dev(np.zeros(4)))
    A = J.bsr_tensor(dev(np.array([1, 2, 3], np.int32)), dev(np.array([1, 3], np.int32)),
                     dev(np.ones(2 * 4, np.float64)), (4, 4), (2, 2))
    with pytest.raises(J.NonCanonicalStorage):                       # block column 3 of 2
        J.execute(J.SpMVOp, A, x, dev(np.zeros(4)))
    good = J.bsr_tensor(dev(np.array([1, 2, 3], np.int32)), bc, dev(np.arange(8, dtype=np.float64)),
                        (4, 4), (2, 2))
    y = dev(np.zeros(4))
    J.execute(J.SpMVOp, good, x, y)
    np.testing.assert_array_equal(host(y), [1.0, 5.0, 9.0, 13.0])
    # the index buffer written in place through torch is checked again
    good.pos_buffers[1][2] = 7
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(J.SpMVOp, good, x, y)


def test_bsr_f32_unaligned_values_plain_and_plan(J, O):
    """fp32 16 x 16 BSRRight values that are not 16-byte aligned (a view at an
    odd element offset): the plain call takes the CSR expansion, as the
    prepared plan does, and both match the definition."""
    import torch
    mb, nb, k = 24, 20, 40
    browptr, bcolind, val = random_bsr(mb, nb, 5, seed=31)
    store = torch.empty(val.size + 1, dtype=torch.float32, device="cuda")
    store[1:] = torch.from_numpy(val).cuda()
    vview = store[1:]
    assert vview.data_ptr() % 16 != 0
    A = J.bsr_tensor(dev(browptr), dev(bcolind), vview, (mb * 16, nb * 16), (16, 16))
    B = np.asfortranarray(np.random.default_rng(32).standard_normal((nb * 16, k)).astype(np.float32))
    C = J.dense_matrix(mb * 16, k, dtype=torch.float32, fill=float("nan"))
    J.execute(J.SpMMOp, A, dev(B), C)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    ref, _ = O.csr_spmm(rp, ci, v, B)
    absref = O.csr_spmm_absref(rp, ci, v, B)
    assert_within(host(C), ref, absref, np.float32, "unaligned plain")
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    C2 = J.dense_matrix(mb * 16, k, dtype=torch.float32, fill=float("nan"))
    J.execute(h, dev(B), C2)
    assert_within(host(C2), ref, absref, np.float32, "unaligned plan")


@pytest.mark.parametrize("b1,b2", [(16, 16), (3, 5)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("row_major", [True, False])
@pytest.mark.parametrize("segments", ["1", "0"])
def test_bsr_spmv_power_law_rows(J, O, b1, b2, dtype, row_major, segments, monkeypatch):
    """BSR SpMV over power-law block-rows (one of 700 blocks, several past
    the 32-block segment, empty ones): the segmented kernels spread a
    block-row over waves (16 x 16) or threads (other shapes) and add the
    segments' sums in order (JLUST_HIP_BSR_SPMV_SEGMENTS=0: the
    one-thread-per-row kernel).  Against the oracle's expansion + CSR SpMV,
    alpha/beta, values viewed at an odd offset too (element loads)."""
    import torch
    monkeypatch.setenv("JLUST_HIP_BSR_SPMV_SEGMENTS", segments)
    mb, nb = 300, 900
    rng = np.random.default_rng(17 + row_major + b1)
    lens = np.minimum((rng.pareto(1.3, mb) + 1) * 3, nb).astype(np.int64)
    lens[::11] = 0
    lens[5], lens[6], lens[7] = 700, 33, 32
    bcols = [np.sort(rng.choice(nb, int(n), replace=False)) for n in lens]
    origin = 1 if row_major else 0
    bp = (np.r_[0, np.cumsum(lens)] + origin).astype(np.int32)
    bc = (np.concatenate(bcols) + origin).astype(np.int32)
    flat = rng.standard_normal(bc.size * b1 * b2).astype(dtype)
    x = rng.uniform(-1, 1, nb * b2).astype(dtype)
    y0 = rng.uniform(-1, 1, mb * b1).astype(dtype)
    rp, ci, v = O.bsr_to_csr(bp, bc, flat, b1, origin, row_major, b2)
    og = J.OneBased() if origin == 1 else J.ZeroBased()
    vbuf = dev(np.r_[np.zeros(1, dtype), flat])
    for vals in (dev(flat), vbuf[1:]):
        A = J.bsr_tensor(dev(bp), dev(bc), vals, (mb * b1, nb * b2), (b1, b2), row_major, og)
        for alpha, beta in ((1.0, 0.0), (-0.5, 1.5)):
            y = dev(y0.copy()) if beta else torch.full((mb * b1,), float("nan"), dtype=A.dtype, device="cuda")
            J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
            yb = y0 if beta else None
            ref = O.csr_spmv(rp, ci, v, x, alpha, beta, yb, origin)
            absref = O.csr_spmv_absref(rp, ci, v, x, alpha, beta, yb, origin)
            assert_within(host(y), ref, absref, dtype, f"bsr {b1}x{b2} spmv power-law beta={beta}")


@pytest.mark.parametrize("wide", ["1", "0"])
@pytest.mark.parametrize("k,beta", [(40, 0.0), (64, 0.0), (100, -0.5), (256, 1.0)])
def test_bsr_strip_schedule(J, O, k, beta, wide, monkeypatch):
    """A matrix of 6,900 block-rows (288 strips of 24; 575 of 12) through the
    24-row persistent strip kernel (JLUST_HIP_BSR_WIDE=1) and the 12-row one:
    each XCD's workgroups take several strips in turn, setting up the next
    strip during a strip's last tiles (4 tiles or more: k = 64, 100, 256) or
    at its start (k = 40), and an XCD's last round of 4 strips is cut into
    column ranges.  Strips of long rows or wide windows (direct operand loads)
    sit between banded ones, some rows are empty and the last strip is
    partial; every output against the oracle."""
    monkeypatch.setenv("JLUST_HIP_BSR_WIDE", wide)
    mb = nb = 6900
    rng = np.random.default_rng(k)
    bcols = []
    for R in range(mb):
        s = R // 24
        if s % 17 == 5 and R % 3 == 0:                # long rows: up to 11 blocks
            c = rng.choice(nb, int(rng.integers(9, 12)), replace=False)
        elif s % 23 == 9 and R % 5 == 0:              # a window wider than 88 block-rows
            c = rng.choice(nb, 4, replace=False)
        elif R % 13 == 0:
            c = np.zeros(0, np.int64)
        else:
            lo, hi = max(0, R - 32), min(nb, R + 33)
            c = rng.choice(np.arange(lo, hi), int(rng.integers(1, 9)), replace=False)
        bcols.append(np.sort(c))
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcols) + 1).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256).astype(np.float32)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)).astype(np.float32))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k)).astype(np.float32)) if beta else None
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=0.75, beta=beta, C0=C0)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 0.75, beta, C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, B, 0.75, beta, C0)
    assert_within(C, ref, absref, np.float32, f"strip schedule wide={wide} k={k} beta={beta}")


@pytest.mark.parametrize("wide", ["1", "0"])
def test_bsr_nonfinite_b_rows_reach_only_their_blocks(J, O, wide, monkeypatch):
    """B rows holding NaN and Inf inside the strips' windows: only the
    block-rows with a block in those B rows may see them.  The 24-row kernel
    runs the MFMAs of absent blocks on a zero row of its window rather than
    on B, so no other output may turn non-finite; rows of 1 to 8 blocks (the
    absent blocks in between) within a +-32 band, through both strip kernels."""
    monkeypatch.setenv("JLUST_HIP_BSR_WIDE", wide)
    mb = nb = 600
    k = 48
    rng = np.random.default_rng(77)
    bcols = []
    for R in range(mb):
        lo, hi = max(0, R - 32), min(nb, R + 33)
        bcols.append(np.sort(rng.choice(np.arange(lo, hi), int(rng.integers(1, 9)), replace=False)))
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcols) + 1).astype(np.int32)
    val = rng.standard_normal(bcolind.size * 256).astype(np.float32)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)).astype(np.float32))
    bad_blocks = rng.choice(nb, 40, replace=False)
    B[bad_blocks[:20] * 16 + 3, :] = np.nan
    B[bad_blocks[20:] * 16 + 11, :] = np.inf
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=1.0, beta=0.0)
    touched = np.array([np.isin(c, bad_blocks).any() for c in bcols])
    rows_ok = np.repeat(~touched, 16)
    assert rows_ok.any() and (~rows_ok).any()
    assert np.isfinite(C[rows_ok]).all(), f"wide={wide}: a non-finite B row reached a row without its block"
    keep = ~touched
    sel = np.flatnonzero(keep)
    sub_bp = np.r_[0, np.cumsum([bcols[R].size for R in sel])] + 1
    sub_bc = np.concatenate([bcols[R] for R in sel]) + 1
    sub_val = np.concatenate([val[(browptr[R] - 1) * 256:(browptr[R + 1] - 1) * 256] for R in sel])
    Bf = np.where(np.isfinite(B), B, 0).astype(np.float32)
    ref = O.bsr_spmm(sub_bp.astype(np.int32), sub_bc.astype(np.int32), sub_val, 16, Bf, 1.0, 0.0, None)
    rp, ci, v = O.bsr_to_csr(sub_bp.astype(np.int32), sub_bc.astype(np.int32), sub_val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, Bf, 1.0, 0.0, None)
    assert_within(C[rows_ok], ref, absref, np.float32, f"wide={wide}: finite rows")


@pytest.mark.parametrize("b1,b2", [(16, 16), (3, 5)])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("row_major", [True, False])
def test_bsr_spmv_plan(J, O, b1, b2, dtype, row_major):
    """prepare(HIPBackend(), SpMVOp, A::BSR) builds the segment table once
    (jlust_hip_bsr_spmv_plan_*): products on power-law block-rows (empty
    ones, one past many segments) against the oracle, repeated with new x;
    values written in place are seen; another value tensor through
    update_values! and through execute(h, A, x, y); a block column written in
    place rebuilds the table, a malformed one raises NonCanonicalStorage."""
    import torch
    from jlust_amd.hip_backend import HIPBSRSpMVHandle
    mb, nb = 200, 300
    rng = np.random.default_rng(41 + b1 + row_major)
    lens = np.minimum((rng.pareto(1.3, mb) + 1) * 2, nb).astype(np.int64)
    lens[::9] = 0
    lens[3] = 250
    bcols = [np.sort(rng.choice(nb, int(n), replace=False)) for n in lens]
    origin = 1 if row_major else 0
    bp = (np.r_[0, np.cumsum(lens)] + origin).astype(np.int32)
    bc = (np.concatenate(bcols) + origin).astype(np.int32)
    flat = rng.standard_normal(bc.size * b1 * b2).astype(dtype)
    og = J.OneBased() if origin == 1 else J.ZeroBased()
    A = J.bsr_tensor(dev(bp), dev(bc), dev(flat), (mb * b1, nb * b2), (b1, b2), row_major, og)
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    assert isinstance(h, HIPBSRSpMVHandle)
    y0 = rng.uniform(-1, 1, mb * b1).astype(dtype)

    def check(vals, bcv, what):
        rp, ci, v = O.bsr_to_csr(bp, bcv, vals, b1, origin, row_major, b2)
        for alpha, beta in ((1.0, 0.0), (-0.5, 1.5)):
            x = rng.uniform(-1, 1, nb * b2).astype(dtype)
            y = dev(y0.copy()) if beta else torch.full((mb * b1,), float("nan"), dtype=A.dtype, device="cuda")
            J.execute(h, dev(x), y, alpha=alpha, beta=beta)
            yb = y0 if beta else None
            ref = O.csr_spmv(rp, ci, v, x, alpha, beta, yb, origin)
            absref = O.csr_spmv_absref(rp, ci, v, x, alpha, beta, yb, origin)
            assert_within(host(y), ref, absref, dtype, f"bsr {b1}x{b2} spmv plan, {what}, beta={beta}")

    check(flat, bc, "first")
    A.val.mul_(-2.0)                                     # in place: the plan reads the values at the call
    check(flat * -2, bc, "values scaled in place")
    flat2 = rng.standard_normal(flat.size).astype(dtype)
    J.update_values_(h, J.bsr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(flat2), A.extents,
                                     (b1, b2), row_major, og))
    check(flat2, bc, "update_values!")
    flat3 = rng.standard_normal(flat.size).astype(dtype)
    A3 = J.bsr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(flat3), A.extents, (b1, b2), row_major, og)
    x = rng.uniform(-1, 1, nb * b2).astype(dtype)
    y = dev(np.zeros(mb * b1, dtype))
    J.execute(h, A3, dev(x), y)
    rp, ci, v = O.bsr_to_csr(bp, bc, flat3, b1, origin, row_major, b2)
    assert_within(host(y), O.csr_spmv(rp, ci, v, x, 1.0, 0.0, None, origin),
                  O.csr_spmv_absref(rp, ci, v, x, 1.0, 0.0, None, origin), dtype, "execute(h, A, x, y)")
    # the first block of block-row 3 moved to a column the row does not use
    bc2 = bc.copy()
    q = bp[3] - origin
    free = np.setdiff1d(np.arange(nb), bcols[3])
    bc2[q] = free[0] + origin
    order = np.argsort(bc2[q:q + lens[3]], kind="stable")
    bc2[q:q + lens[3]] = bc2[q:q + lens[3]][order]
    blocks = flat3.reshape(-1, b1 * b2).copy()
    blocks[q:q + lens[3]] = blocks[q:q + lens[3]][order]
    h.u_A.crd_buffers[1].copy_(dev(bc2))
    h.u_A.val.copy_(dev(blocks.reshape(-1)))
    check(blocks.reshape(-1), bc2, "block columns written in place")
    h.u_A.crd_buffers[1][0] = nb + origin                # past the last block column
    with pytest.raises(J.NonCanonicalStorage):
        J.execute(h, dev(x), y)


@pytest.mark.parametrize("k,beta", [(40, 0.0), (100, -0.5), (256, 1.0)])
def test_bsr_long_rows_two_halves(J, O, k, beta):
    """Rows of 9 to 16 blocks, more than 8 on average (the long-row kernel:
    a strip as two halves of 12 rows, a row's blocks in two groups of 8):
    mixed with strips of 8-block rows, rows of 17 to 20 blocks (direct
    operand loads), empty rows, a window wider than 88 block-rows in one
    half, and a partial last strip; every output against the oracle."""
    mb = nb = 2000
    rng = np.random.default_rng(k + 5)
    bcols = []
    for R in range(mb):
        s = R // 24
        lo, hi = max(0, R - 32), min(nb, R + 33)
        if s % 7 == 3:
            n = 8
        elif s % 11 == 6 and R % 5 == 0:
            n = int(rng.integers(17, 21))
        elif s % 13 == 2 and R % 24 == 14:               # second half: a block far away
            c = np.r_[rng.choice(np.arange(lo, hi), 10, replace=False), (R + 500) % nb]
            bcols.append(np.sort(np.unique(c)))
            continue
        elif R % 17 == 0:
            n = 0
        else:
            n = int(rng.integers(9, 17))
        bcols.append(np.sort(rng.choice(np.arange(lo, hi), min(n, hi - lo), replace=False)))
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + 1).astype(np.int32)
    bcolind = (np.concatenate(bcols) + 1).astype(np.int32)
    assert bcolind.size > 8 * mb
    val = rng.standard_normal(bcolind.size * 256).astype(np.float32)
    B = np.asfortranarray(rng.standard_normal((nb * 16, k)).astype(np.float32))
    C0 = np.asfortranarray(rng.standard_normal((mb * 16, k)).astype(np.float32)) if beta else None
    C = run_bsr(J, browptr, bcolind, val, B, mb, nb, alpha=0.75, beta=beta, C0=C0)
    ref = O.bsr_spmm(browptr, bcolind, val, 16, B, 0.75, beta, C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, val, 16)
    absref = O.csr_spmm_absref(rp, ci, v, B, 0.75, beta, C0)
    assert_within(C, ref, absref, np.float32, f"long rows k={k} beta={beta}")
