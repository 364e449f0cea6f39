"""GPU parity of CSR SpMM, CSR SDDMM and COO SpMV against the CPU oracle."""
import json
import os

import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr, sample_rows

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


# ------------------------------------------------------------------- SpMM

def run_spmm(J, rowptr, colind, val, B, m, n, alpha=1.0, beta=0.0, C0=None, origin=1,
             skip_empty_rows=False):
    import torch
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n),
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    k = B.shape[1]
    if C0 is None:
        C = J.dense_matrix(m, k, dtype=A.dtype, fill=float("nan"))
    else:
        C = dev(np.asfortranarray(C0))
    J.execute(J.SpMMOp, A, dev(np.asfortranarray(B)), C, alpha=alpha, beta=beta,
              skip_empty_rows=skip_empty_rows)
    assert C.stride(0) == 1
    return host(C)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_reference_fixture(J, dtype):
    c = GOLDEN["spmm"][0]
    C = run_spmm(J, np.array(c["rowptr"], np.int32), np.array(c["colind"], np.int32),
                 np.array(c["val"], dtype), np.array(c["B"], dtype), 3, 3)
    np.testing.assert_array_equal(C, np.array(c["C"], dtype))


@pytest.mark.parametrize("k", [1, 2, 3, 4, 7, 8, 16, 31, 32, 33, 64, 100, 128, 200, 256, 300])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_random(J, O, k, dtype):
    m, n = 3000, 2000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(k).integers(0, 70, m),
                                     seed=k, dtype=dtype)
    B = np.asfortranarray(np.random.default_rng(7).standard_normal((n, k)).astype(dtype))
    C = run_spmm(J, rowptr, colind, val, B, m, n)
    ref, strat = O.csr_spmm(rowptr, colind, val, B)
    absref = O.csr_spmm_absref(rowptr, colind, val, B)
    assert_within(C, ref, absref, dtype, f"k={k} ({strat})")


@pytest.mark.parametrize("alpha,beta", [(2.0, 0.0), (0.5, -1.5)])
def test_spmm_alpha_beta_zero_based(J, O, alpha, beta):
    m, n, k = 1000, 1500, 128
    rowptr, colind, val = random_csr(m, n, density=0.01, seed=3, origin=0)
    B = np.asfortranarray(np.random.default_rng(1).standard_normal((n, k)))
    C0 = np.asfortranarray(np.random.default_rng(2).standard_normal((m, k)))
    C = run_spmm(J, rowptr, colind, val, B, m, n, alpha, beta, C0, origin=0)
    ref, _ = O.csr_spmm(rowptr, colind, val, B, alpha, beta, C0, origin=0)
    absref = O.csr_spmm_absref(rowptr, colind, val, B, alpha, beta, C0, origin=0)
    assert_within(C, ref, absref, np.float64, "alpha/beta")


def test_spmm_skip_empty_rows(J, O):
    m, n, k = 500, 400, 16
    lens = np.where(np.arange(m) % 3 == 0, 0, 5)
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=9)
    B = np.asfortranarray(np.random.default_rng(1).standard_normal((n, k)))
    C0 = np.asfortranarray(np.full((m, k), 7.0))
    C = run_spmm(J, rowptr, colind, val, B, m, n, 1.0, 0.0, C0, skip_empty_rows=True)
    ref, strat = O.csr_spmm(rowptr, colind, val, B, 1.0, 0.0, C0, skip_empty_rows=True)
    assert strat == "2D"
    np.testing.assert_array_equal(C[lens == 0], 7.0)
    absref = O.csr_spmm_absref(rowptr, colind, val, B)
    assert_within(C, ref, absref + (lens == 0)[:, None], np.float64, "skip_empty_rows")


def test_spmm_config3_scaled(J, O):
    from jlust_amd import workloads as W
    cfg = W.make(3, scale=16)
    C = run_spmm(J, cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"], cfg["m"], cfg["n"])
    ref, strat = O.csr_spmm(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"])
    assert strat == "Tiled"
    absref = O.csr_spmm_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"])
    assert_within(C, ref, absref, np.float32, cfg["name"] + " /16")


def test_spmm_config3_full_sampled_rows(J, O):
    """Full config 3 on the GPU; 4000 random rows checked against the oracle."""
    from jlust_amd import workloads as W
    cfg = W.make(3)
    C = run_spmm(J, cfg["rowptr"], cfg["colind"], cfg["val"], cfg["B"], cfg["m"], cfg["n"])
    rows = np.sort(np.random.default_rng(0).choice(cfg["m"], 4000, replace=False))
    rp, ci, v, _ = sample_rows(cfg["rowptr"], cfg["colind"], cfg["val"], rows)
    ref, _ = O.csr_spmm(rp, ci, v, cfg["B"])
    absref = O.csr_spmm_absref(rp, ci, v, cfg["B"])
    assert_within(C[rows], ref, absref, np.float32, cfg["name"])
    assert np.isfinite(C).all()


# ------------------------------------------------------------------ SDDMM

def run_sddmm(J, rowptr, colind, A, B, m, n, alpha=1.0, beta=0.0, c0=None, mask=None, origin=1):
    import torch
    nz = colind.size
    cv = dev(c0) if c0 is not None else torch.full((nz,), float("nan"),
                                                   dtype=torch.float64 if A.dtype == np.float64
                                                   else torch.float32, device="cuda")
    Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n),
                      origin=J.OneBased() if origin == 1 else J.ZeroBased())
    J.execute(J.SDDMMOp, dev(np.asfortranarray(A)), dev(np.asfortranarray(B)), Cs, alpha=alpha,
              beta=beta, mask=None if mask is None else dev(mask))
    return host(cv)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_reference_fixture(J, dtype):
    c = GOLDEN["sddmm"][0]
    out = run_sddmm(J, np.array(c["rowptr"], np.int32), np.array(c["colind"], np.int32),
                    np.array(c["A"], dtype), np.array(c["B"], dtype), 3, 3,
                    c0=np.array(c["c0"], dtype), beta=c["beta"])
    np.testing.assert_array_equal(out, np.array(c["cval"], dtype))


@pytest.mark.parametrize("K", [1, 2, 3, 4, 8, 12, 16, 32, 64, 128, 130, 256, 512])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_random(J, O, K, dtype):
    m, n = 2000, 1500
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(K).integers(0, 50, m),
                                     seed=K, dtype=dtype)
    rng = np.random.default_rng(5)
    A = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    B = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    c0 = rng.standard_normal(colind.size).astype(dtype)
    out = run_sddmm(J, rowptr, colind, A, B, m, n, alpha=1.5, beta=0.25, c0=c0)
    ref = O.csr_sddmm(rowptr, colind, A, B, 1.5, 0.25, c0)
    absref = O.csr_sddmm_absref(rowptr, colind, A, B, 1.5, 0.25, c0)
    assert_within(out, ref, absref, dtype, f"K={K}")


@pytest.mark.parametrize("K", [128, 4, 1])
def test_sddmm_mask_in_place(J, O, K):
    """The config-4 form: out = S_ij * dot, with the mask read from C.val itself
    (K = 4 and 1 run several nonzeros per lane group per step)."""
    import torch
    m, n = 3000, 2500
    rowptr, colind, _ = random_csr(m, n, lengths=np.full(m, 32), seed=11, dtype=np.float32)
    rng = np.random.default_rng(6)
    A = np.asfortranarray(rng.standard_normal((m, K)).astype(np.float32))
    B = np.asfortranarray(rng.standard_normal((K, n)).astype(np.float32))
    S = rng.uniform(0.5, 1.5, colind.size).astype(np.float32)
    cv = dev(S)
    Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n))
    J.execute(J.SDDMMOp, dev(A), dev(B), Cs, beta=0.0, mask=Cs)
    torch.cuda.synchronize()
    ref = O.csr_sddmm(rowptr, colind, A, B, mask=S)
    absref = O.csr_sddmm_absref(rowptr, colind, A, B, mask=S)
    assert_within(host(cv), ref, absref, np.float32, f"mask in place K={K}")


def test_sddmm_config4_full_sampled_rows(J, O):
    from jlust_amd import workloads as W
    cfg = W.make(4)
    out = run_sddmm(J, cfg["rowptr"], cfg["colind"], cfg["A"], cfg["B"], cfg["m"], cfg["n"],
                    mask=cfg["mask"])
    rows = np.sort(np.random.default_rng(1).choice(cfg["m"], 5000, replace=False))
    rp, ci, mk, idx = sample_rows(cfg["rowptr"], cfg["colind"], cfg["mask"], rows)
    Asub = np.asfortranarray(cfg["A"][rows])
    ref = O.csr_sddmm(rp, ci, Asub, cfg["B"], mask=mk)
    absref = O.csr_sddmm_absref(rp, ci, Asub, cfg["B"], mask=mk)
    assert_within(out[idx], ref, absref, np.float32, cfg["name"])
    assert np.isfinite(out).all()


# --------------------------------------------------------------- COO SpMV

def test_coo_reference_fixture(J):
    c = [c for c in GOLDEN["spmv"] if c["format"] == "COO"][0]
    A = J.coo_tensor(dev(np.array(c["rows"], np.int32)), dev(np.array(c["cols"], np.int32)),
                     dev(np.array(c["val"])), (3, 3))
    y = dev(np.full(3, np.nan))
    J.execute(J.SpMVOp, A, dev(np.array(c["x"])), y)
    np.testing.assert_array_equal(host(y), c["y"])


@pytest.mark.parametrize("sorted_rows", [True, False])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_coo_random(J, O, sorted_rows, dtype):
    m, n = 5000, 4000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(2).integers(0, 60, m),
                                     seed=4, dtype=dtype)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    if not sorted_rows:
        perm = np.random.default_rng(8).permutation(rows.size)
        rows, colind, val = rows[perm], colind[perm], val[perm]
    x = np.random.default_rng(3).uniform(-1, 1, n).astype(dtype)
    y0 = np.random.default_rng(4).uniform(-1, 1, m).astype(dtype)
    A = J.coo_tensor(dev(rows), dev(colind), dev(val), (m, n))
    y = dev(y0)
    J.execute(J.SpMVOp, A, dev(x), y, alpha=1.5, beta=0.5)
    ref = O.coo_spmv(rows, colind, val, x, m, alpha=1.5, beta=0.5, y0=y0)
    # magnitude reference through the equivalent CSR
    order = np.lexsort((colind, rows))
    cnt = np.bincount(rows - 1, minlength=m)
    rp = np.r_[0, np.cumsum(cnt)].astype(np.int32) + 1
    absref = O.csr_spmv_absref(rp, colind[order], val[order], x, 1.5, 0.5, y0)
    assert_within(host(y), ref, absref, dtype, "coo")


# ------------------------------------------------- strided dense operands

def _colmajor_view(J, a, pad, fill=float("nan")):
    """A view of the column-major array a inside a larger column-major buffer
    whose leading dimension is rows + pad (the padding rows hold `fill`)."""
    import torch
    from jlust_amd.tensor import leading_dim
    r, c = a.shape
    big = np.full((r + pad, c), fill, dtype=a.dtype, order="F")
    big[:r] = a
    v = dev(big)[:r]
    assert v.stride(0) == 1 and leading_dim(v) == r + pad
    del torch
    return v


@pytest.mark.parametrize("pad", [1, 4, 7])
@pytest.mark.parametrize("k", [5, 40, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_strided_views(J, O, pad, k, dtype):
    """B and C as column views of larger buffers (ldb = n + pad, ldc = m + pad;
    pad 4 keeps 16-byte alignment, 1 and 7 do not): the plain call and the
    prepared plan, beta != 0, and the padding rows of C left untouched."""
    m, n = 1500, 1300
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(k).integers(0, 30, m),
                                     seed=20 + pad, dtype=dtype)
    rng = np.random.default_rng(21)
    B = np.asfortranarray(rng.standard_normal((n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.standard_normal((m, k)).astype(dtype))
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    ref, _ = O.csr_spmm(rowptr, colind, val, B, 0.5, -1.5, C0)
    absref = O.csr_spmm_absref(rowptr, colind, val, B, 0.5, -1.5, C0)
    for how in ("plain", "plan"):
        Bv = _colmajor_view(J, B, pad)
        Cv = _colmajor_view(J, C0, pad, fill=7.0)
        if how == "plain":
            J.execute(J.SpMMOp, A, Bv, Cv, alpha=0.5, beta=-1.5)
        else:
            h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
            J.execute(h, Bv, Cv, alpha=0.5, beta=-1.5)
        assert_within(host(Cv), ref, absref, dtype, f"spmm {how} k={k} pad={pad}")
        base = Cv.as_strided((m + pad, k), (1, m + pad))     # the whole buffer
        assert (host(base)[m:] == 7.0).all(), f"spmm {how} wrote into the padding rows"


@pytest.mark.parametrize("pad", [1, 4, 7])
@pytest.mark.parametrize("K", [3, 64, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_strided_views(J, O, pad, K, dtype):
    """A (m x K, lda = m + pad) and B (K x n, ldb = K + pad) as column views of
    larger buffers: the plain call and the prepared plan."""
    m, n = 1200, 900
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(K).integers(0, 40, m),
                                     seed=30 + pad, dtype=dtype)
    rng = np.random.default_rng(31)
    A = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    Bm = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    c0 = rng.standard_normal(colind.size).astype(dtype)
    ref = O.csr_sddmm(rowptr, colind, A, Bm, 2.0, 0.25, c0)
    absref = O.csr_sddmm_absref(rowptr, colind, A, Bm, 2.0, 0.25, c0)
    for how in ("plain", "plan"):
        cv = dev(c0)
        Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n))
        Av, Bv = _colmajor_view(J, A, pad), _colmajor_view(J, Bm, pad)
        if how == "plain":
            J.execute(J.SDDMMOp, Av, Bv, Cs, alpha=2.0, beta=0.25)
        else:
            h = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
            J.execute(J.SDDMMOp, h, Av, Bv, Cs, alpha=2.0, beta=0.25)
        assert_within(host(cv), ref, absref, dtype, f"sddmm {how} K={K} pad={pad}")


@pytest.mark.parametrize("mask_kind", ["csr", "coo"])
@pytest.mark.parametrize("dtype,K", [(np.float64, 6500), (np.float32, 13000)])
def test_sddmm_k_beyond_lds(J, O, mask_kind, dtype, K):
    """K too large for a 32-row block of A in 48 KB of LDS (f64 K > 6110,
    f32 K > 12222): the direct kernel, which reads A's rows with stride lda;
    plain call and prepared plan, CSR and shuffled COO masks."""
    m, n = 300, 200
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(K).integers(0, 9, m),
                                     seed=50, dtype=dtype)
    rng = np.random.default_rng(51)
    A = np.asfortranarray(rng.uniform(-1, 1, (m, K)).astype(dtype))
    Bm = np.asfortranarray(rng.uniform(-1, 1, (K, n)).astype(dtype))
    c0 = rng.uniform(-1, 1, colind.size).astype(dtype)
    ref = O.csr_sddmm(rowptr, colind, A, Bm, 0.5, 1.5, c0)
    absref = O.csr_sddmm_absref(rowptr, colind, A, Bm, 0.5, 1.5, c0)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    perm = rng.permutation(colind.size) if mask_kind == "coo" else np.arange(colind.size)
    for how in ("plain", "plan"):
        cv = dev(c0[perm])
        if mask_kind == "csr":
            Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n))
        else:
            Cs = J.coo_tensor(dev(rows[perm]), dev(colind[perm]), cv, (m, n))
        if how == "plain":
            J.execute(J.SDDMMOp, dev(A), dev(Bm), Cs, alpha=0.5, beta=1.5)
        else:
            h = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
            J.execute(J.SDDMMOp, h, dev(A), dev(Bm), Cs, alpha=0.5, beta=1.5)
        assert_within(host(cv), ref[perm], absref[perm], dtype, f"{mask_kind} {how} K={K}")
