"""GPU parity of the prepared SpMM and SDDMM plans, COO-mask SDDMM and CSC
(scatter) SpMV against the CPU oracle.

Handles follow the cuSPARSE handle contract prepare -> execute(h, ...) ->
update_values!(h, ...) (ext/CUDAExt/ops/spmm.jl:8-70, sddmm.jl:10-76;
test/test_cuda.jl:318-332).  Bar: |out - ref| <= 1e-12 (fp64) / 1e-5 (fp32)
x (|alpha| |A||B| + |beta||C0|) elementwise; reference fixtures exactly.
"""
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


def _powerlaw_lengths(m, n, seed, long_rows=()):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 40, m)
    lens[rng.random(m) < 0.1] = 0              # empty rows
    for r, L in long_rows:
        lens[r] = min(L, n)
    return lens


# ------------------------------------------------------------------ SpMM

@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_handle_reference_fixture(J, dtype):
    """test/test_cuda.jl:318-332: prepare(SpMMOp; n_cols=2), execute,
    update_values!, execute -> C = [1 6; 6 3; 4 15] both times."""
    c = GOLDEN["spmm"][0]
    A = J.csr_tensor(dev(np.array(c["rowptr"], np.int32)), dev(np.array(c["colind"], np.int32)),
                     dev(np.array(c["val"], dtype)), (3, 3))
    B = dev(np.asfortranarray(np.array(c["B"], dtype)))
    C = J.dense_matrix(3, 2, dtype=A.dtype, fill=float("nan"))
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=2)
    J.execute(J.SpMMOp, h, B, C)
    np.testing.assert_array_equal(host(C), np.array(c["C"], dtype))
    C.fill_(0)
    J.update_values_(h, A)
    J.execute(h, B, C)
    np.testing.assert_array_equal(host(C), np.array(c["C"], dtype))


@pytest.mark.parametrize("k", [1, 5, 32, 64, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_spmm_plan_long_rows(J, O, k, dtype):
    """Rows above 1024 entries are split into segments; every row checked."""
    import torch
    m, n = 4000, 6000
    lens = _powerlaw_lengths(m, n, 3 + k, long_rows=[(7, 1025), (100, 3000), (3999, 5000),
                                                     (2000, 1024)])
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=k, dtype=dtype)
    B = np.asfortranarray(np.random.default_rng(5).standard_normal((n, k)).astype(dtype))
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    info = h.info()
    assert info["split_rows"] == 3, info          # 1025, 3000, 5000 (1024 is not split)
    assert info["segments"] == 5 + 12 + 20, info
    C = J.dense_matrix(m, k, dtype=A.dtype, fill=float("nan"))
    J.execute(h, dev(B), C)
    ref, _ = O.csr_spmm(rowptr, colind, val, B)
    absref = O.csr_spmm_absref(rowptr, colind, val, B)
    assert_within(host(C), ref, absref, dtype, f"spmm plan k={k}")
    # Rows that are not split equal the plain call bit for bit; the plan is
    # deterministic run to run.
    C2 = J.dense_matrix(m, k, dtype=A.dtype, fill=float("nan"))
    J.execute(J.SpMMOp, A, dev(B), C2)
    keep = np.ones(m, bool)
    keep[[7, 100, 3999]] = False
    np.testing.assert_array_equal(host(C)[keep], host(C2)[keep])
    C3 = J.dense_matrix(m, k, dtype=A.dtype, fill=0.0)
    J.execute(h, dev(B), C3)
    np.testing.assert_array_equal(host(C3), host(C))
    del torch


@pytest.mark.parametrize("skip", [False, True])
def test_spmm_plan_beta_and_skip_empty_rows(J, O, skip):
    m, n, k = 3000, 2500, 48
    lens = _powerlaw_lengths(m, n, 11, long_rows=[(5, 2000), (2999, 1500)])
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=12, origin=0)
    rng = np.random.default_rng(13)
    B = np.asfortranarray(rng.standard_normal((n, k)))
    C0 = np.asfortranarray(rng.standard_normal((m, k)))
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n), origin=J.ZeroBased())
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k, skip_empty_rows=skip)
    C = dev(C0)
    J.execute(h, dev(B), C, alpha=-1.5, beta=0.25)
    ref, _ = O.csr_spmm(rowptr, colind, val, B, -1.5, 0.25, C0, origin=0)
    absref = O.csr_spmm_absref(rowptr, colind, val, B, -1.5, 0.25, C0, origin=0)
    got = host(C)
    empty = np.diff(rowptr) == 0
    if skip:
        np.testing.assert_array_equal(got[empty], C0[empty])    # untouched, beta or not
        ref[empty] = C0[empty]
    assert_within(got, ref, absref, np.float64, f"skip={skip}")


def test_spmm_plan_values_and_k_change(J, O):
    """In-place writes to A's values are read by the next execute; another
    value tensor (execute(h, A2, B, C) / update_values_) is taken; a B with
    other columns rebuilds the plan."""
    m, n = 2500, 3000
    lens = _powerlaw_lengths(m, n, 21, long_rows=[(3, 4000)])
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=22)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A)
    rng = np.random.default_rng(23)
    for step, k in enumerate((16, 16, 96, 96)):
        B = np.asfortranarray(rng.standard_normal((n, k)))
        v = rng.uniform(-1, 1, val.size)
        if step == 3:
            A2 = J.csr_tensor(J.positions(A, 2), J.coordinates(A, 2), dev(v), (m, n))
            C = J.dense_matrix(m, k, dtype=A.dtype)
            J.execute(h, A2, dev(B), C)
        else:
            J.nonzeros(h.u_A).copy_(dev(v))
            C = J.dense_matrix(m, k, dtype=A.dtype)
            J.execute(h, J.ust(dev(B)), J.ust(C))
        assert h.k == k
        ref, _ = O.csr_spmm(rowptr, colind, v, B)
        absref = O.csr_spmm_absref(rowptr, colind, v, B)
        assert_within(host(C), ref, absref, np.float64, f"step {step} k={k}")


# ----------------------------------------------------------------- SDDMM

@pytest.mark.parametrize("fmt", ["CSR", "COO"])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_reference_fixture_plain_and_plan(J, fmt, dtype):
    """test/test_emitter.jl:276-307, test/test_cuda.jl:417-432: [1,1,1,1,2]."""
    c = next(c for c in GOLDEN["sddmm"] if c["format"] == fmt)
    A = dev(np.asfortranarray(np.array(c["A"], dtype)))
    B = dev(np.asfortranarray(np.array(c["B"], dtype)))

    def mask_tensor():
        if fmt == "CSR":
            return J.csr_tensor(dev(np.array(c["rowptr"], np.int32)),
                                dev(np.array(c["colind"], np.int32)),
                                dev(np.array(c["c0"], dtype)), (3, 3))
        return J.coo_tensor(dev(np.array(c["rows"], np.int32)), dev(np.array(c["cols"], np.int32)),
                            dev(np.array(c["c0"], dtype)), (3, 3))
    C = mask_tensor()
    J.execute(J.SDDMMOp, A, B, C, beta=c["beta"])
    np.testing.assert_array_equal(host(J.nonzeros(C)), np.array(c["cval"], dtype))
    C = mask_tensor()
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, A, B, C)
    J.execute(J.SDDMMOp, h, A, B, C, beta=c["beta"])
    np.testing.assert_array_equal(host(J.nonzeros(C)), np.array(c["cval"], dtype))
    C2 = mask_tensor()
    J.update_values_(h, C2)
    J.execute(h, A, B)
    np.testing.assert_array_equal(host(J.nonzeros(C2)), np.array(c["cval"], dtype))


@pytest.mark.parametrize("K", [1, 4, 8, 32, 128])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_sddmm_plan_csr_long_rows(J, O, K, dtype):
    """A mask with rows of up to 20000 entries (work items split) and empty
    row blocks (no items), against the oracle on every entry."""
    m, n = 3000, 25000
    lens = _powerlaw_lengths(m, n, K, long_rows=[(10, 20000), (1500, 9000)])
    lens[200:400] = 0                          # whole row blocks without entries
    rowptr, colind, _ = random_csr(m, n, lengths=lens, seed=K + 1, dtype=dtype)
    rng = np.random.default_rng(K)
    A = np.asfortranarray(rng.standard_normal((m, K)).astype(dtype))
    B = np.asfortranarray(rng.standard_normal((K, n)).astype(dtype))
    S = rng.uniform(0.5, 1.5, colind.size).astype(dtype)
    C0 = rng.standard_normal(colind.size).astype(dtype)
    C = J.csr_tensor(dev(rowptr), dev(colind), dev(C0), (m, n))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, dev(A), dev(B), C)
    info = h.info()
    assert info["work_items"] >= 6 + (m // 32 - 8), info
    J.execute(h, dev(A), dev(B), C, alpha=0.75, beta=-0.5, mask=dev(S))
    ref = O.csr_sddmm(rowptr, colind, A, B, 0.75, -0.5, C0, S)
    absref = O.csr_sddmm_absref(rowptr, colind, A, B, 0.75, -0.5, C0, S)
    assert_within(host(J.nonzeros(C)), ref, absref, dtype, f"sddmm plan K={K}")


@pytest.mark.parametrize("unsorted", [False, True])
@pytest.mark.parametrize("K", [3, 64])
def test_sddmm_coo_plain_and_plan(J, O, unsorted, K):
    m, n = 2000, 1500
    rowptr, colind, _ = random_csr(m, n, lengths=_powerlaw_lengths(m, n, 31), seed=32)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
    cols = colind.copy()
    rng = np.random.default_rng(33)
    if unsorted:
        p = rng.permutation(rows.size)
        rows, cols = rows[p], cols[p]
    A = np.asfortranarray(rng.standard_normal((m, K)))
    B = np.asfortranarray(rng.standard_normal((K, n)))
    C0 = rng.standard_normal(rows.size)
    S = rng.uniform(0.5, 1.5, rows.size)
    ref = O.coo_sddmm(rows, cols, A, B, 1.25, 0.5, C0, S)
    absref = np.abs(O.coo_sddmm(rows, cols, np.abs(A), np.abs(B), 1.25, 0.5, np.abs(C0),
                                np.abs(S)))
    C = J.coo_tensor(dev(rows), dev(cols), dev(C0), (m, n))
    J.execute(J.SDDMMOp, dev(A), dev(B), C, alpha=1.25, beta=0.5, mask=dev(S))
    assert_within(host(J.nonzeros(C)), ref, absref, np.float64, f"plain COO unsorted={unsorted}")
    C = J.coo_tensor(dev(rows), dev(cols), dev(C0), (m, n))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, C, n_inner=K)
    assert h.info()["reordered"] == unsorted
    J.execute(h, dev(A), dev(B), alpha=1.25, beta=0.5, mask=dev(S))
    assert_within(host(J.nonzeros(C)), ref, absref, np.float64, f"COO plan unsorted={unsorted}")


def test_sddmm_coo_row_out_of_range_is_rejected(J):
    C = J.coo_tensor(dev(np.array([1, 9], np.int32)), dev(np.array([1, 2], np.int32)),
                     dev(np.zeros(2)), (3, 3))
    with pytest.raises(J.NonCanonicalStorage):
        J.prepare(J.HIPBackend(), J.SDDMMOp, C, n_inner=2)


# -------------------------------------------------------------- CSC SpMV

def _csc(O, rowptr, colind, val, n, origin=1):
    return O.csr_to_csc(rowptr, colind, val, n, origin)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csc_spmv_reference_answer(J, O, dtype):
    c = GOLDEN["spmv"][0]
    cp, ri, cv = _csc(O, np.array(c["rowptr"]), np.array(c["colind"]), np.array(c["val"], dtype), 3)
    A = J.csc_tensor(dev(cp), dev(ri), dev(cv), (3, 3))
    y = dev(np.full(3, np.nan, dtype))
    J.execute(J.SpMVOp, A, dev(np.array(c["x"], dtype)), y)
    np.testing.assert_array_equal(host(y), np.array(c["y"], dtype))


@pytest.mark.parametrize("origin", [1, 0])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_csc_spmv_random(J, O, origin, dtype):
    m, n = 5000, 7000
    lens = np.random.default_rng(51).integers(0, 30, m)
    lens[::50] = 0
    lens[3] = 6000                             # a long row = many columns hitting it
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=52, origin=origin, dtype=dtype)
    cp, ri, cv = _csc(O, rowptr, colind, val, n, origin)
    rng = np.random.default_rng(53)
    x = rng.uniform(-1, 1, n).astype(dtype)
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    A = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n),
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    for alpha, beta in ((1.0, 0.0), (-2.5, 0.75)):
        y = dev(y0)
        J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
        ref = O.csc_spmv(cp, ri, cv, x, m, alpha, beta, y0, origin=origin)
        absref = O.csr_spmv_absref(rowptr, colind, val, x, alpha, beta, y0, origin=origin)
        assert_within(host(y), ref, absref, dtype, f"csc alpha={alpha} beta={beta}")


def test_csc_spmv_input_fn_and_output_fn(J, O):
    m, n = 800, 600
    rowptr, colind, val = random_csr(m, n, density=0.02, seed=61)
    cp, ri, cv = _csc(O, rowptr, colind, val, n)
    x = np.random.default_rng(62).uniform(-1, 1, n)
    A = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n))
    y = dev(np.zeros(m))
    J.execute(J.SpMVOp, A, dev(x), y, input_fn=J.abs_fn)
    ref = O.csc_spmv(cp, ri, cv, np.abs(x), m)
    absref = O.csr_spmv_absref(rowptr, colind, val, np.abs(x))
    assert_within(host(y), ref, absref, np.float64, "csc input_fn")
    with pytest.raises(J.UnsupportedFormat, match="output_fn"):
        J.execute(J.SpMVOp, A, dev(x), y, output_fn=J.abs_fn)


# ------------------------------------------------------------- BSR plans

def _rect_bsr(mb, nb, b1, b2, per_row, seed, dtype, row_major, origin=1):
    """Random BSR of b1 x b2 blocks with small-integer values (exact sums),
    some stored zeros; flat values in the block order asked for."""
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, per_row + 1, mb)
    bcols = [np.sort(rng.choice(nb, min(c, nb), replace=False)) for c in counts]
    browptr = (np.r_[0, np.cumsum([c.size for c in bcols])] + origin).astype(np.int32)
    bcolind = (np.concatenate(bcols) + origin).astype(np.int32)
    blocks = rng.integers(-4, 5, (bcolind.size, b1, b2)).astype(dtype)
    blocks[blocks == 4] = 0
    flat = blocks.reshape(-1) if row_major else blocks.transpose(0, 2, 1).reshape(-1)
    return browptr, bcolind, np.ascontiguousarray(flat)


@pytest.mark.parametrize("b1,b2,dtype,row_major,path", [
    (16, 16, np.float32, True, "mfma"),
    (16, 16, np.float32, False, "mfma"),
    (4, 8, np.float64, True, "csr_expansion"),
    (3, 5, np.float32, False, "csr_expansion"),
    (16, 16, np.float64, True, "mfma"),
    (16, 16, np.float64, False, "mfma"),
])
def test_bsr_spmm_plan(J, O, b1, b2, dtype, row_major, path):
    """prepare(SpMMOp, A::BSR; n_cols=k): the chosen path, the product
    against the oracle (exact on integer data), bit-identity with the plain
    call, values written in place seen by the next execute, update_values_
    with another tensor, and a k change rebuilding the plan."""
    import torch
    mb, nb, k = 45, 38, 20
    bp, bc, flat = _rect_bsr(mb, nb, b1, b2, 6, 300 + b1 + 10 * b2, dtype, row_major)
    vals = dev(flat)
    A = J.bsr_tensor(dev(bp), dev(bc), vals, (mb * b1, nb * b2), (b1, b2), row_major)
    tdt = torch.float64 if dtype == np.float64 else torch.float32
    rng = np.random.default_rng(9)
    B = np.asfortranarray(rng.integers(-3, 4, (nb * b2, k)).astype(dtype))
    C0 = np.asfortranarray(rng.integers(-3, 4, (mb * b1, k)).astype(dtype))

    def ref(v, Bm, a, b):
        return O.bsr_spmm(bp, bc, v, b1, Bm, a, b, C0[:, :Bm.shape[1]].copy(order="F"),
                          row_major_blocks=row_major, b2=b2)

    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    assert h.info()["path"] == path
    C = J.dense_matrix(mb * b1, k, dtype=tdt)
    C.copy_(dev(C0))
    J.execute(J.SpMMOp, h, dev(B), C, alpha=1.5, beta=-1.0)
    np.testing.assert_array_equal(host(C), ref(flat, B, 1.5, -1.0))
    C2 = J.dense_matrix(mb * b1, k, dtype=tdt)
    C2.copy_(dev(C0))
    J.execute(J.SpMMOp, A, dev(B), C2, alpha=1.5, beta=-1.0)
    assert np.array_equal(host(C2), host(C))
    # values written in place
    vals.mul_(-2)
    J.execute(J.SpMMOp, h, dev(B), C, alpha=1.0, beta=0.0)
    np.testing.assert_array_equal(host(C), ref(-2 * flat, B, 1.0, 0.0))
    # another value tensor through update_values_, then execute(h, A, B, C)
    flat3 = np.ascontiguousarray(flat + 1).astype(dtype)
    A3 = J.bsr_tensor(dev(bp), dev(bc), dev(flat3), (mb * b1, nb * b2), (b1, b2), row_major)
    J.update_values_(h, A3)
    J.execute(J.SpMMOp, h, dev(B), C, alpha=1.0, beta=0.0)
    np.testing.assert_array_equal(host(C), ref(flat3, B, 1.0, 0.0))
    # a different k rebuilds the plan
    B5 = np.asfortranarray(B[:, :5])
    C5 = J.dense_matrix(mb * b1, 5, dtype=tdt)
    J.execute(J.SpMMOp, h, A, dev(B5), C5, alpha=1.0, beta=0.0)
    np.testing.assert_array_equal(host(C5), ref(-2 * flat, B5, 1.0, 0.0))
