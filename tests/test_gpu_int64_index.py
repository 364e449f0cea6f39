"""Int64 index buffers on the HIP path.  The reference's walker keeps the
index type as stored (ext/KernelAbstractionsExt/ops/_walker.jl:105-110); here
the buffers are narrowed to the Int32 the kernels take, on the device, once
per torch version of each buffer (jlust_hip_narrow_index_i64).  Every product
must then equal, bit for bit, the same product over Int32 copies of the
indices (COO SpMV, whose row runs meet in atomics, to 1e-12), and an index
beyond Int32 raises UnsupportedIndexType (src/errors.jl:4)."""
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


def _i64(a):
    return dev(np.asarray(a).astype(np.int64))


def test_csr_and_coo_spmv_int64(J):
    import torch
    m, n = 3000, 2500
    rp, ci, v = random_csr(m, n, density=0.004, seed=3)
    x = dev(np.random.default_rng(1).standard_normal(n))
    A32 = J.csr_tensor(dev(rp), dev(ci), dev(v), (m, n))
    A64 = J.csr_tensor(_i64(rp), _i64(ci), dev(v), (m, n))
    for rep in range(4):       # plain calls, then (third call on) each matrix's cached plan
        y32 = torch.zeros(m, dtype=torch.float64, device="cuda")
        J.execute(J.SpMVOp, A32, x, y32)
        y64 = torch.full((m,), float("nan"), dtype=torch.float64, device="cuda")
        J.execute(J.SpMVOp, A64, x, y64)
        assert torch.equal(y64, y32), f"call {rep}"
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A64)
    y64 = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(h, x, y64)
    hy = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(J.prepare(J.HIPBackend(), J.SpMVOp, A32), x, hy)
    assert torch.equal(y64, hy)
    rows = np.repeat(np.arange(m), np.diff(rp)) + 1
    C32 = J.coo_tensor(dev(rows.astype(np.int32)), dev(ci), dev(v), (m, n))
    C64 = J.coo_tensor(_i64(rows), _i64(ci), dev(v), (m, n))
    yc32 = torch.zeros(m, dtype=torch.float64, device="cuda")
    yc64 = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, C32, x, yc32, alpha=0.5)
    J.execute(J.SpMVOp, C64, x, yc64, alpha=0.5)
    # COO adds its row runs with atomics: equal up to the order of those additions
    torch.testing.assert_close(yc64, yc32, rtol=1e-12, atol=1e-12)


def test_int64_index_written_in_place_is_narrowed_again(J):
    import torch
    m, n = 400, 300
    rp, ci, v = random_csr(m, n, density=0.02, seed=5)
    x = dev(np.random.default_rng(2).standard_normal(n))
    A64 = J.csr_tensor(_i64(rp), _i64(ci), dev(v), (m, n))
    y = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, A64, x, y)
    # the first entry of the row whose first column is largest moves to
    # column 1, which that row does not hold (its columns stay sorted)
    firsts = [(int(ci[rp[r] - 1]), r) for r in range(m) if rp[r + 1] > rp[r]]
    first_col, r = max(firsts)
    assert first_col > 1
    lo = rp[r] - 1
    ci2 = ci.copy()
    ci2[lo] = 1
    A64.crd_buffers[1][lo] = 1
    y2 = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, A64, x, y2)
    ref = torch.zeros(m, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, J.csr_tensor(dev(rp), dev(ci2), dev(v), (m, n)), x, ref)
    assert torch.equal(y2, ref)
    assert not torch.equal(y2, y)


def test_spmm_sddmm_bsr_int64(J):
    import torch
    m, n, k = 700, 500, 24
    rp, ci, v = random_csr(m, n, density=0.01, seed=7, dtype=np.float32)
    B = dev(np.asfortranarray(np.random.default_rng(3).standard_normal((n, k)).astype(np.float32)))
    A32 = J.csr_tensor(dev(rp), dev(ci), dev(v), (m, n))
    A64 = J.csr_tensor(_i64(rp), _i64(ci), dev(v), (m, n))
    C32 = J.dense_matrix(m, k, dtype=torch.float32)
    C64 = J.dense_matrix(m, k, dtype=torch.float32)
    J.execute(J.SpMMOp, A32, B, C32)
    J.execute(J.SpMMOp, A64, B, C64)
    assert torch.equal(C32, C64)
    # SDDMM: the Int64 mask's own tensor is returned, its values written
    Ad = dev(np.asfortranarray(np.random.default_rng(4).standard_normal((m, k)).astype(np.float32)))
    Bd = dev(np.asfortranarray(np.random.default_rng(5).standard_normal((k, n)).astype(np.float32)))
    S32 = J.csr_tensor(dev(rp), dev(ci), dev(np.zeros_like(v)), (m, n))
    S64 = J.csr_tensor(_i64(rp), _i64(ci), dev(np.zeros_like(v)), (m, n))
    r32 = J.execute(J.SDDMMOp, Ad, Bd, S32)
    r64 = J.execute(J.SDDMMOp, Ad, Bd, S64)
    assert r64 is S64
    assert torch.equal(r32.val, S64.val)
    # BSR SpMM and SpMV over Int64 block pointers and columns
    mb, nb = 40, 30
    bp, bc, _ = random_csr(mb, nb, density=0.15, seed=9)
    bv = np.random.default_rng(6).standard_normal(bc.size * 256).astype(np.float32)
    Bb = dev(np.asfortranarray(np.random.default_rng(7).standard_normal((nb * 16, 32)).astype(np.float32)))
    X32 = J.bsr_tensor(dev(bp), dev(bc), dev(bv), (mb * 16, nb * 16))
    X64 = J.bsr_tensor(_i64(bp), _i64(bc), dev(bv), (mb * 16, nb * 16))
    D32 = J.dense_matrix(mb * 16, 32, dtype=torch.float32)
    D64 = J.dense_matrix(mb * 16, 32, dtype=torch.float32)
    J.execute(J.SpMMOp, X32, Bb, D32)
    J.execute(J.SpMMOp, X64, Bb, D64)
    assert torch.equal(D32, D64)
    xv = dev(np.random.default_rng(8).standard_normal(nb * 16).astype(np.float32))
    y32 = torch.zeros(mb * 16, dtype=torch.float32, device="cuda")
    y64 = torch.zeros(mb * 16, dtype=torch.float32, device="cuda")
    J.execute(J.SpMVOp, X32, xv, y32)
    J.execute(J.prepare(J.HIPBackend(), J.SpMVOp, X64), xv, y64)
    assert torch.equal(y32, y64)


def test_int64_index_beyond_int32_raises(J):
    import torch
    m, n = 10, 10
    rp = np.array([1, 2, 3] + [3] * 8, np.int64)
    ci = np.array([1, (1 << 31) + 4], np.int64)
    A = J.csr_tensor(_i64(rp), _i64(ci), dev(np.ones(2)), (m, n))
    with pytest.raises(J.UnsupportedIndexType):
        J.execute(J.SpMVOp, A, dev(np.ones(n)), torch.zeros(m, dtype=torch.float64, device="cuda"))
