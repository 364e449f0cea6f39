"""Host-side mirror of JLUST's tensor/format/operator API (no GPU needed):
formats and their dim<->level maps against the reference's fixtures, tensor
constructors and accessors, capability table, dispatch errors."""
import json
import os

import numpy as np
import pytest
import torch

import jlust_amd as J
from jlust_amd.formats import is_coo_shaped, is_csr_shaped

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))
FMT = {"CSR": J.Formats.CSR, "CSC": J.Formats.CSC, "COO": J.Formats.COO,
       "DCSR": J.Formats.DCSR, "BSRRight2x2": J.Formats.BSRRight((2, 2)),
       "BSRLeft2x2": J.Formats.BSRLeft((2, 2))}


def test_dim2lvl_fixtures():
    for c in GOLDEN["dim2lvl"]["cases"]:
        f = FMT[c["format"]]
        assert J.dim2lvl(f, c["dims"]) == c["lvl"], c
        assert J.lvl2dim(f, c["lvl"]) == c["dims"], c
    for c in GOLDEN["dim2lvl"]["size_cases"]:
        assert J.dim2lvl(FMT[c["format"]], c["dims"], as_size=True) == c["lvl"], c


def test_dim2lvl_round_trip_grid():
    """test/test_formats.jl:93-102, on the formats of the hot path."""
    for f in (J.Formats.CSR, J.Formats.CSC, J.Formats.BSRRight((16, 16)),
              J.Formats.BSRLeft((2, 4))):
        for i in range(17):
            for j in range(0, 111, 7):
                assert J.lvl2dim(f, J.dim2lvl(f, [i, j])) == [i, j]


def test_format_identity_and_shape_predicates():
    assert J.Formats.CSR == J.Formats.CSR and J.Formats.CSR != J.Formats.CSC
    assert J.Formats.BSRRight((16, 16)) == J.Formats.BSRRight((16, 16))
    assert J.Formats.BSRRight((16, 16)) != J.Formats.BSRLeft((16, 16))
    assert is_csr_shaped(J.Formats.CSR) and not is_csr_shaped(J.Formats.CSC)
    assert is_coo_shaped(J.Formats.COO) and not is_coo_shaped(J.Formats.CSR)
    assert J.Formats.DensedRight(2).is_dense and not J.Formats.CSR.is_dense
    assert len(J.Formats.BSRRight((16, 16)).levels) == 4


def test_supports_backend_table():
    """Mirrors test/test_emitter.jl:33-62 for the HIP backend's formats."""
    be = J.HIPBackend()
    d1, d2 = J.Formats.DensedRight(1), J.Formats.DensedRight(2)
    assert J.supports_backend(be, J.SpMVOp(J.Formats.CSR, d1, d1))
    assert J.supports_backend(be, J.SpMVOp(J.Formats.COO, d1, d1))
    assert not J.supports_backend(be, J.SpMVOp(d2, d1, d1))
    assert not J.supports_backend(be, J.SpMVOp(J.Formats.CSR, d1, J.Formats.CSR))
    assert J.supports_backend(be, J.SpMMOp(J.Formats.CSR, d2, d2))
    assert not J.supports_backend(be, J.SpMMOp(d2, d2, d2))
    assert J.supports_backend(be, J.SpMMOp(J.Formats.BSRRight((16, 16)), d2, d2))
    assert J.supports_backend(be, J.SpMMOp(J.Formats.BSRLeft((16, 16)), d2, d2))
    # Other block shapes and BSR SpMV go through the device CSR expansion.
    assert J.supports_backend(be, J.SpMMOp(J.Formats.BSRRight((8, 8)), d2, d2))
    assert J.supports_backend(be, J.SpMMOp(J.Formats.BSRLeft((2, 3)), d2, d2))
    assert J.supports_backend(be, J.SpMVOp(J.Formats.BSRRight((4, 8)), d1, d1))
    assert J.supports_backend(be, J.SDDMMOp(d2, d2, J.Formats.CSR))
    assert not J.supports_backend(be, J.SDDMMOp(J.Formats.CSR, d2, J.Formats.CSR))
    assert not J.supports_backend(object(), J.SpMVOp(J.Formats.CSR, d1, d1))


def test_supports_backend_every_sparse_format():
    """Every non-dense operand format the mirror defines, as the reference's
    EmitterBackend claims them (ext/KernelAbstractionsExt/
    KernelAbstractionsExt.jl:31-37: any non-dense A for SpMV/SpMM;
    ops/sddmm.jl:12-14: any non-dense C for SDDMM, here the formats with
    stored values per entry)."""
    be = J.HIPBackend()
    d1, d2 = J.Formats.DensedRight(1), J.Formats.DensedRight(2)
    sparse = [J.Formats.CSR, J.Formats.CSC, J.Formats.COO, J.Formats.DCSR,
              J.Formats.BSRRight((16, 16)), J.Formats.BSRLeft((2, 3)),
              J.Formats.ShiftedDiag(torch.float64, shift=1), J.Formats.PeriodicCSR(3, 4, 5)]
    for f in sparse:
        assert J.supports_backend(be, J.SpMVOp(f, d1, d1)), f
        assert J.supports_backend(be, J.SpMMOp(f, d2, d2)), f
    for f in (J.Formats.CSR, J.Formats.CSC, J.Formats.COO, J.Formats.DCSR):
        assert J.supports_backend(be, J.SDDMMOp(d2, d2, f)), f
    assert not J.supports_backend(be, J.SDDMMOp(d2, d2, J.Formats.ShiftedDiag(torch.float64)))


def fixture_csr(origin=1):
    c = GOLDEN["spmv"][0 if origin == 1 else 1]
    return J.csr_tensor(torch.tensor(c["rowptr"], dtype=torch.int32),
                        torch.tensor(c["colind"], dtype=torch.int32),
                        torch.tensor(c["val"], dtype=torch.float64), (3, 3),
                        origin=J.OneBased() if origin == 1 else J.ZeroBased())


def test_tensor_accessors():
    A = fixture_csr()
    assert J.nnz(A) == 5 and J.size(A) == (3, 3) and J.size(A, 1) == 3
    assert J.format(A) == J.Formats.CSR and J.index_origin(A) == J.OneBased()
    assert J.positions(A, 2).tolist() == [1, 3, 4, 6]
    assert J.coordinates(A, 2).tolist() == [1, 3, 2, 1, 3]
    assert J.has_positions(A, 2) and not J.has_positions(A, 1)
    with pytest.raises(J.InvalidLevelAccess):
        J.positions(A, 1)
    with pytest.raises(J.InvalidLevelAccess):
        J.coordinates(A, 3)
    C = J.coo_tensor(np.array([1, 1, 2], np.int32), np.array([1, 3, 2], np.int32),
                     np.array([1.0, 2.0, 3.0]), (2, 3))
    assert J.coordinates(C, 1).tolist() == [1, 1, 2] and not J.has_positions(C, 1)
    B = J.bsr_tensor(np.array([1, 2], np.int32), np.array([1], np.int32),
                     np.zeros(256, np.float32), (16, 16))
    assert J.nnz(B) == 256 and J.format(B) == J.Formats.BSRRight((16, 16))   # nnz = nnzb*b^2


def test_dense_views_are_column_major():
    B = J.dense_matrix(5, 3, dtype=torch.float64, device="cpu")
    assert B.stride() == (1, 5)
    u = J.ust(B)
    assert u.format == J.Formats.DensedRight(2) and u.extents == (5, 3)
    with pytest.raises(J.NonCanonicalStorage):
        J.ust(torch.zeros(5, 3))          # row-major
    assert J.ust(torch.zeros(4)).format == J.Formats.DensedRight(1)


def test_materialize_host_to_host():
    """Moving between host buffers keeps the data; an origin change runs on
    the HIP device (tests/test_gpu_convert.py), so host to host it raises."""
    A = fixture_csr(origin=1)
    B = J.materialize(A, J.CPUDevice())
    assert J.positions(B, 2).tolist() == J.positions(A, 2).tolist()
    assert J.index_origin(B) == J.OneBased()
    with pytest.raises(J.UnsupportedFormat, match="HIP device"):
        J.materialize(A, J.CPUDevice(), origin=J.ZeroBased())


def test_host_memory_has_no_cpu_fallback():
    """Host tensors are rejected before any GPU call: this package ships no
    CPU path (JLUST's CPU path is EmitterBackend, not reproduced here)."""
    A = fixture_csr()
    with pytest.raises(J.UnsupportedFormat, match="host memory"):
        J.execute(J.SpMVOp, A, torch.ones(3, dtype=torch.float64),
                  torch.zeros(3, dtype=torch.float64))
    with pytest.raises(J.UnsupportedFormat):
        J.default_backend(A, J.SpMVOp)


def test_op_construction():
    d1 = J.Formats.DensedRight(1)
    op = J.SpMVOp(J.Formats.CSR, d1, d1)
    assert op.tag == "SpMV" and op.formats[0] == J.Formats.CSR
    assert op == J.SpMVOp(J.Formats.CSR, d1, d1)
    assert repr(J.SpMVOp) == "SpMVOp"


def test_execute_rejects_non_op():
    with pytest.raises(TypeError):
        J.execute("SpMV", fixture_csr())


def test_elementwise_fns_and_prepare_keywords():
    assert J.affine_fn(2.0) == J.ElementwiseFn(1, 2.0, 0.0) and repr(J.abs_fn) == "abs"
    from jlust_amd.elementwise import is_identity
    assert is_identity(None) and is_identity(J.identity_fn) and not is_identity(J.exp_fn)
    with pytest.raises(TypeError, match="unexpected keywords"):
        J.prepare(J.HIPBackend(), J.SpMVOp, fixture_csr(), skip_empty_rows=True)
