"""Host-side structure of BlockSparseMatrix / BlockBandedMatrix (no GPU): the
constructor checks of src/block_sparse.jl:36-77, sizes, period starts of
src/block_banded.jl:129-137, the op tags, and that host-memory blocks are
refused rather than multiplied on the CPU."""
import numpy as np
import pytest
import torch

import jlust_amd as J


def csr(m, n, dtype=torch.float64):
    rowptr = np.arange(m + 1, dtype=np.int32)
    cols = np.arange(m, dtype=np.int32) % n
    return J.csr_tensor(rowptr, cols, torch.ones(m, dtype=dtype), (m, n), origin=J.ZeroBased())


def test_bsm_sizes_and_eltype():
    A = J.BlockSparseMatrix([[csr(2, 3), None, csr(2, 4)], [None, csr(5, 1), None]])
    assert A.size() == (7, 8) and A.size(1) == 7 and A.size(2) == 8
    assert A.row_sizes == [2, 5] and A.col_sizes == [3, 1, 4]
    assert A.dtype == torch.float64 and A.eltype() == torch.float64
    assert [(ij, r, c) for ij, _, r, c in A.placed_blocks()] == [((0, 0), 0, 0), ((0, 2), 0, 4),
                                                                  ((1, 1), 2, 3)]
    B = J.BlockSparseMatrix(np.array([[csr(2, 2), None], [None, csr(1, 1)]], dtype=object))
    assert B.size() == (3, 3)


@pytest.mark.parametrize("grid, match", [
    ([[csr(2, 3), csr(3, 3)]], "block row 1 has inconsistent sizes"),
    ([[csr(2, 3)], [csr(2, 4)]], "block col 1 has inconsistent sizes"),
    ([[csr(2, 3), csr(2, 3, torch.float32)]], "mixed element types"),
    ([[csr(2, 3), None], [None, None]], r"block row\(s\) \[2\] are entirely None"),
    ([[csr(2, 3), None]], r"block col\(s\) \[2\] are entirely None"),
    ([[csr(2, 3), "x"]], "must be a USTensor or None"),
    ([], "non-empty rectangular grid"),
    ([[csr(2, 2)], [csr(2, 2), None]], "non-empty rectangular grid"),
])
def test_bsm_constructor_errors(grid, match):
    with pytest.raises(J.BlockStructureError, match=match):
        J.BlockSparseMatrix(grid)


def test_bbm_sizes_and_starts():
    D = J.BlockSparseMatrix([[csr(4, 3), csr(4, 2)]])
    M = J.BlockBandedMatrix(D, csr(2, 5), csr(2, 5), 3, 4, 2, 5)
    assert M.size() == (3 * 4 + 2 * 2, 15) and M.bw == 1 and M.dtype == torch.float64
    assert M.d_starts() == [0, 6, 12]
    M2 = J.BlockBandedMatrix(csr(4, 5), [(csr(2, 5), csr(2, 5)), (csr(1, 5), csr(1, 5))],
                             3, 2, 4, [2, 1], 5)
    assert M2.size() == (3 * 4 + 2 * 2 + 1 * 1, 15)
    assert M2.d_starts() == [0, 7, 13]
    # rows of the assembled order: D1 C1 C2 | D2 C1 | D3
    rows = [(k, r) for k, _, r, _ in M2.placements()]
    assert rows == [(("diag", 0), 0), (("neg", 1, 0), 4), (("pos", 1, 0), 4), (("neg", 2, 0), 6),
                    (("pos", 2, 0), 6), (("diag", 1), 7), (("neg", 1, 1), 11),
                    (("pos", 1, 1), 11), (("diag", 2), 13)]
    M0 = J.BlockBandedMatrix(csr(4, 5), [], 3, 0, 4, [], 5)
    assert M0.size() == (12, 15) and M0.d_starts() == [0, 4, 8]


def test_bbm_errors():
    with pytest.raises(J.IncompatibleExtents):
        J.BlockBandedMatrix(csr(4, 5), csr(2, 4), csr(2, 5), 3, 4, 2, 5)
    with pytest.raises(J.BlockStructureError, match="coupling pairs"):
        J.BlockBandedMatrix(csr(4, 5), [[(csr(2, 5), csr(2, 5))]], 3, 1, 4, [2], 5)
    with pytest.raises(J.BlockStructureError, match="diagonal blocks for T"):
        J.BlockBandedMatrix([csr(4, 5)] * 2, [], 3, 0, 4, [], 5)
    with pytest.raises(J.BlockStructureError, match="mixed element types"):
        J.BlockBandedMatrix(csr(4, 5), csr(2, 5, torch.float32), csr(2, 5), 3, 4, 2, 5)
    with pytest.raises(J.UnsupportedFormat):
        J.BlockBandedMatrix(torch.zeros(4, 5), [], 3, 0, 4, [], 5)


def test_op_tags_and_host_memory_refused():
    assert repr(J.BlockSpMVOp) == "BlockSpMVOp" and J.BBMSpMVOp.tag == "BBMSpMV"
    A = J.BlockSparseMatrix([[csr(2, 3)]])
    with pytest.raises(J.UnsupportedFormat, match="HIP device"):
        J.matmul(A, torch.ones(3, dtype=torch.float64))
    with pytest.raises(TypeError):
        J.execute(J.BBMSpMVOp, A, torch.ones(3), torch.ones(2))


def test_shifted_diag_format():
    f = J.Formats.ShiftedDiag(torch.float64, shift=3, val=-1.5)
    assert f == J.Formats.ShiftedDiag(shift=3, val=-1.5)
    assert f != J.Formats.ShiftedDiag(shift=2, val=-1.5)
    assert f.levels[1] == J.ShiftedDiagLevel(3, -1.5)
    assert J.Formats.ShiftedDiag(torch.float32, val=0.1).levels[1].val == float(np.float32(0.1))
    u = J.shifted_diag_tensor(torch.float64, 4, 7, shift=3, val=2.0, device="cpu")
    assert J.nnz(u) == 0 and J.size(u) == (4, 7)
    d1 = J.Formats.DensedRight(1)
    assert J.supports_backend(J.HIPBackend(), J.SpMVOp(f, d1, d1))
