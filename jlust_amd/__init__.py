"""jlust_amd -- the sparse hot path of JLUST (klamike/jlust) on MI355X.

CSR/COO SpMV, CSR SpMM, CSR SDDMM and 16x16 BSR SpMM run as hand-written
gfx950 HIP kernels in ``libjlust_hip.so`` behind the C ABI of
``include/jlust_hip.h``.  This package is the host-side mirror of JLUST's
operator API for that path (src/ops.jl, src/backends.jl, src/convenience.jl,
src/tensor.jl, src/interop.jl), so code written against the reference reads
the same:

    A = csr_tensor(rowptr, colind, val, (m, n))          # torch GPU buffers
    execute(SpMVOp, A, x, y, alpha=2.0, beta=0.5)        # or mul_(y, A, x)
    h = prepare(HIPBackend(), SpMVOp, A); execute(h, x, y)
"""
from .errors import (DeviceMismatch, HIPError, IncompatibleExtents, IndexOriginMismatch,
                     InvalidLevelAccess, InvalidTensorFormat, JLUSTError, NoDevice,
                     NonCanonicalStorage, UnsupportedFormat, UnsupportedIndexType,
                     UnsupportedValueType)
from .formats import (CompressedLevel, DenseLevel, Formats, PeriodicLevel, ShiftedDiagLevel,
                      SingletonLevel, TensorFormat, dim2lvl, lvl2dim)
from .ops import (AbstractKernelHandle, AbstractUSTBackend, BBMSpMVOp, BlockSpMMOp, BlockSpMVOp,
                  HIPBackend, Op, OpType, SDDMMOp, SpMMOp, SpMVOp, default_backend, execute,
                  matmul, mul_, prepare, supports_backend, update_values_)
from .block_sparse import (BlockSparseMatrix, BlockStructureError, batch_mul, batch_mul_,
                           update_block_values_)
from .block_banded import BlockBandedMatrix
from .elementwise import (ElementwiseFn, abs_fn, affine_fn, exp_fn, identity_fn, log_fn, relu_fn,
                          sqrt_fn, square_fn)
from .convert import (convert_format, convert_index_type, convert_value_type, csc_tensor,
                      dcsr_tensor, sparse_to_dense)
from ._lib import preload
from .tensor import (CPUDevice, HIPDevice, OneBased, USTensor, ZeroBased, bsr_tensor,
                     coo_tensor, coordinates, csr_tensor, dense_matrix, extents, format,
                     has_coordinates, has_positions, index_origin, materialize, nnz, nonzeros,
                     periodic_csr_tensor, positions, shifted_diag_tensor, size, ust)

from . import hip_backend as _hip_backend  # noqa: F401  (the backend, loaded with the package)

__all__ = [n for n in dir() if not n.startswith("_")]
