"""USTensor container and constructors (src/tensor.jl, src/interop.jl).

Buffers are torch tensors.  Index buffers are int32 (JLUST's GPU index type)
and keep the tensor's index origin; dense operands are column-major like
Julia arrays (stride(0) == 1 for a matrix), so a dense USTensor over a torch
tensor is the zero-copy `ust(A)` of src/interop.jl:36-46.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional, Tuple

import numpy as np
import torch

from .errors import (DeviceMismatch, IncompatibleExtents, InvalidLevelAccess,
                     NonCanonicalStorage)
from .formats import Formats, TensorFormat


class AbstractIndexOrigin:
    offset = 0

    def __eq__(self, other):
        return type(self) is type(other)

    def __hash__(self):
        return hash(type(self))

    def __repr__(self):
        return f"{type(self).__name__}()"


class OneBased(AbstractIndexOrigin):
    offset = 1


class ZeroBased(AbstractIndexOrigin):
    offset = 0


class CPUDevice:
    def __repr__(self):
        return "CPUDevice()"


@dataclass(frozen=True)
class HIPDevice:
    """A ROCm GPU (the counterpart of CUDADevice, src/tensor.jl:16-19)."""
    id: int = 0

    @property
    def torch(self):
        return torch.device("cuda", self.id)


def _as_torch(a) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a
    if isinstance(a, np.ndarray):
        return torch.from_numpy(a)
    return torch.as_tensor(a)


@dataclass
class USTensor:
    """src/tensor.jl:29-43: extents, format, per-level pos/crd buffers, values
    and the owner kept alive for zero-copy views."""
    extents: Tuple[int, ...]
    format: TensorFormat
    pos_buffers: Tuple[Optional[torch.Tensor], ...]
    crd_buffers: Tuple[Optional[torch.Tensor], ...]
    val: torch.Tensor
    owner: Any = None
    origin: AbstractIndexOrigin = OneBased()

    @property
    def dtype(self):
        return self.val.dtype

    @property
    def device(self) -> torch.device:
        return self.val.device

    def __repr__(self):
        return (f"USTensor({'x'.join(map(str, self.extents))}, {self.format}, "
                f"nnz={nnz(self)}, {self.dtype}, {self.device}, {self.origin})")


# ----------------------------------------------------------------- accessors

def nonzeros(u: USTensor) -> torch.Tensor:
    return u.val


def nnz(u: USTensor) -> int:
    """length(val) (src/tensor.jl:111); for BSR that is nnzb*b1*b2."""
    return u.val.numel()


def format(u: USTensor) -> TensorFormat:  # noqa: A001  (JLUST name)
    return u.format


def extents(u: USTensor):
    return u.extents


def index_origin(u: USTensor) -> AbstractIndexOrigin:
    return u.origin


def positions(u: USTensor, level: int) -> torch.Tensor:
    """1-based level index, like the reference (src/tensor.jl:91-98)."""
    if not 1 <= level <= len(u.pos_buffers):
        raise InvalidLevelAccess(f"level {level} out of range")
    p = u.pos_buffers[level - 1]
    if p is None:
        raise InvalidLevelAccess(f"level {level} has no position buffer")
    return p


def coordinates(u: USTensor, level: int) -> torch.Tensor:
    if not 1 <= level <= len(u.crd_buffers):
        raise InvalidLevelAccess(f"level {level} out of range")
    c = u.crd_buffers[level - 1]
    if c is None:
        raise InvalidLevelAccess(f"level {level} has no coordinate buffer")
    return c


def has_positions(u: USTensor, level: int) -> bool:
    return 1 <= level <= len(u.pos_buffers) and u.pos_buffers[level - 1] is not None


def has_coordinates(u: USTensor, level: int) -> bool:
    return 1 <= level <= len(u.crd_buffers) and u.crd_buffers[level - 1] is not None


def size(u: USTensor, d: Optional[int] = None):
    return u.extents if d is None else u.extents[d - 1]


# -------------------------------------------------------------- constructors

def csr_tensor(rowptr, colind, nzval, dims, origin: AbstractIndexOrigin = OneBased()) -> USTensor:
    """src/interop.jl:57-67; buffers are not copied."""
    m, n = dims
    return USTensor((int(m), int(n)), Formats.CSR, (None, _as_torch(rowptr)),
                    (None, _as_torch(colind)), _as_torch(nzval), None, origin)


def coo_tensor(rows, cols, nzval, dims, origin: AbstractIndexOrigin = OneBased(),
               sorted: bool = False) -> USTensor:  # noqa: A002  (JLUST keyword)
    """src/interop.jl:248-260: rows are the compressed level's crd, cols the
    singleton level's crd, no pos buffer."""
    m, n = dims
    return USTensor((int(m), int(n)), Formats.COO, (None, None),
                    (_as_torch(rows), _as_torch(cols)), _as_torch(nzval), None, origin)


def bsr_tensor(browptr, bcolind, nzval, dims, blocksize=(16, 16), row_major_blocks: bool = True,
               origin: AbstractIndexOrigin = OneBased()) -> USTensor:
    """BSR over caller buffers, laid out as the reference's BSR adapter does
    (ext/CUDAExt/CUDAExt.jl:144-156): pos/crd at level 2, values block-major,
    row-major inside a block for BSRRight ('R'), column-major for BSRLeft."""
    m, n = dims
    fmt = Formats.BSRRight(blocksize) if row_major_blocks else Formats.BSRLeft(blocksize)
    return USTensor((int(m), int(n)), fmt, (None, _as_torch(browptr), None, None),
                    (None, _as_torch(bcolind), None, None), _as_torch(nzval).reshape(-1), None,
                    origin)


def shifted_diag_tensor(dtype, n_rows: int, n_cols: int, shift: int = 0, val=1.0,
                        device="cuda") -> USTensor:
    """src/interop.jl:167-180: a structural shifted scaled identity (row r
    holds val at column r + shift) with no pos/crd/val storage."""
    fmt = Formats.ShiftedDiag(dtype, shift=shift, val=val)
    return USTensor((int(n_rows), int(n_cols)), fmt, (None, None), (None, None),
                    torch.empty(0, dtype=dtype, device=device), None, OneBased())


def periodic_csr_tensor(block: USTensor, periods: int) -> USTensor:
    """src/interop.jl:198-212: kron(I(T), block) without copying the block's
    buffers (pos/crd at level 3, the block kept as owner)."""
    from .errors import UnsupportedFormat
    if block.format != Formats.CSR:
        raise UnsupportedFormat(block.format, "HIPBackend",
                                f"periodic_csr_tensor: block must be CSR-formatted (got {block.format})")
    br, bc = block.extents
    fmt = Formats.PeriodicCSR(int(periods), br, bc)
    return USTensor((int(periods) * br, int(periods) * bc), fmt, (None, None, block.pos_buffers[1]),
                    (None, None, block.crd_buffers[1]), block.val, block, block.origin)


def ust(a) -> USTensor:
    """Zero-copy dense view of a vector or a column-major matrix
    (src/interop.jl:36-46)."""
    if isinstance(a, USTensor):
        return a
    t = _as_torch(a)
    if t.dim() == 1:
        return USTensor((t.shape[0],), Formats.DensedRight(1), (None,), (None,), t, t)
    if t.dim() == 2:
        if t.shape[0] > 1 and t.stride(0) != 1:
            raise NonCanonicalStorage(
                "dense matrices are column-major (Julia layout): expected stride(0) == 1, got "
                f"strides {tuple(t.stride())}; use jlust_amd.dense_matrix() or tensor.t().contiguous().t()")
        return USTensor(tuple(t.shape), Formats.DensedRight(2), (None, None), (None, None), t, t)
    raise IncompatibleExtents(f"ust: {t.dim()}-D arrays are not supported")


def dense_matrix(m: int, n: int, dtype=torch.float64, device="cuda", fill=None) -> torch.Tensor:
    """An m x n column-major torch matrix (ld = m)."""
    t = torch.empty((n, m), dtype=dtype, device=device).t()
    if fill is not None:
        t.fill_(fill)
    return t


def leading_dim(t: torch.Tensor) -> int:
    """Column stride of a column-major matrix (>= rows)."""
    return max(int(t.stride(1)), max(int(t.shape[0]), 1)) if t.shape[1] > 1 else max(int(t.shape[0]), 1)


# ----------------------------------------------------------------- movement

def _buffers(u: USTensor):
    for b in (*u.pos_buffers, *u.crd_buffers, u.val):
        if b is not None:
            yield b


def device_of(u: USTensor) -> torch.device:
    devs = {b.device for b in _buffers(u)}
    if len(devs) != 1:
        raise DeviceMismatch(f"buffers of {u} live on several devices: {sorted(map(str, devs))}")
    return devs.pop()


def materialize(u: USTensor, device, origin: Optional[AbstractIndexOrigin] = None) -> USTensor:
    """Move every buffer to `device` (CPUDevice() or HIPDevice(id)) and, if
    asked, change the index origin by shifting pos/crd by +-1
    (ext/CUDAExt/CUDAExt.jl:199-220)."""
    tdev = torch.device("cpu") if isinstance(device, CPUDevice) else device.torch
    new_origin = u.origin if origin is None else origin
    shift = new_origin.offset - u.origin.offset
    pos, crd = u.pos_buffers, u.crd_buffers
    if shift:
        # The index shift runs on the HIP device (jlust_hip_shift_index): on
        # the source's buffers when they live there, else after the move.
        from .convert import shift_index
        sh = lambda b: None if b is None else shift_index(b, shift)  # noqa: E731
        if u.val.device.type == "cuda":
            pos, crd = tuple(sh(b) for b in pos), tuple(sh(b) for b in crd)
            shift = 0
        elif tdev.type != "cuda":
            from .errors import UnsupportedFormat
            raise UnsupportedFormat(u.format.name, "HIPBackend",
                                    "an origin change runs on the HIP device; move the tensor there")
    mv = lambda b: None if b is None else b.to(tdev)  # noqa: E731
    pos = tuple(mv(b) for b in pos)
    crd = tuple(mv(b) for b in crd)
    val = u.val.to(tdev)
    if shift:
        from .convert import shift_index
        pos = tuple(None if b is None else shift_index(b, shift) for b in pos)
        crd = tuple(None if b is None else shift_index(b, shift) for b in crd)
    return USTensor(u.extents, u.format, pos, crd, val, None, new_origin)
