"""Operator tags, backends and the generic dispatcher (src/ops.jl,
src/backends.jl, src/convenience.jl).

`execute(SpMVOp, A, x, y; alpha, beta)` builds the operator instance from the
operand formats, resolves the backend with `default_backend` (from C for
SDDMM, src/convenience.jl:23-27) and calls the backend's `execute`.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from .errors import UnsupportedFormat
from .formats import TensorFormat
from .tensor import USTensor, device_of, nonzeros, ust


# ------------------------------------------------------------------- op tags

@dataclass(frozen=True)
class Op:
    """Op{Tag, Formats} (src/ops.jl:24-31): the tag plus operand formats."""
    tag: str
    formats: Tuple[TensorFormat, ...]

    def __repr__(self):
        return f"{self.tag}Op({', '.join(map(repr, self.formats))})"


@dataclass(frozen=True)
class OpType:
    """The UnionAll alias Op{:Tag}; calling it with formats makes an Op."""
    tag: str

    def __call__(self, *formats: TensorFormat) -> Op:
        return Op(self.tag, tuple(formats))

    def __repr__(self):
        return f"{self.tag}Op"


SpMVOp = OpType("SpMV")      # src/ops.jl:50
SpMMOp = OpType("SpMM")      # src/ops.jl:54
SDDMMOp = OpType("SDDMM")    # src/ops.jl:74
BlockSpMVOp = OpType("BlockSpMV")    # src/ops.jl (Op{:BlockSpMV})
BlockSpMMOp = OpType("BlockSpMM")    # src/ops.jl:111
BBMSpMVOp = OpType("BBMSpMV")        # src/ops.jl:115
_AGGREGATE_TAGS = ("BlockSpMV", "BlockSpMM", "BBMSpMV")


# ------------------------------------------------------------------ backends

class AbstractUSTBackend:
    def __repr__(self):
        return f"{type(self).__name__}()"

    def __eq__(self, other):
        return type(self) is type(other)

    def __hash__(self):
        return hash(type(self))


class AbstractKernelHandle:
    """A prepared operator (src/backends.jl:97)."""


class HIPBackend(AbstractUSTBackend):
    """Hand-written gfx950 kernels in libjlust_hip.so, reached through its C ABI.
    The counterpart of EmitterBackend / CUSPARSEBackend (src/backends.jl:176-181)."""


def supports_backend(backend, op: Op) -> bool:
    """src/backends.jl:111; the HIP capability table is in hip_backend."""
    if isinstance(backend, HIPBackend):
        from . import hip_backend
        return hip_backend.supports(op)
    return False


def default_backend(u: USTensor, optype: OpType):
    """src/backends.jl:195 and the GPU policy of ext/CUDAExt/CUDAExt.jl:232-241:
    tensors in GPU memory go to HIPBackend.  This package ships no CPU backend
    (JLUST's CPU path is EmitterBackend on KernelAbstractions), so host-memory
    tensors are an error rather than a silent fallback."""
    dev = device_of(u)
    if dev.type == "cuda":
        return HIPBackend()
    raise UnsupportedFormat(u.format, "HIPBackend",
                            f"{optype} operands live in host memory ({dev}); move them with "
                            "materialize(u, HIPDevice())")


# ---------------------------------------------------------------- dispatcher

def _wrap(a):
    return a if isinstance(a, (USTensor, AbstractKernelHandle)) else ust(a)


_ALPHA_BETA = frozenset(("alpha", "beta"))


def execute(optype, *args, backend=None, **kw):
    """execute(OpType, tensors...; backend, kw...)   (src/convenience.jl:15-39)
    execute(handle, tensors...; kw...)             (handle-driven call)."""
    if optype is SpMVOp and backend is None and len(args) == 3 and (not kw or kw.keys() <= _ALPHA_BETA):
        # The plain SpMV call on device vectors: HIPBackend's fast path (the
        # same checks, made once per matrix); anything it does not take goes on.
        A, x, y = args
        if type(A) is USTensor and type(x) is torch.Tensor and type(y) is torch.Tensor:
            from . import hip_backend
            r = hip_backend.spmv_fast(A, x, y, kw.get("alpha", 1.0), kw.get("beta", 0.0))
            if r is not None:
                return r
    if isinstance(optype, AbstractKernelHandle) or (args and isinstance(args[0], AbstractKernelHandle)):
        h, rest = (optype, args) if isinstance(optype, AbstractKernelHandle) else (args[0], args[1:])
        if getattr(h, "takes_raw", False):
            return h.execute(*rest, **kw)       # the handle wraps what it does not take raw
        return h.execute(*[_wrap(a) for a in rest], **kw)
    if isinstance(optype, AbstractUSTBackend):          # execute(backend, op, tensors...)
        be, op, tensors = optype, args[0], [_wrap(a) for a in args[1:]]
        return _backend_execute(be, op, tensors, kw)
    if isinstance(optype, OpType) and optype.tag in _AGGREGATE_TAGS:
        return _execute_aggregate(optype, *args, backend=backend, **kw)
    tensors = [_wrap(a) for a in args]
    if not isinstance(optype, OpType):
        raise TypeError(f"execute: expected an op type such as SpMVOp, got {optype!r}")
    primary = tensors[2] if optype.tag == "SDDMM" else tensors[0]
    be = backend if backend is not None else default_backend(primary, optype)
    op = optype(*[t.format for t in tensors])
    return _backend_execute(be, op, tensors, kw)


def _execute_aggregate(optype: OpType, A, x, y, backend=None, alpha=1.0, beta=0.0):
    """execute(BlockSpMVOp, A, x, y), execute(BlockSpMMOp, A, X, Y)
    (src/block_sparse.jl:259-302) and execute(BBMSpMVOp, M, x, y)
    (src/block_banded.jl:79-122): the aggregate runs its own products."""
    from .block_banded import BlockBandedMatrix
    from .block_sparse import BlockSparseMatrix
    if backend is not None and not isinstance(backend, HIPBackend):
        raise UnsupportedFormat(optype.tag, backend, "no such backend in jlust_amd")
    want = BlockBandedMatrix if optype.tag == "BBMSpMV" else BlockSparseMatrix
    if not isinstance(A, want):
        raise TypeError(f"execute({optype!r}, ...): expected a {want.__name__}, got {type(A).__name__}")
    if optype.tag == "BlockSpMM":
        return A.spmm(x, y, alpha, beta)
    return A.spmv(x, y, alpha, beta)


def _backend_execute(be, op: Op, tensors, kw):
    if isinstance(be, HIPBackend):
        from . import hip_backend
        return hip_backend.execute(op, *tensors, **kw)
    raise UnsupportedFormat(op.formats, be, "no such backend in jlust_amd")


def prepare(backend, optype: OpType, u_A, *more, **kw):
    """prepare(backend, OpType, A; kw...) -> handle (src/ops.jl:179);
    prepare(backend, SDDMMOp, A, B, C) as the cuSPARSE SDDMM handle takes it
    (ext/CUDAExt/ops/sddmm.jl:24-26)."""
    u_A = _wrap(u_A)
    if not isinstance(backend, HIPBackend):
        raise UnsupportedFormat(u_A.format, backend, "prepare is implemented for HIPBackend")
    from . import hip_backend
    return hip_backend.prepare(optype, u_A, *[_wrap(t) for t in more], **kw)


def update_values_(handle, u_A: USTensor):
    """update_values!(handle, A) (src/ops.jl:188): new values, same pattern."""
    return handle.update_values(u_A)


def mul_(Y, A: USTensor, X, alpha=None, beta=None):
    """LinearAlgebra.mul!(y, A, x[, alpha, beta]) and mul!(C, A, B[, alpha, beta])
    (src/convenience.jl:46-53): returns Y."""
    kw = {}
    if alpha is not None or beta is not None:
        kw = dict(alpha=1 if alpha is None else alpha, beta=0 if beta is None else beta)
    xt = X.val if isinstance(X, USTensor) else X
    if not isinstance(A, USTensor):          # BlockSparseMatrix / BlockBandedMatrix
        from .block_banded import BlockBandedMatrix
        if isinstance(A, BlockBandedMatrix):
            if xt.dim() != 1:
                raise TypeError("mul!(Y, ::BlockBandedMatrix, X) takes vectors only")
            optype = BBMSpMVOp
        else:
            optype = BlockSpMVOp if xt.dim() == 1 else BlockSpMMOp
        execute(optype, A, X, Y, **kw)
        return Y
    optype = SpMVOp if xt.dim() == 1 else SpMMOp
    execute(optype, A, ust(X), ust(Y), **kw)
    return Y


def matmul(A: USTensor, x):
    """Base.:*(A, x) (src/convenience.jl:55-59): a new y of A's value type."""
    import torch
    xt = x.val if isinstance(x, USTensor) else x
    if not isinstance(A, USTensor):          # BlockSparseMatrix / BlockBandedMatrix
        if xt.dim() == 1:
            y = torch.empty(A.size(1), dtype=A.dtype, device=xt.device)
        else:
            from .tensor import dense_matrix
            y = dense_matrix(A.size(1), xt.shape[1], dtype=A.dtype, device=xt.device)
        return mul_(y, A, x)
    if xt.dim() == 1:
        y = torch.empty(A.extents[0], dtype=nonzeros(A).dtype, device=nonzeros(A).device)
    else:
        from .tensor import dense_matrix
        y = dense_matrix(A.extents[0], xt.shape[1], dtype=nonzeros(A).dtype,
                         device=nonzeros(A).device)
    return mul_(y, A, x)
