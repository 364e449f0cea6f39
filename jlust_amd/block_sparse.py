"""BlockSparseMatrix: a grid of USTensor blocks or None (src/block_sparse.jl).

The reference multiplies a block matrix either block by block (one SpMV per
block, the first block of a block row with beta = 0 and the rest with
beta = 1, block_sparse.jl:259-282) or, on its GPU backend, through one CSR
assembled once from the blocks plus one SpMV per call
(ext/CUDAExt/ops/block_mul.jl:128-306).  Here the assembled CSR is the
default: it is built on the device (jlust_hip_csr_assemble), kept with the
matrix, and every product is one launch of the CSR SpMV plan or of the CSR
SpMM kernel.  Blocks that cannot be assembled (COO, CSC, BSR) fall back to
the block-by-block products of the reference's generic path.

update_block_values_ rewrites one block's values and scatters them into the
assembled values through the slot map kept at assembly
(block_mul.jl:310-336), so the assembled matrix and the plan stay valid.

With JLUST_HIP_BLOCK_GRAPHS=1 (or USE_GRAPHS = True), SpMV through the
assembled CSR replays a HIP graph of the plan's launch
(jlust_hip_csr_spmv_plan_capture_*, captured natively, outside torch's graph
pools), one per (y, x, alpha, beta), the way the reference caches a CUDA
graph per (pointer(y), pointer(x)) with a last-key fast path
(block_mul.jl:233-267): the first call with a key runs the product directly
and captures it, later calls replay the capture.  Value updates rewrite the
buffers the capture reads, so captures stay valid across them.  A call made
while the current stream is itself being captured launches directly (the
outer capture records it).  Direct launch is the default because it is the
faster one here: on MI355X with ROCm 7 one hipGraphLaunch of a single
product costs more host time than the kernel launch it replaces (the
DCOPF case30000 product: 25 us queued per replay against 8 us launched
directly).  Callers with many products per step get the launch savings by
capturing the whole step in one graph.
"""
from __future__ import annotations

import ctypes
import os
import warnings
import weakref
from typing import List, Optional

import torch

from . import _lib
from .convert import Sparse, _descriptor, _device_of
from .errors import JLUSTError, UnsupportedFormat, UnsupportedValueType
from .formats import Formats, is_shifted_diag
from .tensor import USTensor, ZeroBased, csr_tensor, nnz, nonzeros, ust

_VT = {torch.float64: 0, torch.float32: 1}

# Replay assembled-CSR SpMV from captured HIP graphs (module switch; the
# environment sets its initial value; off by default, see above).
USE_GRAPHS = os.environ.get("JLUST_HIP_BLOCK_GRAPHS", "0") == "1"
# Captures kept per assembled matrix; the oldest is dropped past this.
GRAPH_CACHE = 16


class BlockStructureError(JLUSTError, ValueError):
    """A block grid that does not form a matrix (the reference's `error(...)`
    calls in block_sparse.jl:36-77)."""


class Placement(ctypes.Structure):
    """struct jlust_placement."""
    _fields_ = [("block", ctypes.POINTER(Sparse)),
                ("row_off", ctypes.c_int64), ("col_off", ctypes.c_int64),
                ("diag_m", ctypes.c_int64), ("diag_n", ctypes.c_int64),
                ("diag_shift", ctypes.c_int64), ("diag_val", ctypes.c_double),
                ("slots", ctypes.c_void_p)]


def assemblable(b: USTensor) -> bool:
    """Blocks the device assembly takes: CSR, DCSR and shifted diagonals
    (the reference compiles CSR and (Dense, ShiftedDiag) blocks,
    block_mul.jl:60-82; DCSR rows are placed by their stored row index)."""
    return b.format == Formats.CSR or b.format == Formats.DCSR or is_shifted_diag(b.format)


def _check_block_buffers(b: USTensor):
    """Buffer lengths the assembly kernels index by (they read pos[0..nseg]
    and crd/val[0..nnz) only)."""
    from .errors import NonCanonicalStorage
    m, _ = b.extents
    pos, crd = b.pos_buffers[1], b.crd_buffers[1]
    if pos is None or crd is None:
        raise NonCanonicalStorage(f"{b.format} block: missing level-2 pos/crd buffer")
    nseg = m if b.format == Formats.CSR else (b.crd_buffers[0].numel() if b.crd_buffers[0] is not None else -1)
    if nseg < 0 or pos.numel() != nseg + 1 or crd.numel() != nnz(b):
        raise NonCanonicalStorage(
            f"{b.format} block: pos has {pos.numel()} entries for {nseg} segments, crd "
            f"{crd.numel()} for {nnz(b)} values")
    for t in (pos, crd, b.crd_buffers[0], b.val):
        if t is not None and not t.is_contiguous():
            raise NonCanonicalStorage(f"{b.format} block: buffers must be contiguous")


class AssembledCSR:
    """One CSR (origin 0) built on the device from placed blocks, with the
    slot map of every placed CSR/DCSR block, an SpMV plan made on first use,
    and value refresh through the slot maps."""

    def __init__(self, m: int, n: int, pieces, dtype, device):
        """pieces: (key, block USTensor, row_off, col_off) in assembly order;
        blocks sharing a key receive the same new values on update."""
        if dtype not in _VT:
            raise UnsupportedValueType(dtype, "HIPBackend", "block matrices hold Float64 or Float32")
        self.m, self.n, self.dtype, self.device = m, n, dtype, device
        descs, places, self.slots = [], [], {}
        total = 0
        for key, b, r0, c0 in pieces:
            p = Placement(row_off=r0, col_off=c0)
            if is_shifted_diag(b.format):
                lv = b.format.levels[1]
                bm, bn = b.extents
                p.diag_m, p.diag_n, p.diag_shift, p.diag_val = bm, bn, lv.shift, lv.val
                total += max(0, min(bn - lv.shift, bm) - max(-lv.shift, 0))
            else:
                if b.val.device != device:
                    raise UnsupportedFormat(b.format, "HIPBackend", "blocks live on several devices")
                _device_of(b)
                _check_block_buffers(b)
                d = _descriptor(b)
                descs.append(d)
                p.block = ctypes.pointer(d)
                s = torch.empty(nnz(b), dtype=torch.int32, device=device)
                self.slots.setdefault(key, []).append(s)
                p.slots = s.data_ptr() if s.numel() else None
                total += nnz(b)
            places.append(p)
        i32 = dict(dtype=torch.int32, device=device)
        rowptr = torch.empty(m + 1, **i32)
        colind = torch.empty(total, **i32)
        val = torch.empty(total, dtype=dtype, device=device)
        arr = (Placement * max(len(places), 1))(*places)
        with torch.cuda.device(device):
            st = _lib.lib().jlust_hip_csr_assemble(
                m, n, len(places), arr, _VT[dtype], rowptr.data_ptr(),
                colind.data_ptr() if total else None, val.data_ptr() if total else None, total,
                ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
        _lib.check(st, "csr_assemble", Formats.CSR, "HIPBackend", dtype)
        self.asm = csr_tensor(rowptr, colind, val, (m, n), origin=ZeroBased())
        self._plan = None
        self._graphs = {}            # (y ptr, x ptr, alpha, beta) -> SpMVGraph
        self._last_key = None
        self._last_graph = None
        self.graph_error = None

    @property
    def nnz(self) -> int:
        return nnz(self.asm)

    def plan(self):
        if self._plan is None:
            from .hip_backend import HIPSpMVHandle
            self._plan = HIPSpMVHandle(self.asm)
        return self._plan

    def spmv(self, x: torch.Tensor, y: torch.Tensor, alpha=1.0, beta=0.0):
        h = self.plan()
        alpha, beta = float(alpha), float(beta)
        if USE_GRAPHS and self._graphs is not None and self._plain(x, y):
            key = (y.data_ptr(), x.data_ptr(), alpha, beta)
            g = self._last_graph if key == self._last_key else self._graphs.get(key)
            if g is None:
                h.execute_tensors(x, y, alpha, beta)      # this call's product
                self._capture(h, x, y, alpha, beta, key)  # replayed from the next call on
                return y
            self._last_key, self._last_graph = key, g
            if g.launch():
                return y
        return h.execute_tensors(x, y, alpha, beta)

    def _plain(self, x, y) -> bool:
        """x and y are what the plan's direct path takes without conversion."""
        di = self.device.index
        return (x.dtype is self.dtype and y.dtype is self.dtype and x.get_device() == di and
                y.get_device() == di and x.numel() == self.n and y.numel() == self.m and
                x.is_contiguous() and y.is_contiguous() and self.m > 0)

    def _capture(self, h, x, y, alpha, beta, key):
        """Record the product for later calls with this key
        (_bsm_mul_slowpath!, block_mul.jl:247-267); not while the current
        stream is itself being captured (that capture records the direct
        launch instead)."""
        if torch.cuda.is_current_stream_capturing():
            return
        try:
            g = h.capture(x, y, alpha, beta)
        except JLUSTError as e:
            # This matrix runs its products directly from now on; the reason
            # is kept in graph_error.
            self._graphs = None
            self.graph_error = str(e)
            warnings.warn(f"BlockSparse SpMV graph capture failed, launching directly: {e}")
            return
        if len(self._graphs) >= GRAPH_CACHE:
            self._graphs.pop(next(iter(self._graphs)))
        self._graphs[key] = g
        self._last_key, self._last_graph = key, g

    def spmm(self, X: torch.Tensor, Y: torch.Tensor, alpha=1.0, beta=0.0):
        from .hip_backend import _spmm
        _spmm(self.asm, ust(X), ust(Y), alpha, beta)
        return Y

    def update(self, key, new_val: torch.Tensor):
        """Scatter new values of the blocks placed under `key`."""
        src = new_val.contiguous()
        val = nonzeros(self.asm)
        with torch.cuda.device(self.device):
            for s in self.slots.get(key, ()):
                st = _lib.lib().jlust_hip_scatter_values(
                    val.data_ptr() if val.numel() else None, val.numel(),
                    s.data_ptr() if s.numel() else None, src.data_ptr() if src.numel() else None,
                    s.numel(), _VT[self.dtype],
                    ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))
                _lib.check(st, "scatter_values", Formats.CSR, "HIPBackend", self.dtype)
        if self._plan is not None:
            self._plan.update_values(self.asm)


def _grid(blocks) -> List[list]:
    if hasattr(blocks, "tolist") and not isinstance(blocks, torch.Tensor):
        blocks = blocks.tolist()
    grid = [list(r) for r in blocks]
    if not grid or any(len(r) != len(grid[0]) for r in grid) or not grid[0]:
        raise BlockStructureError("BlockSparseMatrix: blocks must form a non-empty rectangular grid")
    return grid


class BlockSparseMatrix:
    """src/block_sparse.jl:27-77: blocks[i][j] is a USTensor or None; blocks of
    one block row share their row count, blocks of one block column their
    column count, all blocks their value type."""

    def __init__(self, blocks):
        grid = _grid(blocks)
        nb_r, nb_c = len(grid), len(grid[0])
        row_sizes, col_sizes = [0] * nb_r, [0] * nb_c
        ref_T = None
        for i in range(nb_r):
            for j in range(nb_c):
                b = grid[i][j]
                if b is None:
                    continue
                if not isinstance(b, USTensor):
                    raise BlockStructureError(
                        f"BlockSparseMatrix: block ({i + 1},{j + 1}) must be a USTensor or None, "
                        f"got {type(b).__name__}")
                rs, cs = b.extents
                if row_sizes[i] == 0:
                    row_sizes[i] = rs
                elif row_sizes[i] != rs:
                    raise BlockStructureError(
                        f"BlockSparseMatrix: block row {i + 1} has inconsistent sizes "
                        f"({row_sizes[i]} vs {rs} at col {j + 1})")
                if col_sizes[j] == 0:
                    col_sizes[j] = cs
                elif col_sizes[j] != cs:
                    raise BlockStructureError(
                        f"BlockSparseMatrix: block col {j + 1} has inconsistent sizes "
                        f"({col_sizes[j]} vs {cs} at row {i + 1})")
                if ref_T is None:
                    ref_T = b.dtype
                elif ref_T != b.dtype:
                    raise BlockStructureError(
                        f"BlockSparseMatrix: mixed element types ({ref_T} vs {b.dtype} at block "
                        f"({i + 1},{j + 1}))")
        if any(s == 0 for s in row_sizes):
            raise BlockStructureError(
                "BlockSparseMatrix: block row(s) "
                f"{[i + 1 for i, s in enumerate(row_sizes) if s == 0]} are entirely None")
        if any(s == 0 for s in col_sizes):
            raise BlockStructureError(
                "BlockSparseMatrix: block col(s) "
                f"{[j + 1 for j, s in enumerate(col_sizes) if s == 0]} are entirely None")
        self.blocks = grid
        self.row_sizes, self.col_sizes = row_sizes, col_sizes
        self._row_off = [0]
        for s in row_sizes:
            self._row_off.append(self._row_off[-1] + s)
        self._col_off = [0]
        for s in col_sizes:
            self._col_off.append(self._col_off[-1] + s)
        self._T = ref_T
        self._asm: Optional[AssembledCSR] = None
        self._assemblable = all(assemblable(b) for _, b, _, _ in self.placed_blocks())
        self._listeners = weakref.WeakSet()      # block-banded matrices built on this one

    # ------------------------------------------------------------ interface

    @property
    def shape(self):
        return (self._row_off[-1], self._col_off[-1])

    def size(self, d: Optional[int] = None):
        """Base.size (block_sparse.jl:79-80); d is 1-based."""
        return self.shape if d is None else self.shape[d - 1]

    @property
    def dtype(self):
        """Base.eltype (block_sparse.jl:81)."""
        return self._T

    def eltype(self):
        return self._T

    def __repr__(self):
        return (f"BlockSparseMatrix({self.shape[0]}x{self.shape[1]}, "
                f"{len(self.blocks)}x{len(self.blocks[0])} blocks, {self._T})")

    def placed_blocks(self):
        """((i, j), block, row_off, col_off) of every stored block, block rows
        outer and block columns inner: the order of the reference's
        assembled rows (block_mul.jl:140-150, 196-210)."""
        for i, row in enumerate(self.blocks):
            for j, b in enumerate(row):
                if b is not None:
                    yield (i, j), b, self._row_off[i], self._col_off[j]

    def assemblable(self) -> bool:
        return self._assemblable

    def _device(self):
        devs = {b.val.device for _, b, _, _ in self.placed_blocks()}
        if len(devs) != 1 or next(iter(devs)).type != "cuda":
            raise UnsupportedFormat("BlockSparseMatrix", "HIPBackend",
                                    f"blocks must live on one HIP device, found {sorted(map(str, devs))}")
        return devs.pop()

    def assembled(self) -> AssembledCSR:
        """The assembled CSR, built on first use (_ensure_compiled_bsm,
        block_mul.jl:226-227)."""
        if self._asm is None:
            if not self.assemblable():
                raise UnsupportedFormat("BlockSparseMatrix", "HIPBackend",
                                        "assembly takes CSR, DCSR and ShiftedDiag blocks")
            m, n = self.shape
            self._asm = AssembledCSR(m, n, list(self.placed_blocks()), self._T, self._device())
        return self._asm

    # ------------------------------------------------------------ products

    def _check_vec(self, x, y):
        m, n = self.shape
        if x.dim() != 1 or y.dim() != 1 or x.numel() != n or y.numel() != m:
            from .errors import IncompatibleExtents
            raise IncompatibleExtents(
                f"BlockSpMV: A is {m}x{n}, x has {tuple(x.shape)}, y has {tuple(y.shape)}")

    def _check_mat(self, X, Y):
        m, n = self.shape
        if X.dim() != 2 or Y.dim() != 2 or X.shape[0] != n or Y.shape[0] != m or \
                X.shape[1] != Y.shape[1]:
            from .errors import IncompatibleExtents
            raise IncompatibleExtents(
                f"BlockSpMM: A is {m}x{n}, X is {tuple(X.shape)}, Y is {tuple(Y.shape)}")

    def spmv(self, x: torch.Tensor, y: torch.Tensor, alpha=1.0, beta=0.0) -> torch.Tensor:
        """execute(BlockSpMVOp, A, x, y) (block_sparse.jl:259-282): y = A*x
        (alpha*A*x + beta*y when given, mul!'s five-argument form)."""
        x, y = _t(x), _t(y)
        self._check_vec(x, y)
        if self.assemblable():
            return self.assembled().spmv(x, y, alpha, beta)
        from .ops import SpMVOp, execute
        for i, row in enumerate(self.blocks):
            y_sl = y[self._row_off[i]:self._row_off[i + 1]]
            first = True
            for j, b in enumerate(row):
                if b is None:
                    continue
                x_sl = x[self._col_off[j]:self._col_off[j + 1]]
                execute(SpMVOp, b, ust(x_sl), ust(y_sl), alpha=alpha, beta=beta if first else 1.0)
                first = False
        return y

    def spmm(self, X: torch.Tensor, Y: torch.Tensor, alpha=1.0, beta=0.0) -> torch.Tensor:
        """execute(BlockSpMMOp, A, X, Y) (block_sparse.jl:284-302): Y = A*X,
        X and Y column-major (alpha*A*X + beta*Y when given)."""
        X, Y = _t(X), _t(Y)
        self._check_mat(X, Y)
        if self.assemblable():
            return self.assembled().spmm(X, Y, alpha, beta)
        from .ops import SpMMOp, execute
        if beta == 0:
            Y.zero_()
        elif beta != 1:
            Y.mul_(beta)
        for i, row in enumerate(self.blocks):
            Y_sl = Y[self._row_off[i]:self._row_off[i + 1], :]
            for j, b in enumerate(row):
                if b is None:
                    continue
                X_sl = X[self._col_off[j]:self._col_off[j + 1], :]
                execute(SpMMOp, b, ust(X_sl), ust(Y_sl), alpha=alpha, beta=1.0)
        return Y

    def update_block_values(self, i: int, j: int, new_nzval) -> "BlockSparseMatrix":
        """update_block_values!(A, i, j, v) (block_sparse.jl:339-351 and the
        GPU form block_mul.jl:310-336); i and j are 1-based like the
        reference's.  The block's value buffer is overwritten in place, the
        assembled values are refreshed through the block's slot map, and the
        block-banded matrices built on this one are refreshed the same way."""
        if not (1 <= i <= len(self.blocks) and 1 <= j <= len(self.blocks[0])):
            raise BlockStructureError(f"update_block_values!: no block ({i},{j})")
        b = self.blocks[i - 1][j - 1]
        if not isinstance(b, USTensor):
            raise BlockStructureError(
                f"update_block_values!: block ({i},{j}) is not a USTensor (got {type(b).__name__})")
        v = _t(new_nzval)
        if v.numel() != nnz(b):
            raise BlockStructureError(
                f"update_block_values!: new_nzval length {v.numel()} != nnz {nnz(b)}")
        if v.dtype != b.dtype:
            raise UnsupportedValueType(v.dtype, "HIPBackend",
                                       f"block ({i},{j}) holds {b.dtype} values")
        nonzeros(b).copy_(v.reshape(-1))
        if self._asm is not None:
            self._asm.update((i - 1, j - 1), nonzeros(b))
        for bbm in list(self._listeners):
            bbm._block_values_changed(self, (i - 1, j - 1), nonzeros(b))
        return self


def _t(a) -> torch.Tensor:
    if isinstance(a, USTensor):
        return a.val
    return a if isinstance(a, torch.Tensor) else torch.as_tensor(a)


def update_block_values_(A: BlockSparseMatrix, i: int, j: int, new_nzval):
    """update_block_values!(A, i, j, new_nzval) (block_sparse.jl:339-351)."""
    return A.update_block_values(i, j, new_nzval)


def batch_mul_(Y, A: BlockSparseMatrix, X):
    """batch_mul!(Y, A, X) (block_sparse.jl:359-370): Y[:, k] = A*X[:, k] for
    every column, here as one SpMM over all columns of the column-major X."""
    X, Y = _t(X), _t(Y)
    nb = X.shape[1]
    if Y.shape[1] != nb:
        raise BlockStructureError(f"batch_mul!: Y has {Y.shape[1]} columns, X has {nb}")
    if Y.shape[0] != A.size(1):
        raise BlockStructureError(f"batch_mul!: Y rows {Y.shape[0]} != BM rows {A.size(1)}")
    if X.shape[0] != A.size(2):
        raise BlockStructureError(f"batch_mul!: X rows {X.shape[0]} != BM cols {A.size(2)}")
    if A.assemblable():
        return A.spmm(X, Y)
    for k in range(nb):
        A.spmv(X[:, k], Y[:, k])
    return Y


def batch_mul(A: BlockSparseMatrix, X):
    """batch_mul(A, X) (block_sparse.jl:372-375)."""
    from .tensor import dense_matrix
    X = _t(X)
    Y = dense_matrix(A.size(1), X.shape[1], dtype=X.dtype, device=X.device)
    return batch_mul_(Y, A, X)
