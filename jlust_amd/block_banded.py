"""BlockBandedMatrix: a T-period block-banded matrix (src/block_banded.jl).

Rows interleave each period's diagonal block with the coupling rows to the
following periods (block_banded.jl:5-14):

    D[1]                            n_diag_rows rows (period 1)
    C[1][1].neg  C[1][1].pos        n_off_rows[1] rows (band 1, t=1 -> 2)
    C[2][1].neg        C[2][1].pos  n_off_rows[2] rows (band 2, t=1 -> 3)
         D[2]                       ...

Period t's diagonal block starts at row d_starts[t] (_bbm_diag_starts,
block_banded.jl:129-137): the band-k coupling rows of period t exist only
while t + k <= T, so the period stride shrinks over the last bw periods.
Column block t of x holds period t's n_cols variables.

With bandwidth 1, one BlockSparseMatrix diagonal shared by every period and
one (neg, pos) pair shared by every transition, each CSR or ShiftedDiag,
the product is one launch of the periodic kernel
(jlust_hip_bbm_periodic_spmv_*; the reference's periodic view,
ext/CUDAExt/ops/block_mul.jl:584-676, block_periodic.jl:108-236): it walks
the diagonal's own assembled CSR and the coupling blocks' buffers in place
for every period, so the T-fold matrix is never built and a product moves
little more than x and y.  It launches directly (the graph cache of the
assembled path, block_sparse.USE_GRAPHS, does not apply).
JLUST_HIP_BBM_PERIODIC=0 turns it off.

Otherwise the product runs as one SpMV over a CSR assembled once on the
device from every placed block (the reference's _compile_bbm,
ext/CUDAExt/ops/block_mul.jl:453-556, row for row the same arrays).  A
diagonal that is a BlockSparseMatrix is placed block by block; its
update_block_values_ is propagated into this matrix's assembled values
through the slot maps.  Blocks the assembly does not take fall back to the
per-period products of the reference's generic execute(BBMSpMVOp)
(block_banded.jl:79-122), with every period placed at d_starts.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Sequence

import torch

from . import _lib
from .block_sparse import (AssembledCSR, BlockSparseMatrix, BlockStructureError, Placement, _t,
                           _check_block_buffers, assemblable)
from .convert import _descriptor
from .errors import IncompatibleExtents, JLUSTError, UnsupportedFormat
from .formats import is_shifted_diag
from .tensor import USTensor

# Periodic kernel for the shared-block bandwidth-1 case (module switch; the
# environment sets its initial value).
USE_PERIODIC = os.environ.get("JLUST_HIP_BBM_PERIODIC", "1") != "0"


def _periodic_block(u: USTensor):
    """The placement the periodic kernel reads for a coupling or diagonal
    block: its CSR buffers in place, or its shifted diagonal."""
    p = Placement()
    if is_shifted_diag(u.format):
        lv = u.format.levels[1]
        p.diag_m, p.diag_n = u.extents
        p.diag_shift, p.diag_val = lv.shift, lv.val
        return p
    _check_block_buffers(u)
    d = _descriptor(u)
    if d.format != 0:
        raise UnsupportedFormat(u.format, "HIPBackend", "periodic blocks are CSR or ShiftedDiag")
    p.block = ctypes.pointer(d)
    return p


class _PeriodicView:
    """Arguments of jlust_hip_bbm_periodic_spmv_*: the diagonal matrix's own
    assembled CSR (refreshed in place by its update_block_values_) and the
    coupling pair as stored."""

    def __init__(self, M: "BlockBandedMatrix"):
        self.asm = M.diags.assembled()
        neg, pos = M.off_diags[0]
        self.blocks = (self.asm, neg, pos)              # keeps the buffers alive
        self.pl = (_periodic_block(self.asm.asm), _periodic_block(neg), _periodic_block(pos))
        self.refs = tuple(ctypes.byref(p) for p in self.pl)
        self.args = (M.T, M.n_diag_rows, M.n_off_rows[0], M.n_cols)
        self.m, self.n = M.shape
        self.T, self.dev = M._T, self.asm.device
        self.fn = getattr(_lib.lib(), "jlust_hip_bbm_periodic_spmv_" +
                          ("f64" if self.T == torch.float64 else "f32"))

    def plain(self, x, y) -> bool:
        di = self.dev.index
        return (x.dtype is self.T and y.dtype is self.T and x.get_device() == di and
                y.get_device() == di and x.numel() == self.n and y.numel() == self.m and
                x.is_contiguous() and y.is_contiguous())

    def spmv(self, x, y, alpha, beta):
        with _lib.on_device(self.dev):
            st = self.fn(*self.args, *self.refs, alpha, x.data_ptr(), beta, y.data_ptr(),
                         _lib.stream_handle(self.dev))
        if st:
            _lib.check(st, "bbm_periodic_spmv", "BlockBandedMatrix", "HIPBackend", self.T)
        return y


def diag_starts(n_diag_rows: int, n_off_rows: Sequence[int], T: int) -> List[int]:
    """0-based first row of each period's diagonal block (block_banded.jl:129-137)."""
    bw = len(n_off_rows)
    cum = [0]
    for s in n_off_rows:
        cum.append(cum[-1] + s)
    starts = [0] * T
    for t in range(T - 1):
        k_max = min(bw, T - 1 - t)
        starts[t + 1] = starts[t] + n_diag_rows + cum[k_max]
    return starts


def _pieces(obj, key, r0: int, c0: int):
    """(key, block, row, col) placements of a USTensor or BlockSparseMatrix."""
    if isinstance(obj, BlockSparseMatrix):
        for ij, b, br, bc in obj.placed_blocks():
            yield (id(obj), ij), b, r0 + br, c0 + bc
    else:
        yield key, obj, r0, c0


def _extents(obj):
    return obj.shape if isinstance(obj, BlockSparseMatrix) else tuple(obj.extents)


def _dtype(obj):
    return obj.dtype


def _all_blocks(obj):
    if isinstance(obj, BlockSparseMatrix):
        return [b for _, b, _, _ in obj.placed_blocks()]
    return [obj]


class BlockBandedMatrix:
    """BlockBandedMatrix(diags, off_diags, T, bw, n_diag_rows, n_off_rows,
    n_cols) (block_banded.jl:41-60) or the band-1 form
    BlockBandedMatrix(diag, neg_off, pos_off, T, n_diag_rows, n_off_rows,
    n_cols) (:63-66).  `diags` is one matrix shared by all periods or a list
    of T; off_diags[k] is a (neg, pos) pair shared by all band-(k+1)
    transitions or a list of T-(k+1) pairs.  Matrices are USTensors or
    BlockSparseMatrix objects."""

    def __init__(self, *args):
        if len(args) != 7:
            raise TypeError("BlockBandedMatrix takes 7 arguments")
        if isinstance(args[2], int):
            diags, off_diags, T, bw, n_diag_rows, n_off_rows, n_cols = args
        else:
            diag, neg, pos, T, n_diag_rows, n_off_rows, n_cols = args
            diags, off_diags, bw, n_off_rows = diag, [(neg, pos)], 1, [n_off_rows]
        T, bw, n_diag_rows, n_cols = int(T), int(bw), int(n_diag_rows), int(n_cols)
        n_off_rows = [int(s) for s in n_off_rows]
        off_diags = list(off_diags)
        if T < 1 or bw < 0 or len(off_diags) != bw or len(n_off_rows) != bw:
            raise BlockStructureError(
                f"BlockBandedMatrix: T={T}, bw={bw} with {len(off_diags)} coupling levels and "
                f"{len(n_off_rows)} coupling row counts")
        self.diags, self.off_diags = diags, off_diags
        self.T, self.bw = T, bw
        self.n_diag_rows, self.n_off_rows, self.n_cols = n_diag_rows, n_off_rows, n_cols
        self._check()
        self._asm: Optional[AssembledCSR] = None
        self._pv = None                                 # periodic view, False when not eligible
        self._assemblable = all(assemblable(b) for obj in self._matrices() for b in _all_blocks(obj))
        for obj in self._matrices():
            if isinstance(obj, BlockSparseMatrix):
                obj._listeners.add(self)

    # ------------------------------------------------------------ structure

    def diag_at(self, t: int):
        """Period t's diagonal block (0-based t)."""
        return self.diags[t] if isinstance(self.diags, (list, tuple)) else self.diags

    def off_at(self, k: int, t: int):
        """(neg, pos) coupling period t to t + k (1-based band k, 0-based t);
        _bbm_get_level, block_banded.jl:140-141."""
        lv = self.off_diags[k - 1]
        return lv if isinstance(lv, tuple) else lv[t]

    def _matrices(self):
        seen = []
        for t in range(self.T):
            seen.append(self.diag_at(t))
        for k in range(1, self.bw + 1):
            for t in range(self.T - k):
                seen.extend(self.off_at(k, t))
        out, ids = [], set()
        for obj in seen:
            if id(obj) not in ids:
                ids.add(id(obj))
                out.append(obj)
        return out

    def _check(self):
        if isinstance(self.diags, (list, tuple)) and len(self.diags) != self.T:
            raise BlockStructureError(
                f"BlockBandedMatrix: {len(self.diags)} diagonal blocks for T={self.T} periods")
        for k in range(1, self.bw + 1):
            lv = self.off_diags[k - 1]
            if not isinstance(lv, tuple) and len(lv) != self.T - k:
                raise BlockStructureError(
                    f"BlockBandedMatrix: band {k} has {len(lv)} coupling pairs, needs {self.T - k}")
            if isinstance(lv, tuple) and len(lv) != 2:
                raise BlockStructureError(f"BlockBandedMatrix: band {k} is not a (neg, pos) pair")
        types = set()
        for t in range(self.T):
            d = self.diag_at(t)
            if not isinstance(d, (USTensor, BlockSparseMatrix)):
                raise UnsupportedFormat(type(d).__name__, "HIPBackend",
                                        "diagonal blocks are USTensors or BlockSparseMatrix")
            if _extents(d) != (self.n_diag_rows, self.n_cols):
                raise IncompatibleExtents(
                    f"BlockBandedMatrix: period {t + 1} diagonal is {_extents(d)}, expected "
                    f"{(self.n_diag_rows, self.n_cols)}")
            types.add(_dtype(d))
        for k in range(1, self.bw + 1):
            for t in range(self.T - k):
                for side, mat in zip(("neg", "pos"), self.off_at(k, t)):
                    if not isinstance(mat, (USTensor, BlockSparseMatrix)):
                        raise UnsupportedFormat(type(mat).__name__, "HIPBackend",
                                                "coupling blocks are USTensors or BlockSparseMatrix")
                    if _extents(mat) != (self.n_off_rows[k - 1], self.n_cols):
                        raise IncompatibleExtents(
                            f"BlockBandedMatrix: band {k} {side} block is {_extents(mat)}, "
                            f"expected {(self.n_off_rows[k - 1], self.n_cols)}")
                    types.add(_dtype(mat))
        if len(types) != 1:
            raise BlockStructureError(f"BlockBandedMatrix: mixed element types {sorted(map(str, types))}")
        self._T = types.pop()

    # ------------------------------------------------------------ interface

    @property
    def shape(self):
        """Base.size (block_banded.jl:70-74)."""
        rows = self.T * self.n_diag_rows + sum((self.T - k) * self.n_off_rows[k - 1]
                                               for k in range(1, self.bw + 1))
        return (rows, self.T * self.n_cols)

    def size(self, d: Optional[int] = None):
        return self.shape if d is None else self.shape[d - 1]

    @property
    def dtype(self):
        return self._T

    def eltype(self):
        return self._T

    def __repr__(self):
        return (f"BlockBandedMatrix({self.shape[0]}x{self.shape[1]}, T={self.T}, bw={self.bw}, "
                f"{self._T})")

    def d_starts(self) -> List[int]:
        return diag_starts(self.n_diag_rows, self.n_off_rows, self.T)

    def placements(self):
        """(key, block, row, col) of every placed block in the row order of
        the reference's assembled BBM (block_mul.jl:518-548): per period the
        diagonal rows, then per band the coupling rows (neg entries before
        pos entries in each row)."""
        starts = self.d_starts()
        cum = [0]
        for s in self.n_off_rows:
            cum.append(cum[-1] + s)
        for t in range(self.T):
            r0 = starts[t]
            yield from _pieces(self.diag_at(t), ("diag", t), r0, t * self.n_cols)
            for k in range(1, self.bw + 1):
                if t + k > self.T - 1:
                    continue
                neg, pos = self.off_at(k, t)
                ro = r0 + self.n_diag_rows + cum[k - 1]
                yield from _pieces(neg, ("neg", k, t), ro, t * self.n_cols)
                yield from _pieces(pos, ("pos", k, t), ro, (t + k) * self.n_cols)

    def assemblable(self) -> bool:
        return self._assemblable

    def _device(self):
        devs = {b.val.device for obj in self._matrices() for b in _all_blocks(obj)}
        if len(devs) != 1 or next(iter(devs)).type != "cuda":
            raise UnsupportedFormat("BlockBandedMatrix", "HIPBackend",
                                    f"blocks must live on one HIP device, found {sorted(map(str, devs))}")
        return devs.pop()

    def assembled(self) -> AssembledCSR:
        """The assembled CSR, built on first use (_ensure_compiled_bbm,
        block_mul.jl:558-559)."""
        if self._asm is None:
            if not self.assemblable():
                raise UnsupportedFormat("BlockBandedMatrix", "HIPBackend",
                                        "assembly takes CSR, DCSR and ShiftedDiag blocks")
            m, n = self.shape
            self._asm = AssembledCSR(m, n, list(self.placements()), self._T, self._device())
        return self._asm

    def periodic(self) -> Optional[_PeriodicView]:
        """The periodic view when this matrix has one (bandwidth 1, one
        BlockSparseMatrix diagonal, one shared (neg, pos) pair of CSR or
        ShiftedDiag tensors; _bbm_supports_periodic, block_mul.jl:600-606)."""
        if self._pv is None:
            self._pv = False
            od = self.off_diags[0] if self.bw == 1 else None
            if (isinstance(self.diags, BlockSparseMatrix) and isinstance(od, tuple) and
                    all(isinstance(b, USTensor) for b in od) and self.diags.assemblable()):
                try:
                    self._device()
                    self._pv = _PeriodicView(self)
                except JLUSTError:
                    self._pv = False
        return self._pv or None

    def _block_values_changed(self, bsm, ij, vals):
        if self._asm is not None:
            self._asm.update((id(bsm), ij), vals)

    # ------------------------------------------------------------ products

    def spmv(self, x, y, alpha=1.0, beta=0.0):
        """execute(BBMSpMVOp, M, x, y) (block_banded.jl:79-122): y = M*x
        (alpha*M*x + beta*y when given)."""
        x, y = _t(x), _t(y)
        m, n = self.shape
        if x.dim() != 1 or y.dim() != 1 or x.numel() != n or y.numel() != m:
            raise IncompatibleExtents(
                f"BBMSpMV: M is {m}x{n}, x has {tuple(x.shape)}, y has {tuple(y.shape)}")
        if USE_PERIODIC:
            pv = self.periodic()
            if pv is not None and pv.plain(x, y):
                return pv.spmv(x, y, float(alpha), float(beta))
        if self.assemblable():
            return self.assembled().spmv(x, y, alpha, beta)
        from .ops import mul_
        starts = self.d_starts()
        cum = [0]
        for s in self.n_off_rows:
            cum.append(cum[-1] + s)
        nc = self.n_cols
        for t in range(self.T):
            mul_(y[starts[t]:starts[t] + self.n_diag_rows], self.diag_at(t), x[t * nc:(t + 1) * nc],
                 alpha, beta)
        for k in range(1, self.bw + 1):
            for t in range(self.T - k):
                ro = starts[t] + self.n_diag_rows + cum[k - 1]
                y_off = y[ro:ro + self.n_off_rows[k - 1]]
                neg, pos = self.off_at(k, t)
                mul_(y_off, neg, x[t * nc:(t + 1) * nc], alpha, beta)
                mul_(y_off, pos, x[(t + k) * nc:(t + k + 1) * nc], alpha, 1.0)
        return y
