"""numpy restatement of JLUST's block aggregates: BlockSparseMatrix products
(src/block_sparse.jl), BlockBandedMatrix products (src/block_banded.jl) and
the assembled CSR both are compiled into on the GPU backend
(ext/CUDAExt/ops/block_mul.jl).

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker; the product
package never imports it).

A block is a dict in the layout of oracle/convert_oracle.py ("CSR", "DCSR",
"COO" with pos/crd/val and an origin), or {"format": "ShiftedDiag", "m", "n",
"shift", "val"} for the structural shifted scaled identity (row r holds val
at column r + shift; src/named_formats.jl:53-61, level_step in
src/backends.jl:223-227).
"""
from __future__ import annotations

import numpy as np

from . import convert_oracle as CO


def entries(b):
    """(rows, cols, vals) of a block's stored entries in storage order, 0-based."""
    if b["format"] == "ShiftedDiag":
        r = np.arange(b["m"], dtype=np.int64)
        c = r + b["shift"]
        ok = (c >= 0) & (c < b["n"])
        return r[ok], c[ok], np.full(int(ok.sum()), b["val"], dtype=b.get("dtype", np.float64))
    return CO.decompose(b)


def dense(b):
    """The block as a dense m x n array (stored entries summed; blocks of the
    hot path hold no duplicates)."""
    r, c, v = entries(b)
    D = np.zeros((b["m"], b["n"]), np.asarray(v).dtype)
    np.add.at(D, (r, c), v)
    return D


def assemble(m, n, placements):
    """The assembled CSR (0-based rowptr, colind, val) of placed blocks:
    row R holds, for each placement covering R in the given order, that block
    row's stored entries in storage order with columns shifted
    (_compile_bsm, block_mul.jl:176-210; _compile_bbm, :518-548).
    placements: (block, row_off, col_off)."""
    R, C, V = [], [], []
    for b, r0, c0 in placements:
        r, c, v = entries(b)
        R.append(r + r0)
        C.append(c + c0)
        V.append(np.asarray(v))
    R = np.concatenate(R) if R else np.zeros(0, np.int64)
    C = np.concatenate(C) if C else np.zeros(0, np.int64)
    V = np.concatenate(V) if V else np.zeros(0)
    order = np.argsort(R, kind="stable")              # placement order, then storage order
    rowptr = np.zeros(m + 1, np.int64)
    np.add.at(rowptr, R + 1, 1)
    return np.cumsum(rowptr).astype(np.int32), C[order].astype(np.int32), V[order]


def csr_matvec(rowptr, colind, val, x):
    """y[r] = sum of the row's entries times x, accumulated in row order."""
    m = rowptr.size - 1
    y = np.zeros(m, np.result_type(val, x))
    for r in range(m):
        s, e = rowptr[r], rowptr[r + 1]
        y[r] = np.dot(val[s:e], x[colind[s:e]])
    return y


class BSM:
    """BlockSparseMatrix structure (block_sparse.jl:27-77): grid of blocks or None."""

    def __init__(self, grid):
        self.grid = grid
        nb_r, nb_c = len(grid), len(grid[0])
        self.row_sizes = [next(b["m"] for b in grid[i] if b is not None) for i in range(nb_r)]
        self.col_sizes = [next(grid[i][j]["n"] for i in range(nb_r) if grid[i][j] is not None)
                          for j in range(nb_c)]
        self.row_off = np.concatenate([[0], np.cumsum(self.row_sizes)]).astype(int)
        self.col_off = np.concatenate([[0], np.cumsum(self.col_sizes)]).astype(int)
        self.shape = (int(self.row_off[-1]), int(self.col_off[-1]))

    def placements(self, r0=0, c0=0):
        """Block rows outer, block columns inner (block_mul.jl:140-150)."""
        for i, row in enumerate(self.grid):
            for j, b in enumerate(row):
                if b is not None:
                    yield b, r0 + int(self.row_off[i]), c0 + int(self.col_off[j])

    def dense(self):
        D = None
        for b, r0, c0 in self.placements():
            d = dense(b)
            if D is None:
                D = np.zeros(self.shape, d.dtype)
            D[r0:r0 + d.shape[0], c0:c0 + d.shape[1]] += d
        return D

    def matvec(self, x):
        """execute(BlockSpMVOp) (block_sparse.jl:259-282): per block row, the
        first block's SpMV with beta = 0, the following ones accumulate."""
        y = None
        for i, row in enumerate(self.grid):
            acc = None
            for j, b in enumerate(row):
                if b is None:
                    continue
                xs = x[self.col_off[j]:self.col_off[j + 1]]
                t = dense(b) @ xs
                acc = t if acc is None else acc + t
            if y is None:
                y = np.zeros(self.shape[0], acc.dtype)
            y[self.row_off[i]:self.row_off[i + 1]] = acc
        return y

    def matmat(self, X):
        """execute(BlockSpMMOp) (block_sparse.jl:284-302): Y = 0, then every
        block accumulates into its row slice."""
        Y = np.zeros((self.shape[0], X.shape[1]), X.dtype)
        for b, r0, c0 in self.placements():
            d = dense(b)
            Y[r0:r0 + d.shape[0]] += d @ X[c0:c0 + d.shape[1]]
        return Y


def diag_starts(n_diag, n_off, T):
    """0-based rows where each period's diagonal block starts
    (_bbm_diag_starts, block_banded.jl:129-137)."""
    bw = len(n_off)
    cum = np.concatenate([[0], np.cumsum(n_off)]).astype(int)
    s = [0] * T
    for t in range(T - 1):
        s[t + 1] = s[t] + n_diag + int(cum[min(bw, T - 1 - t)])
    return s


class BBM:
    """BlockBandedMatrix (block_banded.jl:21-66).  diags: one matrix (BSM or
    block dict) or a list of T; off[k]: (neg, pos) or a list of T-k-1 pairs."""

    def __init__(self, diags, off, T, n_diag, n_off, n_cols):
        self.diags, self.off, self.T = diags, off, T
        self.n_diag, self.n_off, self.n_cols = n_diag, list(n_off), n_cols
        self.bw = len(off)
        self.shape = (T * n_diag + sum((T - k) * n_off[k - 1] for k in range(1, self.bw + 1)),
                      T * n_cols)

    def diag_at(self, t):
        return self.diags[t] if isinstance(self.diags, list) else self.diags

    def off_at(self, k, t):
        lv = self.off[k - 1]
        return lv if isinstance(lv, tuple) else lv[t]

    @staticmethod
    def _dense(obj):
        return obj.dense() if isinstance(obj, BSM) else dense(obj)

    @staticmethod
    def _place(obj, r0, c0):
        if isinstance(obj, BSM):
            yield from obj.placements(r0, c0)
        else:
            yield obj, r0, c0

    def placements(self):
        """Row order of _compile_bbm (block_mul.jl:518-548)."""
        starts = diag_starts(self.n_diag, self.n_off, self.T)
        cum = np.concatenate([[0], np.cumsum(self.n_off)]).astype(int)
        for t in range(self.T):
            yield from self._place(self.diag_at(t), starts[t], t * self.n_cols)
            for k in range(1, self.bw + 1):
                if t + k > self.T - 1:
                    continue
                neg, pos = self.off_at(k, t)
                ro = starts[t] + self.n_diag + int(cum[k - 1])
                yield from self._place(neg, ro, t * self.n_cols)
                yield from self._place(pos, ro, (t + k) * self.n_cols)

    def matvec(self, x):
        """execute(BBMSpMVOp) on the host (block_banded.jl:79-122, with the
        diagonal written at d_starts as the CPU path does, :161-168)."""
        starts = diag_starts(self.n_diag, self.n_off, self.T)
        cum = np.concatenate([[0], np.cumsum(self.n_off)]).astype(int)
        nc = self.n_cols
        y = np.zeros(self.shape[0], x.dtype)
        for t in range(self.T):
            y[starts[t]:starts[t] + self.n_diag] = self._dense(self.diag_at(t)) @ x[t * nc:(t + 1) * nc]
        for k in range(1, self.bw + 1):
            for t in range(self.T - k):
                ro = starts[t] + self.n_diag + int(cum[k - 1])
                neg, pos = self.off_at(k, t)
                y[ro:ro + self.n_off[k - 1]] = (self._dense(neg) @ x[t * nc:(t + 1) * nc]
                                               + self._dense(pos) @ x[(t + k) * nc:(t + k + 1) * nc])
        return y
