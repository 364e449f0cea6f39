"""numpy restatement of JLUST's convert_format for the 2-D hot-path formats.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker; the product
package never imports it).

A sparse matrix is a dict:
    {"format": "CSR"|"CSC"|"COO"|"DCSR"|"BSR", "origin": 0|1, "m", "n",
     "b1", "b2", "row_major" (BSR only),
     "pos1", "crd1", "pos2", "crd2" (int32 arrays or None), "val"}
with the level buffers of the reference's USTensor (src/tensor.jl:33-44):
    CSR  pos2 = rowptr, crd2 = colind          (src/named_formats.jl:25)
    CSC  pos2 = colptr, crd2 = rowind          (:26)
    COO  pos1 = [0, nnz] (optional on input), crd1 = rows, crd2 = cols  (:24)
    DCSR pos1 = [0, nrows], crd1 = rows, pos2 = row segments, crd2 = cols  (:27)
    BSR  pos2 = browptr, crd2 = bcolind, val block-major, row-major inside a
         block when row_major (BSRRight, :106-116) else column-major (BSRLeft).
All index values carry the origin.

convert_format follows src/convert.jl:302-388 step by step:
  decompose in storage order (TensorDecomposer, :5-122), drop explicit zeros
  (:316), map to the target's level coordinates and sort them with a stable
  lexicographic sort unless the target is the identity ordering and the source
  an ordered identity format (:331-349, `_lexsort_cols` :419-424), compose
  (TensorComposer, :124-299: on a unique level adjacent equal coordinates form
  one segment and only its first value is appended, :232-250; Dense in-block
  levels are zero-filled, :197-201), and shift pos/crd by the origin (:363-377).
"""
from __future__ import annotations

import numpy as np

IDENTITY = {"CSR", "COO", "DCSR"}          # level order (i, j) = dimension order
ORDERED_IDENTITY_SOURCES = {"CSR", "COO", "DCSR"}


def _i32(a):
    return np.asarray(a, np.int32)


def decompose(s):
    """(rows, cols, vals) of every stored entry in storage order, 0-based
    (TensorDecomposer, convert.jl:5-122)."""
    fmt, o = s["format"], s["origin"]
    val = np.asarray(s["val"])
    if fmt in ("CSR", "CSC"):
        ptr = _i32(s["pos2"]).astype(np.int64) - o
        seg = np.repeat(np.arange(ptr.size - 1, dtype=np.int64), np.diff(ptr))
        crd = _i32(s["crd2"]).astype(np.int64) - o
        return (seg, crd, val) if fmt == "CSR" else (crd, seg, val)
    if fmt == "COO":
        return (_i32(s["crd1"]).astype(np.int64) - o, _i32(s["crd2"]).astype(np.int64) - o, val)
    if fmt == "DCSR":
        ptr = _i32(s["pos2"]).astype(np.int64) - o
        k = np.repeat(np.arange(ptr.size - 1, dtype=np.int64), np.diff(ptr))
        rows = _i32(s["crd1"]).astype(np.int64)[k] - o
        return rows, _i32(s["crd2"]).astype(np.int64) - o, val
    if fmt == "BSR":
        b1, b2, rm = s["b1"], s["b2"], s["row_major"]
        bptr = _i32(s["pos2"]).astype(np.int64) - o
        brow = np.repeat(np.arange(bptr.size - 1, dtype=np.int64), np.diff(bptr))
        bcol = _i32(s["crd2"]).astype(np.int64) - o
        e = np.arange(b1 * b2, dtype=np.int64)
        ii, jj = (e // b2, e % b2) if rm else (e % b1, e // b1)
        rows = (brow[:, None] * b1 + ii[None, :]).reshape(-1)
        cols = (bcol[:, None] * b2 + jj[None, :]).reshape(-1)
        return rows, cols, val
    raise ValueError(fmt)


def level_coords(fmt, rows, cols, b1=1, b2=1, row_major=True):
    """dim2lvl of the target format: its level coordinates in level order."""
    if fmt in ("CSR", "COO", "DCSR"):
        return [rows, cols]
    if fmt == "CSC":
        return [cols, rows]
    if fmt == "BSR":
        inner = [rows % b1, cols % b2] if row_major else [cols % b2, rows % b1]
        return [rows // b1, cols // b2] + inner
    raise ValueError(fmt)


def _heads(keys):
    """Adjacent runs: True where any key differs from the entry before."""
    n = keys[0].size
    h = np.ones(n, bool)
    if n > 1:
        diff = np.zeros(n - 1, bool)
        for k in keys:
            diff |= k[1:] != k[:-1]
        h[1:] = diff
    return h


def convert_format(s, fmt, b1=None, b2=None, row_major=True):
    """src/convert.jl:302-388: the target tensor as a dict (same origin)."""
    o = s["origin"]
    rows, cols, vals = decompose(s)
    keep = vals != 0                                   # convert.jl:316 (-0.0 == 0 too)
    rows, cols, vals = rows[keep], cols[keep], vals[keep]
    b1 = b1 or 1
    b2 = b2 or 1
    lv = level_coords(fmt, rows, cols, b1, b2, row_major)
    if not (fmt in IDENTITY and s["format"] in ORDERED_IDENTITY_SOURCES):
        order = np.lexsort(lv[::-1])                   # stable, first level primary
        lv = [c[order] for c in lv]
        vals = vals[order]
    m, n = s["m"], s["n"]
    out = dict(format=fmt, origin=o, m=m, n=n, pos1=None, crd1=None, pos2=None, crd2=None)
    if fmt == "COO":                                   # non-unique first level: no merging
        out.update(pos1=_i32([o, vals.size + o]), crd1=_i32(lv[0] + o), crd2=_i32(lv[1] + o),
                   val=vals)
        return out
    h = _heads(lv)                                     # unique levels: keep the first
    lv = [c[h] for c in lv]
    vals = vals[h]
    if fmt in ("CSR", "CSC"):
        if lv[0].size > 1 and np.any(lv[0][1:] < lv[0][:-1]):
            # The Dense major level asserts non-decreasing coordinates (convert.jl:254).
            raise AssertionError("convert_format: rows not in non-decreasing order")
        nmaj = m if fmt == "CSR" else n
        ptr = np.searchsorted(lv[0], np.arange(nmaj + 1), side="left")
        out.update(pos2=_i32(ptr + o), crd2=_i32(lv[1] + o), val=vals)
        return out
    if fmt == "DCSR":
        rh = _heads([lv[0]])
        starts = np.flatnonzero(rh)
        out.update(pos1=_i32([o, starts.size + o]), crd1=_i32(lv[0][rh] + o),
                   pos2=_i32(np.r_[starts, lv[0].size] + o), crd2=_i32(lv[1] + o), val=vals)
        return out
    if fmt == "BSR":
        bh = _heads(lv[:2])
        bidx = np.cumsum(bh) - 1
        nb = int(bh.sum())
        inner = lv[2] * (b2 if row_major else b1) + lv[3]
        bval = np.zeros(nb * b1 * b2, vals.dtype)
        bval[bidx * b1 * b2 + inner] = vals
        brow = lv[0][bh]
        ptr = np.searchsorted(brow, np.arange(m // b1 + 1), side="left")
        out.update(pos2=_i32(ptr + o), crd2=_i32(lv[1][bh] + o), val=bval, b1=b1, b2=b2,
                   row_major=row_major)
        return out
    raise ValueError(fmt)


def to_dense(s):
    """sparse_to_dense (ext/KernelAbstractionsExt/ops/conversion.jl:47-65):
    every stored entry written into zeros (the last of duplicates wins here;
    the reference leaves duplicates undefined)."""
    rows, cols, vals = decompose(s)
    D = np.zeros((s["m"], s["n"]), np.asarray(s["val"]).dtype, order="F")
    D[rows, cols] = vals
    return D
