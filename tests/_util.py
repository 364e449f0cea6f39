"""Shared helpers of the parity tests (not collected by pytest)."""
from __future__ import annotations

import numpy as np

# Tolerances of the parity bar: |got - ref| <= tol * (|alpha||A||x| + |beta||y0|).
TOL = {np.dtype(np.float64): 1e-12, np.dtype(np.float32): 1e-5}


def dev(a, dtype=None):
    """numpy -> torch cuda tensor (1-D, or 2-D column-major kept column-major)."""
    import torch
    a = np.asarray(a) if dtype is None else np.asarray(a, dtype)
    if a.ndim == 2:
        return torch.from_numpy(np.ascontiguousarray(a.T)).cuda().t()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    """torch (cuda) tensor -> numpy, 2-D results in Fortran order."""
    a = t.detach().cpu()
    if a.dim() == 2:
        return np.asfortranarray(a.t().contiguous().numpy().T)
    return a.numpy()


def assert_within(got, ref, absref, dtype, what=""):
    tol = TOL[np.dtype(dtype)]
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = tol * np.asarray(absref, np.float64)
    bad = ~(err <= bound)
    if bad.any():
        idx = np.flatnonzero(bad.reshape(-1))[:5]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} entries outside tol {tol}: first at "
            f"{idx.tolist()} got {got.reshape(-1)[idx]} ref {ref.reshape(-1)[idx]} "
            f"bound {bound.reshape(-1)[idx]}")


def random_csr(m, n, density=None, lengths=None, seed=0, origin=1, dtype=np.float64,
               sorted_cols=True):
    """Random CSR (int32, given origin) with per-row distinct columns."""
    rng = np.random.default_rng(seed)
    if lengths is None:
        lengths = rng.binomial(n, density, size=m)
    lengths = np.minimum(np.asarray(lengths, np.int64), n)
    rowptr = np.zeros(m + 1, np.int64)
    np.cumsum(lengths, out=rowptr[1:])
    cols = np.empty(int(rowptr[-1]), np.int64)
    for i in range(m):
        c = rng.choice(n, size=int(lengths[i]), replace=False)
        if sorted_cols:
            c.sort()
        cols[rowptr[i]:rowptr[i + 1]] = c
    val = rng.uniform(-1, 1, size=cols.size).astype(dtype)
    return ((rowptr + origin).astype(np.int32), (cols + origin).astype(np.int32), val)


def sample_rows(rowptr, colind, val, rows, origin=1):
    """Sub-CSR made of the given rows (same columns and origin)."""
    lo = rowptr[rows] - origin
    hi = rowptr[rows + 1] - origin
    lens = (hi - lo).astype(np.int64)
    rp = np.zeros(rows.size + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    idx = np.concatenate([np.arange(a, b) for a, b in zip(lo, hi)]) if rows.size else \
        np.zeros(0, np.int64)
    return (rp + origin).astype(np.int32), colind[idx], val[idx], idx
