"""Synthetic input generator: determinism, thread-count independence, the
structural properties each configuration promises, and the algorithmic-byte
formula against BASELINE's figures."""
import ctypes

import numpy as np

from jlust_amd import workloads as W


def test_deterministic_and_thread_independent():
    a = W.make(1, scale=10)
    b = W.make(1, scale=10)
    for k in ("rowptr", "colind", "val", "x"):
        np.testing.assert_array_equal(a[k], b[k])
    # same columns with 1 and 8 threads
    rp = a["rowptr"]
    c1 = np.empty(rp[-1] - 1, np.int32)
    c8 = np.empty_like(c1)
    for out, nt in ((c1, 1), (c8, 8)):
        W.lib().wl_fill_columns(a["m"], a["n"], rp.ctypes.data_as(ctypes.c_void_p), 1, -1, 0,
                                out.ctypes.data_as(ctypes.c_void_p), nt)
    np.testing.assert_array_equal(c1, c8)
    v1 = np.empty(1000)
    v8 = np.empty(1000)
    W.lib().wl_normal_f64(3, 9, 1000, v1.ctypes.data_as(ctypes.c_void_p), 1)
    W.lib().wl_normal_f64(3, 9, 1000, v8.ctypes.data_as(ctypes.c_void_p), 8)
    np.testing.assert_array_equal(v1, v8)


def _rows_sorted_unique(rowptr, colind, n, origin=1):
    lens = np.diff(rowptr)
    assert colind.min() >= origin and colind.max() < n + origin
    d = np.diff(colind.astype(np.int64))
    starts = (rowptr[:-1] - origin)[lens > 0]
    inside = np.ones(d.size, bool)
    inside[starts[1:] - 1] = False          # boundaries between rows
    assert (d[inside] > 0).all()


def test_config1_shape():
    c = W.make(1)
    assert c["m"] == c["n"] == 100_000
    assert (np.diff(c["rowptr"]) == 16).all() and c["rowptr"][0] == 1
    _rows_sorted_unique(c["rowptr"], c["colind"], c["n"])
    assert -1 <= c["val"].min() < -0.99 and 0.99 < c["val"].max() <= 1
    assert W.algorithmic_bytes(c) == 21_200_004           # 12*nnz + 4(m+1) + 8(n+m), config 1


def test_config2_power_law_scaled():
    c = W.make(2, scale=16)
    lens = np.diff(c["rowptr"])
    assert lens.min() >= 1 and lens.max() <= 100_000
    assert abs(lens.mean() - 16) < 0.5
    assert lens.max() > 50 * lens.mean()                  # heavy tail
    _rows_sorted_unique(c["rowptr"], c["colind"], c["n"])


def test_config5_band():
    c = W.make(5, scale=64)
    bp, bc = c["browptr"], c["bcolind"] - 1
    assert (np.diff(bp) == 8).all()
    rows = np.repeat(np.arange(c["mb"]), 8)
    assert (np.abs(bc - rows) <= 32).all()
    _rows_sorted_unique(bp, c["bcolind"], c["nb"])
    assert c["val"].size == bc.size * 256


def test_baseline_byte_formulas():
    """Compulsory bytes of configs 3-5: each array counted once (the baseline's byte formulas)."""
    spmm = dict(kind="csr_spmm", rowptr=np.array([1, 32_000_001]), m=1_000_000, n=1_000_000,
                k=128)
    assert W.algorithmic_bytes(spmm) == 1_284_000_004
    sddmm = dict(kind="csr_sddmm", rowptr=np.array([1, 16_000_001]), m=500_000, n=500_000, K=128)
    assert W.algorithmic_bytes(sddmm) == 706_000_004
    bsr = dict(kind="bsr_spmm", browptr=np.array([1, 524_289]), mb=65_536, m=1_048_576,
               n=1_048_576, k=256)
    assert W.algorithmic_bytes(bsr) == 2_686_713_860
    assert W.flops(bsr) == 68_719_476_736
