#!/usr/bin/env python3
"""Benchmark of the JLUST sparse hot path on one MI355X.

    python bench.py [--config 2] [--steps K] [--warmup W] [--gpus 1]

A step is one call of the operator over the configuration's synthetic input,
already resident in HBM (one C ABI call).  SpMV runs, as JLUST's
prepare/execute handles do, through a plan prepared once outside the timed
region (for x wider than one XCD's L2 the column-sliced merge kernel, its
carry fix-up and the slice reduction); the plain per-call entry point (merge
kernel plus carry fix-up, nothing cached) is timed in the same run and
reported as `plain_call`.  SpMM's step includes the B re-layout.
Prints ONE JSON line: the metric of BASELINE.json (effective GB/s from the
reference's compulsory-byte formula, benchmark/bench_suitesparse.jl:170-172,
plus GFLOP/s), a `roofline` object for the step's dominant kernel and a
`cpu_baseline` measured on this host with the oracle (a C restatement of
JLUST's CPU path; Julia/JLUST itself is not available on the GPU box).

Default workload: config 2 (CSR SpMV fp64, power-law 4M x 4M, ~64M nnz).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "SpMV/SpMM/SDDMM effective GB/s (% of MI355X HBM peak) + GFLOP/s"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU work budget of the cpu_baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", action="store_true",
                   help="time only --config (default: the headline --config, then every other "
                        "BASELINE configuration, reported in all_configs)")
    p.add_argument("--other-cpu-seconds", type=float, default=6.0,
                   help="CPU work budget of the cpu_baseline sample of the non-headline configs")
    p.add_argument("--no-plan", action="store_true",
                   help="SpMV: time only the plain per-call entry point (default: a prepared plan, "
                        "as JLUST's prepare/execute handle API, with the plain call timed beside it)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a 1 GiB device copy (PMC byte-counter calibration)")
    p.add_argument("--gather-ceiling", action="store_true",
                   help="only measure random-gather bandwidth (8 B and 512 B rows) per source size")
    p.add_argument("--sweep-spmm", action="store_true",
                   help="only time CSR SpMM on config 3's matrix for k = 1 .. 256 (and the f32 SpMV)")
    p.add_argument("--sweep-sddmm", action="store_true",
                   help="only time SDDMM on config 4's mask for K = 1 .. 256")
    p.add_argument("--sweep-spmv", action="store_true",
                   help="only time SpMV on random matrices of 1 .. 16 entries per row: plain call, "
                        "plans forced unsliced / sliced, and the plan's own choice")
    p.add_argument("--mfma-peak", action="store_true",
                   help="only measure the sustained fp32 MFMA rate (v_mfma_f32_16x16x4_f32 chains)")
    p.add_argument("--stream-ceiling", action="store_true",
                   help="only measure the attainable HBM copy / read / fill rates (2 GiB f64)")
    p.add_argument("--convert", action="store_true",
                   help="only time format conversions (convert_format) at config sizes")
    p.add_argument("--coo", action="store_true",
                   help="only time COO and DCSR SpMV (plain calls and prepared plans) on config 2's "
                        "matrix, sorted and shuffled, beside the oracle's COO SpMV on this host")
    p.add_argument("--gather-floor", action="store_true",
                   help="only time the random-row gathers of configs 3 and 4 alone (their floor)")
    p.add_argument("--spmv-parts", action="store_true",
                   help="config 1's SpMV step taken apart: with its x gathers, with a coalesced x "
                        "read in their place, without x, y only (bench_probes.hip)")
    p.add_argument("--bsr-f64", action="store_true",
                   help="config 5's BSR pattern in Float64: the fp64 MFMA kernel against the CSR "
                        "expansion path")
    p.add_argument("--plan-build", action="store_true",
                   help="config 2's SpMV plan built six times: wall time per build, the first "
                        "included, after jlust_amd.preload()")
    p.add_argument("--bsr-long-rows", action="store_true",
                   help="config 5's band at a quarter of its block-rows with 8, 9, 12 and 16 blocks a "
                        "row: the fp32 strip kernels against the CSR expansion path")
    p.add_argument("--bsr-spmv", action="store_true",
                   help="16 x 16 BSR SpMV over power-law block-rows: the segmented kernel, the "
                        "one-thread-per-row kernel and the CSR expansion route")
    p.add_argument("--coo-spmm", action="store_true",
                   help="plain SpMM calls with a COO (shuffled) or CSC A: with the plan cache, on the "
                        "plain path (cache off), and a prepared plan")
    p.add_argument("--gather-overlap", action="store_true",
                   help="only time config 3's chunk gathers alone, a 256 MB transpose alone, and the "
                        "two on two streams at once")
    p.add_argument("--gather-cpol", action="store_true",
                   help="only time 8-byte random gathers as buffer loads under each cache policy")
    p.add_argument("--structured", action="store_true",
                   help="only time SpMV on structured matrices (2D/3D Laplacians, a random band)")
    p.add_argument("--mall-probe", action="store_true",
                   help="only measure whether a just-written buffer reads back faster than a cold one")
    p.add_argument("--cold", action="store_true",
                   help="time each step after a 1 GiB read that flushes the L2s and the MALL "
                        "(reported as cold_ms_per_step beside the warm figures)")
    p.add_argument("--blocks", action="store_true",
                   help="only time BlockSparseMatrix / BlockBandedMatrix mul! on a synthetic "
                        "DCOPF operator of pglib case30000_goc size (T = 24)")
    return p.parse_args()


def convert_bench(cpu_seconds):
    """Format conversions at BASELINE sizes: GPU convert_format (analyse +
    fill, as a caller sees it) and the numpy restatement of src/convert.jl on
    the host (the reference's convert_format runs on the CPU only).  Bytes =
    source buffers + target buffers, each counted once."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    from oracle import convert_oracle as CO
    res = []

    def nbytes(u):
        return sum(b.numel() * b.element_size() for b in (*u.pos_buffers, *u.crd_buffers, u.val)
                   if b is not None)

    def run(name, u, fmt, src_dict, target, extra=()):
        out = J.convert_format(u, fmt)
        torch.cuda.synchronize()
        reps = 5
        t0 = time.perf_counter()
        for _ in range(reps):
            out = J.convert_format(u, fmt)
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / reps
        b = nbytes(u) + nbytes(out)
        t1 = time.perf_counter()
        CO.convert_format(src_dict, target, *extra)
        tc = time.perf_counter() - t1
        res.append({"conversion": name, "nnz_in": int(u.val.numel()), "nnz_out": int(out.val.numel()),
                    "ms": round(t * 1e3, 3), "GBps": round(b / t / 1e9, 1),
                    "cpu_numpy_ms": round(tc * 1e3, 1), "speedup_vs_cpu": round(tc / t, 1)})
        log(f"{name}: {t*1e3:.2f} ms GPU, {tc*1e3:.0f} ms numpy")

    cfg = W.make(2)
    m, n = cfg["m"], cfg["n"]
    u = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
    s = dict(format="CSR", origin=1, m=m, n=n, pos2=cfg["rowptr"], crd2=cfg["colind"], val=cfg["val"])
    run("config2 CSR->CSC", u, J.Formats.CSC, s, "CSC")
    run("config2 CSR->COO", u, J.Formats.COO, s, "COO")
    q = J.convert_format(u, J.Formats.COO)
    sq = dict(format="COO", origin=1, m=m, n=n, crd1=host_np(q.crd_buffers[0]),
              crd2=host_np(q.crd_buffers[1]), val=host_np(q.val))
    run("config2 COO->CSR", q, J.Formats.CSR, sq, "CSR")
    del u, q, s, sq, cfg
    cfg = W.make(5)
    b = J.bsr_tensor(dev(cfg["browptr"]), dev(cfg["bcolind"]), dev(cfg["val"]), (cfg["m"], cfg["n"]))
    sb = dict(format="BSR", origin=1, m=cfg["m"], n=cfg["n"], b1=16, b2=16, row_major=True,
              pos2=cfg["browptr"], crd2=cfg["bcolind"], val=cfg["val"])
    run("config5 BSR->CSR", b, J.Formats.CSR, sb, "CSR")
    c = J.convert_format(b, J.Formats.CSR)
    sc = dict(format="CSR", origin=1, m=cfg["m"], n=cfg["n"], pos2=host_np(c.pos_buffers[1]),
              crd2=host_np(c.crd_buffers[1]), val=host_np(c.val))
    run("config5 CSR->BSR16", c, J.Formats.BSRRight((16, 16)), sc, "BSR", (16, 16, True))
    return res


def blocks_bench(steps, warmup):
    """mul! of the DCOPF BlockSparseMatrix [Cg 0 -Bbus; 0 -I Bf] and of the
    T = 24 BlockBandedMatrix with ramp coupling (-R, R), the two block
    operators of the reference's GPU tour (benchmark/tour_spmv.jl:178-370,
    sweep_cases.jl:103-166), on synthetic matrices of pglib case30000_goc
    size.  Per operator: time per call with a sync after each (the
    reference's @belapsed(mul!; sync)), time per call when calls are queued
    back to back -- each with direct launches (the default) and with mul!'s
    per-(y, x) graph cache; the BlockBandedMatrix with its periodic kernel
    (the default) and through the T-fold assembled CSR -- the one-off
    assembly, effective GB/s of the assembled
    CSR's compulsory bytes, and scipy's CSR matvec of the same matrix on
    this host."""
    import torch
    import scipy.sparse as sps
    import jlust_amd as J
    from jlust_amd import block_banded as BB
    from jlust_amd import block_sparse as BS
    from jlust_amd import workloads as W
    d = W.dcopf(**W.DCOPF_CASE30000)
    nb, nl, ng, nv, nc = d["n_bus"], d["n_line"], d["n_gen"], d["n_var"], d["n_con"]

    def ucsr(t, m, n, sign=1.0):
        rp, ci, v = t
        return J.csr_tensor(dev(rp), dev(ci), dev(sign * v), (m, n))
    one = np.arange(1, nl + 2, dtype=np.int32)
    negI = J.csr_tensor(dev(one), dev(one[:-1]), dev(-np.ones(nl)), (nl, nl))
    BM = J.BlockSparseMatrix([[ucsr(d["Cg"], nb, ng), None, ucsr(d["Bbus"], nb, nb, -1.0)],
                              [None, negI, ucsr(d["Bf"], nl, nb)]])
    g1 = np.arange(1, ng + 2, dtype=np.int32)
    R = J.csr_tensor(dev(g1), dev(g1[:-1]), dev(np.ones(ng)), (ng, nv))
    negR = J.csr_tensor(dev(g1), dev(g1[:-1]), dev(-np.ones(ng)), (ng, nv))
    T = 24
    MS = J.BlockBandedMatrix(BM, negR, R, T, nc, ng, nv)
    rng = np.random.default_rng(0)
    out = []
    for name, A in (("BlockSparseMatrix mul!", BM), ("BlockBandedMatrix mul! (T=24)", MS)):
        m, n = A.size()
        x = dev(rng.standard_normal(n))
        y = torch.empty(m, dtype=torch.float64, device="cuda")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        J.mul_(y, A, x)
        torch.cuda.synchronize()
        t_first = time.perf_counter() - t0
        def per_call(sync):
            for _ in range(warmup):
                J.mul_(y, A, x)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                J.mul_(y, A, x)
                if sync:
                    torch.cuda.synchronize()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / steps
        # mul! launching the product directly (the default), then with the
        # reference-style cache of one captured graph per (y, x) replayed.
        use = BS.USE_GRAPHS
        BS.USE_GRAPHS = False
        t_sync, t_async = per_call(True), per_call(False)
        BS.USE_GRAPHS = True
        t_sync_g, t_async_g = per_call(True), per_call(False)
        BS.USE_GRAPHS = use
        extra = {}
        if A is MS:
            # The block-banded product through the T-fold assembled CSR
            # instead of the periodic kernel.
            per = BB.USE_PERIODIC
            BB.USE_PERIODIC = False
            ts, ta = per_call(True), per_call(False)
            BB.USE_PERIODIC = per
            extra = {"periodic_kernel": per and A.periodic() is not None,
                     "us_per_call_sync_assembled": round(ts * 1e6, 1),
                     "us_per_call_queued_assembled": round(ta * 1e6, 1)}
            log(f"{name}: assembled CSR instead of the periodic kernel: {ts*1e6:.1f} us/call synced, "
                f"{ta*1e6:.1f} queued")
        # The same calls captured by the caller in one HIP graph (G calls per
        # graph) and replayed: the per-call launch cost without host dispatch.
        G = 20
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            J.mul_(y, A, x)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(G):
                J.mul_(y, A, x)
        graph.replay()
        torch.cuda.synchronize()
        reps = max(1, steps // G)
        t0 = time.perf_counter()
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        t_graph = (time.perf_counter() - t0) / (reps * G)
        del graph
        asm = A.assembled().asm
        nz = J.nnz(asm)
        byts = 12 * nz + 4 * (m + 1) + 8 * (m + n)
        S = sps.csr_matrix((host_np(asm.val), host_np(asm.crd_buffers[1]), host_np(asm.pos_buffers[1])),
                           shape=(m, n))
        xh = host_np(x)
        reps = max(3, min(200, int(0.5 / max(1e-6, (S.nnz + m) * 2e-9))))
        t0 = time.perf_counter()
        for _ in range(reps):
            yh = S @ xh
        t_cpu = (time.perf_counter() - t0) / reps
        err = float(np.max(np.abs(yh - host_np(y))) / max(1e-300, float(np.max(np.abs(yh)))))
        out.append({"op": name, "rows": m, "cols": n, "nnz": nz,
                    "first_call_ms": round(t_first * 1e3, 2),
                    "us_per_call_sync": round(t_sync * 1e6, 1),
                    "us_per_call_queued": round(t_async * 1e6, 1),
                    "us_per_call_sync_graph_cache": round(t_sync_g * 1e6, 1),
                    "us_per_call_queued_graph_cache": round(t_async_g * 1e6, 1),
                    "us_per_call_graph": round(t_graph * 1e6, 1),
                    "effective_GBps_sync": round(byts / t_sync / 1e9, 1),
                    "effective_GBps_queued": round(byts / t_async / 1e9, 1),
                    "cpu_scipy_us": round(t_cpu * 1e6, 1), "max_rel_diff_vs_scipy": err, **extra})
        log(f"{name}: {m}x{n} nnz {nz}: {t_sync*1e6:.1f} us/call synced, {t_async*1e6:.1f} queued "
            f"(graph per call {t_sync_g*1e6:.1f} / {t_async_g*1e6:.1f}), "
            f"{t_graph*1e6:.1f} in a caller's graph, "
            f"first call {t_first*1e3:.1f} ms, scipy {t_cpu*1e6:.0f} us")
    return out


def coo_bench(steps, warmup, cpu_seconds):
    """COO SpMV (src/interop.jl:248-260 storage; spmv.jl:407-448) on BASELINE
    config 2's matrix: the plain entry point (atomics per row run) and the
    prepared plan (entries row-ordered once, then the CSR plan), with the
    entries in row order and randomly shuffled; DCSR SpMV of the same matrix
    with every other row emptied; CSC SpMV of it with and without the plan
    cache.  Bytes: the COO compulsory bytes
    12*nnz + 4*nnz (rows) + 8(n + m).  CPU: the oracle's COO SpMV (C,
    sequential, oracle/jlust_cpu.c) on the box's host."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    from oracle import oracle as O
    cfg = W.make(2)
    m, n = cfg["m"], cfg["n"]
    rp = cfg["rowptr"].astype(np.int64)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rp))
    cols, val, xh = cfg["colind"], cfg["val"], cfg["x"]
    nz = val.size
    perm = np.random.default_rng(0).permutation(nz)
    byts = 16 * nz + 8 * (n + m)
    x = dev(xh)
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    out = []

    def run(name, step):
        ms, ev = timed(step, steps, warmup)
        out.append({"case": name, "ms_per_call": round(ms, 4), "GBps": round(byts / (ms * 1e-3) / 1e9, 1),
                    "event_ms": round(float(ev), 4)})
        log(f"{name}: {ms:.3f} ms/call")

    for order, (r, c, v) in (("row order", (rows, cols, val)),
                             ("shuffled", (rows[perm], cols[perm], val[perm]))):
        A = J.coo_tensor(dev(r), dev(c), dev(v), (m, n))
        run(f"COO {order}, plain call", lambda: J.execute(J.SpMVOp, A, x, y))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        torch.cuda.synchronize()
        t_build = time.perf_counter() - t0
        run(f"COO {order}, prepared plan", lambda: J.execute(h, x, y))
        out[-1]["plan_build_ms"] = round(t_build * 1e3, 2)
        del A, h
        torch.cuda.empty_cache()
    # DCSR: every other row emptied.
    keep = np.zeros(m, bool)
    keep[::2] = True
    lens = np.diff(rp)
    stored = np.flatnonzero(keep & (lens > 0))
    mask = np.repeat(keep, lens)
    dcols, dval = cols[mask], val[mask]
    dpos = (np.concatenate([[0], np.cumsum(lens[stored])]) + 1).astype(np.int32)
    D = J.dcsr_tensor(dev((stored + 1).astype(np.int32)), dev(dpos), dev(dcols), dev(dval), (m, n))
    run("DCSR (every other row stored), plain call", lambda: J.execute(J.SpMVOp, D, x, y))
    del D
    # CSC of the same matrix: plain calls (the plan cache plans it as COO from
    # the third call), and the plain path with the cache off.
    from jlust_amd.hip_backend import PLAN_CACHE
    o = np.lexsort((rows, cols))
    colptr = (np.r_[0, np.cumsum(np.bincount(cols - 1, minlength=n))] + 1).astype(np.int32)
    Acsc = J.csc_tensor(dev(colptr), dev(rows[o]), dev(val[o]), (m, n))
    del o
    run("CSC, plain call (cached plan)", lambda: J.execute(J.SpMVOp, Acsc, x, y))
    PLAN_CACHE.clear()
    cache_on, PLAN_CACHE.enabled = PLAN_CACHE.enabled, False
    try:
        run("CSC, plain call (plan cache off)", lambda: J.execute(J.SpMVOp, Acsc, x, y))
    finally:
        PLAN_CACHE.enabled = cache_on
    del Acsc
    torch.cuda.empty_cache()
    # CPU: the oracle's COO SpMV on a bounded sample (leading entries in row order).
    t0 = time.perf_counter()
    probe = max(1, nz // 50)
    O.coo_spmv(rows[:probe], cols[:probe], val[:probe], xh, m)
    tp = max(time.perf_counter() - t0, 1e-4)
    take = int(min(nz, probe * max(1.0, (cpu_seconds / 4) / tp)))
    t0 = time.perf_counter()
    O.coo_spmv(rows[:take], cols[:take], val[:take], xh, m)
    tc = time.perf_counter() - t0
    cpu_gbps = (16 * take + 8 * (n + m)) / tc / 1e9
    out.append({"case": "CPU oracle COO SpMV (1 thread)", "sample_entries": take,
                "GBps": round(cpu_gbps, 2)})
    log(f"cpu oracle COO: {cpu_gbps:.2f} GB/s on {take} entries")
    return out


def host_np(t):
    return t.detach().cpu().numpy()


def gather_ceiling():
    """Random-gather throughput on this GPU: out[i] = src[idx[i]] with uniform
    random idx, for the operand sizes the configs gather from (x: 8-byte
    elements; B rows: 512-byte rows).  Reported as useful gathered bytes/s and
    as gathers/s; torch.index_select is the gather kernel."""
    import torch
    res = []
    g = torch.Generator(device="cuda").manual_seed(0)
    for elem_bytes, sizes_mb in ((8, (4, 32, 256, 512)), (512, (32, 256, 512, 1024))):
        for mb in sizes_mb:
            if elem_bytes == 8:
                src = torch.randn(mb * 2**20 // 8, dtype=torch.float64, device="cuda")
                count = 64 * 2**20
            else:
                src = torch.randn(mb * 2**20 // 512, 128, dtype=torch.float32, device="cuda")
                count = 8 * 2**20
            idx = torch.randint(0, src.shape[0], (count,), generator=g, device="cuda")
            out = torch.index_select(src, 0, idx)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            s.record()
            for _ in range(reps):
                torch.index_select(src, 0, idx, out=out)
            e.record()
            torch.cuda.synchronize()
            t = s.elapsed_time(e) / reps * 1e-3
            res.append({"kernel": "torch.index_select", "elem_bytes": elem_bytes, "source_MB": mb,
                        "gathers": count, "ms": round(t * 1e3, 4),
                        "gathered_GBps": round(count * elem_bytes / t / 1e9, 1),
                        "Ggathers_per_s": round(count / t / 1e9, 2)})
            del src, idx, out
    res += gather_probe()
    return res


PROBE_SRC = os.path.join(ROOT, "bench_probes.hip")
PROBE_LIB = os.path.join(ROOT, "bench_probes.so")


def build_probes() -> str:
    """hipcc bench_probes.hip -> bench_probes.so (measurement kernels of this
    script; not part of libjlust_hip.so)."""
    import subprocess
    tmp = PROBE_LIB + ".tmp"
    subprocess.run(["/opt/rocm/bin/hipcc", "-O3", "-std=c++17", "-fPIC", "-shared", "--offload-arch=gfx950",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", PROBE_SRC, "-o", tmp],
                   check=True)
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def probe_lib():
    """bench_probes.so, built first when it is missing or older than its source."""
    import ctypes
    if not os.path.exists(PROBE_LIB) or os.path.getmtime(PROBE_LIB) < os.path.getmtime(PROBE_SRC):
        build_probes()
    return ctypes.CDLL(PROBE_LIB)


def gather_floor():
    """The gathers of configs 3 and 4 alone (bench_probes.hip,
    rows_probe_kernel): config 3's SpMM gathers, per 64-column chunk, one
    256-byte row of the 256 MB row-major copy of B for each of its 32M
    nonzeros; config 4's SDDMM gathers one 512-byte column of B (256 MB) for
    each of its 16M nonzeros.  Uniform random rows, a wave per 32 or 64
    (or 128) consecutive indices, 8 load instructions in flight per wave:
    with 4/8-byte lanes one row per instruction, with 16-byte lanes
    (rows_wide_probe_kernel) 4 or 2 rows per instruction.  The time bounds
    any kernel making those gathers."""
    import ctypes
    import torch
    lib = probe_lib()
    for f in (lib.jlust_probe_rows_f32, lib.jlust_probe_rows_wide_f32):
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                      ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    stream = torch.cuda.current_stream()
    g = torch.Generator(device="cuda").manual_seed(3)
    res = []
    for name, nrows, row, count in (("config 3 SpMM chunk: 256 B rows of a 256 MB B copy", 1_000_000, 64,
                                     32_000_000),
                                    ("config 4 SDDMM: 512 B columns of a 256 MB B", 500_000, 128,
                                     16_000_000)):
        src = torch.randn(nrows * row, dtype=torch.float32, device="cuda")
        idx = torch.randint(0, nrows, (count,), generator=g, device="cuda", dtype=torch.int64).to(torch.int32)
        for lanes, per_wave in (("4/8-byte", 32), ("4/8-byte", 64), ("16-byte", 64), ("16-byte", 128)):
            waves = (count + per_wave - 1) // per_wave
            out = torch.empty(waves * 64, dtype=torch.float32, device="cuda")
            fn = lib.jlust_probe_rows_f32 if lanes == "4/8-byte" else lib.jlust_probe_rows_wide_f32
            call = lambda: fn(src.data_ptr(), nrows, row, idx.data_ptr(), count,  # noqa: E731
                              per_wave, out.data_ptr(), stream.cuda_stream)
            for _ in range(3):
                assert call() == 0
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            s.record(stream)
            for _ in range(reps):
                call()
            e.record(stream)
            torch.cuda.synchronize()
            t = s.elapsed_time(e) / reps * 1e-3
            res.append({"case": name, "lanes": lanes, "rows_per_wave": per_wave, "gathers": count,
                        "row_bytes": row * 4, "ms": round(t * 1e3, 4),
                        "gathered_TBps": round(count * row * 4 / t / 1e12, 3)})
            log(f"{name}, {lanes} lanes, {per_wave} per wave: {t * 1e3:.3f} ms")
            del out
        del src, idx
        torch.cuda.empty_cache()
    return res


def spmv_parts():
    """Config 1's SpMV step taken apart (bench_probes.hip, spmv_parts_kernel:
    the library's vector-kernel shape at config 1, 4 lanes per row): with the
    random x gathers, with a coalesced read of x[row] in their place, with no
    x, and writing y only.  HIP events over 400 back-to-back launches, best
    of 3 rounds, in us per launch (the 400 launches are made in a C loop,
    since a launch from Python takes longer on the host than these kernels
    on the GPU)."""
    import ctypes
    import torch
    from jlust_amd import workloads as W
    lib = probe_lib()
    f = lib.jlust_probe_spmv_parts_f64
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p]
    cfg = W.make(1)
    m, n = cfg["m"], cfg["n"]
    nnz = int(cfg["rowptr"][-1]) - 1
    if nnz != 16 * m:
        raise RuntimeError("config 1 rows are expected to hold 16 entries each")
    colind, val, x = dev(cfg["colind"]), dev(cfg["val"]), dev(cfg["x"])
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    stream = torch.cuda.current_stream()
    names = {0: "x[col] gathers (the kernel's step)", 1: "x[row], coalesced, in place of the gathers",
             2: "no x (value x column index)", 3: "y written only"}
    best = {}
    for _ in range(3):
        for mode in names:
            call = lambda reps: f(m, n, 16, 1, colind.data_ptr(), val.data_ptr(),  # noqa: E731
                                  x.data_ptr(), y.data_ptr(), mode, reps, stream.cuda_stream)
            assert call(20) == 0
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            assert call(400) == 0
            e.record(stream)
            torch.cuda.synchronize()
            us = s.elapsed_time(e) / 400 * 1e3
            best[mode] = min(best.get(mode, us), us)
    res = [{"mode": names[k], "us_per_launch": round(v, 3)} for k, v in best.items()]
    for r in res:
        log(f"spmv parts: {r['mode']}: {r['us_per_launch']} us")
    gathers = best[0] - best[1]
    res.append({"gathers_us": round(gathers, 3), "gathers": nnz,
                "gathers_per_s": round(nnz / (gathers * 1e-6) / 1e9, 1)})
    return res


def bsr_f64():
    """Config 5's banded BSR pattern (65,536 block-rows of 16 x 16 blocks,
    8 per block-row within +-32, k = 256) in Float64: the fp64 MFMA strip
    kernel (jlust_hip_bsr_spmm_f64_i32, LDS windows of B) against the
    per-row fp64 kernel it replaced (JLUST_HIP_BSR_STRIP=0) and the same
    product through the device CSR expansion and the CSR SpMM.  HIP events:
    the median of 5 runs of 10 calls after 3 warm-up calls (the expansion:
    one run of 3 calls)."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    from jlust_amd.hip_backend import _bsr_as_csr
    cfg = W.make(5)
    mb, nb, k = cfg["mb"], cfg["nb"], cfg["B"].shape[1]
    A = J.bsr_tensor(dev(cfg["browptr"]), dev(cfg["bcolind"]), dev(cfg["val"].astype(np.float64)),
                     (mb * 16, nb * 16), (16, 16))
    B = dev(np.asfortranarray(cfg["B"].astype(np.float64)))
    del cfg
    C = J.dense_matrix(mb * 16, k, dtype=torch.float64)
    flops = 2.0 * 16 * 16 * k * int(A.crd_buffers[1].numel())
    stream = torch.cuda.current_stream()

    def ms(fn, reps=10, trials=5):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(trials):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for _ in range(reps):
                fn()
            e.record(stream)
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e) / reps)
        return sorted(ts)[len(ts) // 2]

    t_mfma = ms(lambda: J.execute(J.SpMMOp, A, B, C))
    old = os.environ.get("JLUST_HIP_BSR_STRIP")
    os.environ["JLUST_HIP_BSR_STRIP"] = "0"           # the per-row kernel the strip kernel replaced
    try:
        t_row = ms(lambda: J.execute(J.SpMMOp, A, B, C))
    finally:
        if old is None:
            del os.environ["JLUST_HIP_BSR_STRIP"]
        else:
            os.environ["JLUST_HIP_BSR_STRIP"] = old
    Acsr = _bsr_as_csr(A)
    t_csr = ms(lambda: J.execute(J.SpMMOp, Acsr, B, C), reps=3, trials=1)
    tf = lambda t: round(flops / (t * 1e-3) / 1e12, 2)  # noqa: E731
    res = {"workload": "bsr16_spmm_f64_banded_65536x8_k256", "flops": flops,
           "kernel": "bsr16_spmm_f64_strip_kernel",
           "mfma_ms": round(t_mfma, 4), "mfma_tflops": tf(t_mfma),
           "mfma_pct_of_fp64_peak": round(100 * flops / (t_mfma * 1e-3) / 78.6e12, 1),
           "row_kernel_ms": round(t_row, 4), "row_kernel_tflops": tf(t_row),
           "csr_expansion_ms": round(t_csr, 3), "csr_expansion_tflops": tf(t_csr)}
    log(f"bsr f64: {res}")
    return res


def plan_build():
    """Config 2's prepared SpMV plan (`prepare(HIPBackend(), SpMVOp, A)`, the
    LDS-binned layout) built six times in one process after
    jlust_amd.preload(): wall time of each build from the call to the
    device's completion, the plan's kind and its device bytes.  Under
    `rocprofv3 --kernel-trace` the same command gives the build's kernels."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    t0 = time.perf_counter()
    J.preload()
    torch.cuda.synchronize()
    preload_ms = (time.perf_counter() - t0) * 1e3
    cfg = W.make(2)
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (cfg["m"], cfg["n"]))
    del cfg
    builds, kind, nbytes = [], None, None
    for _ in range(6):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        torch.cuda.synchronize()
        builds.append(round((time.perf_counter() - t0) * 1e3, 2))
        kind, nbytes = h.kernel(), h.device_bytes()
        del h
        torch.cuda.synchronize()
    r = {"workload": "csr_spmv_f64_powerlaw_4M_mean16 plan", "kind": kind, "device_bytes": nbytes,
         "preload_ms": round(preload_ms, 2), "build_ms": builds, "first_ms": builds[0],
         "steady_ms": sorted(builds[1:])[len(builds[1:]) // 2]}
    log(f"plan build: {r}")
    return r


def bsr_long_rows():
    """16 x 16 fp32 BSR SpMM (k = 256) on config 5's +-32 band at a quarter of
    its block-rows (16,384) with 8, 9, 12 and 16 blocks a row: up to 8 the
    windowed strip kernels hold a row's A operands in registers; a strip with a
    longer row takes the direct operand loads.  Beside it the same product
    through the device CSR expansion and the CSR SpMM.  HIP events: the median
    of 5 runs of 5 calls after 2 warm-up calls (the expansion path: one run of
    3 calls)."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    from jlust_amd.hip_backend import _bsr_as_csr
    stream = torch.cuda.current_stream()

    def ms(fn, reps=5, trials=5):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(trials):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for _ in range(reps):
                fn()
            e.record(stream)
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e) / reps)
        return sorted(ts)[len(ts) // 2]

    out = []
    mb = nb = 16384
    k = 256
    for per_row in (8, 9, 12, 16):
        browptr = W.rowptr_from_lengths(np.full(mb, per_row, dtype=np.int64), origin=1)
        bcolind = W.columns(browptr, mb, 7, band=32)
        val = np.random.default_rng(1).standard_normal(bcolind.size * 256).astype(np.float32)
        A = J.bsr_tensor(dev(browptr), dev(bcolind), dev(val), (mb * 16, nb * 16))
        B = dev(np.asfortranarray(np.random.default_rng(2).standard_normal((nb * 16, k)).astype(np.float32)))
        C = J.dense_matrix(mb * 16, k, dtype=torch.float32)
        flops = 2.0 * 256 * k * bcolind.size
        t = ms(lambda: J.execute(J.SpMMOp, A, B, C))
        Ac = _bsr_as_csr(A)
        Cc = J.dense_matrix(mb * 16, k, dtype=torch.float32)
        tc = ms(lambda: J.execute(J.SpMMOp, Ac, B, Cc), reps=3, trials=1)
        r = {"blocks_per_row": per_row, "bsr_ms": round(t, 4), "bsr_TFLOPs": round(flops / t / 1e9, 2),
             "csr_expansion_spmm_ms": round(tc, 3)}
        log(f"bsr long rows: {r}")
        out.append(r)
        del A, B, C, Ac, Cc
        torch.cuda.empty_cache()
    return out


def bsr_spmv_powerlaw():
    """16 x 16 BSR SpMV (jlust_hip_bsr_spmv_*) over power-law block-rows:
    65,536 block-rows whose lengths follow a Pareto law (mean about 8 blocks,
    capped at 8,192), random block columns, values N(0, 1).  The segmented
    kernel (default; plain calls, and a prepared plan that keeps the segment
    table), the one-thread-per-row kernel
    (JLUST_HIP_BSR_SPMV_SEGMENTS=0), and the CSR expansion route (expansion,
    then CSR SpMV on the expanded matrix).  HIP events: the median of 5 runs
    of 20 calls after 3 warm-up calls; bytes = values + block columns +
    browptr + x + y.  Plain calls are timed both as they run by default (a
    cached plan from the third call on a matrix) and on the plain kernels."""
    import torch
    import jlust_amd as J
    from jlust_amd.hip_backend import _bsr_as_csr, PLAN_CACHE
    stream = torch.cuda.current_stream()

    def ms(fn, reps=20, trials=5):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(trials):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record(stream)
            for _ in range(reps):
                fn()
            e.record(stream)
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e) / reps)
        return sorted(ts)[len(ts) // 2]

    out = []
    mb = nb = 65536
    rng = np.random.default_rng(1)
    lens = np.maximum(np.minimum((rng.pareto(1.5, mb) + 1) * 8 / 3, 8192).astype(np.int64), 1)
    bcolind = np.concatenate([np.sort(rng.choice(nb, int(n), replace=False)) for n in lens]).astype(np.int32)
    browptr = np.r_[0, np.cumsum(lens)].astype(np.int32)
    nnzb = int(bcolind.size)
    for dt in (np.float32, np.float64):
        val = np.random.default_rng(2).standard_normal(nnzb * 256).astype(dt)
        A = J.bsr_tensor(dev(browptr), dev(bcolind), dev(val), (mb * 16, nb * 16), (16, 16),
                         origin=J.ZeroBased())
        del val
        x = dev(np.random.default_rng(3).standard_normal(nb * 16).astype(dt))
        y = torch.zeros(mb * 16, dtype=x.dtype, device="cuda")
        # Plain calls switch to a cached plan at the third call on a matrix;
        # the plain kernels are timed with the cache off.
        t_cached = ms(lambda: J.execute(J.SpMVOp, A, x, y))
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        t_plan = ms(lambda: J.execute(h, x, y))
        del h
        PLAN_CACHE.clear()
        cache_on, PLAN_CACHE.enabled = PLAN_CACHE.enabled, False
        old = os.environ.get("JLUST_HIP_BSR_SPMV_SEGMENTS")
        try:
            t_seg = ms(lambda: J.execute(J.SpMVOp, A, x, y))
            os.environ["JLUST_HIP_BSR_SPMV_SEGMENTS"] = "0"
            t_row = ms(lambda: J.execute(J.SpMVOp, A, x, y), reps=3, trials=1)
        finally:
            PLAN_CACHE.enabled = cache_on
            if old is None:
                os.environ.pop("JLUST_HIP_BSR_SPMV_SEGMENTS", None)
            else:
                os.environ["JLUST_HIP_BSR_SPMV_SEGMENTS"] = old
        t_exp = ms(lambda: _bsr_as_csr(A), reps=3, trials=1)
        Acsr = _bsr_as_csr(A)
        t_csr = ms(lambda: J.execute(J.SpMVOp, Acsr, x, y))
        isz = np.dtype(dt).itemsize
        nbytes = nnzb * 256 * isz + nnzb * 4 + (mb + 1) * 4 + (nb + mb) * 16 * isz
        gbs = lambda t: round(nbytes / (t * 1e-3) / 1e9, 1)  # noqa: E731
        r = {"workload": f"bsr16_spmv_powerlaw_65536_{np.dtype(dt).name}", "nnzb": nnzb,
             "max_blocks_per_row": int(lens.max()), "bytes": nbytes,
             "segments_ms": round(t_seg, 4), "segments_GBps": gbs(t_seg),
             "plain_cached_ms": round(t_cached, 4), "plain_cached_GBps": gbs(t_cached),
             "plan_ms": round(t_plan, 4), "plan_GBps": gbs(t_plan),
             "row_kernel_ms": round(t_row, 3), "row_kernel_GBps": gbs(t_row),
             "expansion_ms": round(t_exp, 3), "csr_spmv_on_expansion_ms": round(t_csr, 4)}
        log(f"bsr spmv: {r}")
        out.append(r)
        del A, Acsr, x, y
        torch.cuda.empty_cache()
    return out


def coo_csc_spmm():
    """Repeated plain SpMM calls execute(SpMMOp, A, B, C) with a COO A whose
    entries are shuffled, and with the same matrix as CSC: 1M x 1M, 8 random
    columns a row, f32, k = 32 columns of B.  Timed as they run by default
    (the plan cache's COO/CSC SpMM plan from the third call on a matrix), on
    the plain path (the cache off: the entries put in row order at every
    call), and through a prepared plan.  HIP events over 10 calls after 3
    warm-up calls."""
    import torch
    import jlust_amd as J
    from jlust_amd.hip_backend import PLAN_CACHE
    m = n = 1_000_000
    per, k = 8, 32
    rng = np.random.default_rng(1)
    rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), per)
    cols = rng.integers(1, n + 1, rows.size).astype(np.int32)
    val = rng.standard_normal(rows.size).astype(np.float32)
    p = rng.permutation(rows.size)
    A = J.coo_tensor(dev(rows[p]), dev(cols[p]), dev(val[p]), (m, n))
    o = np.lexsort((rows, cols))
    colptr = (np.r_[0, np.cumsum(np.bincount(cols - 1, minlength=n))] + 1).astype(np.int32)
    Acsc = J.csc_tensor(dev(colptr), dev(rows[o]), dev(val[o]), (m, n))
    B = torch.randn(k, n, device="cuda").t()
    C = torch.zeros(k, m, device="cuda").t()
    stream = torch.cuda.current_stream()

    def ms(fn, reps=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(reps):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return round(s.elapsed_time(e) / reps, 4)

    out = []
    for name, M in (("coo_shuffled", A), ("csc", Acsc)):
        r = {"matrix": name, "m": m, "n": n, "nnz": int(rows.size), "k": k}
        r["plain_cached_ms"] = ms(lambda: J.execute(J.SpMMOp, M, B, C))
        PLAN_CACHE.clear()
        cache_on, PLAN_CACHE.enabled = PLAN_CACHE.enabled, False
        try:
            r["plain_uncached_ms"] = ms(lambda: J.execute(J.SpMMOp, M, B, C))
        finally:
            PLAN_CACHE.enabled = cache_on
        h = J.prepare(J.HIPBackend(), J.SpMMOp, M, n_cols=k)
        r["plan_ms"] = ms(lambda: J.execute(h, B, C))
        del h
        log(f"coo/csc spmm: {r}")
        out.append(r)
    return out


def gather_overlap():
    """Would config 3's second column chunk cost less if its transpose ran
    while the first chunk's gathers do?  Times the chunk's gathers
    (rows_probe_kernel, 64 rows per wave, as in gather_floor) alone, the
    transpose of a 64-column chunk of a column-major 1M x 128 B into a
    row-major 1M x 64 copy (torch's strided copy) alone, the two back to back,
    and the two at once on two streams of default priority joined by events."""
    import ctypes
    import torch
    lib = probe_lib()
    lib.jlust_probe_rows_f32.restype = ctypes.c_int
    lib.jlust_probe_rows_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                         ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    nrows, row, count, per_wave = 1_000_000, 64, 32_000_000, 64
    g = torch.Generator(device="cuda").manual_seed(3)
    src = torch.randn(nrows * row, dtype=torch.float32, device="cuda")
    idx = torch.randint(0, nrows, (count,), generator=g, device="cuda", dtype=torch.int64).to(torch.int32)
    out = torch.empty(((count + per_wave - 1) // per_wave) * 64, dtype=torch.float32, device="cuda")
    bt = torch.randn(128, nrows, device="cuda")       # B column-major: row c of bt is column c of B
    dst = torch.empty(nrows, 64, device="cuda")
    cur = torch.cuda.current_stream()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def gather(st):
        assert lib.jlust_probe_rows_f32(src.data_ptr(), nrows, row, idx.data_ptr(), count, per_wave,
                                        out.data_ptr(), st.cuda_stream) == 0

    def transpose(st):
        with torch.cuda.stream(st):
            dst.copy_(bt[64:128].t())

    def concurrent():
        e0 = torch.cuda.Event()
        e0.record(cur)
        s1.wait_event(e0)
        s2.wait_event(e0)
        gather(s1)
        transpose(s2)
        for st in (s1, s2):
            e = torch.cuda.Event()
            e.record(st)
            cur.wait_event(e)

    cases = (("gathers alone", lambda: gather(cur)), ("transpose alone", lambda: transpose(cur)),
             ("gathers then transpose, one stream", lambda: (gather(cur), transpose(cur))),
             ("gathers and transpose on two streams", concurrent))
    res = []
    for name, fn in cases:
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        a.record(cur)
        for _ in range(reps):
            fn()
        b.record(cur)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        res.append({"case": name, "ms": round(ms, 4)})
        log(f"{name}: {ms:.3f} ms")
    return res


def mall_probe():
    """Does a buffer written by one kernel come back faster in the next than a
    cold one (from the 256 MB MALL rather than HBM)?  For sizes 16-512 MB:
    the write, a read right after it, a read after 160 MB of other reads in
    between, and a read after a 1 GiB flush; 16-byte nontemporal loads,
    2048 workgroups, best of 5 (bench_probes.hip)."""
    import ctypes
    import torch
    lib = probe_lib()
    lib.jlust_probe_stream.restype = ctypes.c_int
    lib.jlust_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_void_p]
    MB = 1 << 20
    grid = 2048
    P = torch.empty(512 * MB, dtype=torch.uint8, device="cuda")
    E = torch.empty(160 * MB, dtype=torch.uint8, device="cuda")
    F = torch.empty(1024 * MB, dtype=torch.uint8, device="cuda")
    out = torch.empty(grid * 256, dtype=torch.float64, device="cuda")
    stream = torch.cuda.current_stream()

    def run(buf, nbytes, write):
        assert lib.jlust_probe_stream(buf.data_ptr(), nbytes, int(write), grid, out.data_ptr(),
                                      stream.cuda_stream) == 0

    for b in (P, E, F):
        run(b, b.numel(), True)
    res = []
    for mb in (16, 32, 64, 128, 256, 384, 512):
        nb = mb * MB
        best = {}
        for _ in range(5):
            for case in ("write", "read_after_write", "read_after_160MB", "read_cold"):
                run(F, F.numel(), False)
                if case != "write":
                    run(P, nb, True)
                if case == "read_after_160MB":
                    run(E, E.numel(), False)
                if case == "read_cold":
                    run(F, F.numel(), False)
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record(stream)
                run(P, nb, case == "write")
                e.record(stream)
                torch.cuda.synchronize()
                t = s.elapsed_time(e)
                best[case] = min(best.get(case, 1e9), t)
        row = {"MB": mb}
        for case, t in best.items():
            row[case + "_us"] = round(t * 1e3, 1)
            row[case + "_TBps"] = round(nb / (t * 1e-3) / 1e12, 2)
        res.append(row)
        log(f"mall probe {mb} MB: {row}")
    del P, E, F, out
    return res


def gather_probe():
    """8-byte random gathers by bench_probes.hip (8 per thread),
    from the whole source or, XCD-sliced, from source/8 per XCD (the access
    pattern of the column-sliced SpMV plan)."""
    import ctypes
    import torch
    lib = probe_lib()
    lib.jlust_probe_gather_f64.restype = ctypes.c_int
    lib.jlust_probe_gather_f64.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                           ctypes.c_uint32, ctypes.c_void_p]
    total = 64 * 2**20
    nthreads = total // 8
    idx = torch.empty(total, dtype=torch.int32, device="cuda")
    out = torch.empty(nthreads, dtype=torch.float64, device="cuda")
    stream = torch.cuda.current_stream()
    g = torch.Generator(device="cuda").manual_seed(1)
    res = []
    for sliced in (0, 1):
        for mb in (1, 4, 8, 32, 256):
            n = mb * 2**20 // 8
            rng = n // 8 if sliced else n
            src = torch.rand(n, dtype=torch.float64, device="cuda")
            idx.random_(0, rng, generator=g)
            call = lambda: lib.jlust_probe_gather_f64(src.data_ptr(), n, idx.data_ptr(), out.data_ptr(),
                                                      nthreads, sliced, rng, stream.cuda_stream)
            for _ in range(3):
                assert call() == 0
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            s.record(stream)
            for _ in range(reps):
                call()
            e.record(stream)
            torch.cuda.synchronize()
            t = s.elapsed_time(e) / reps * 1e-3
            res.append({"kernel": "gather_probe" + (" xcd-sliced" if sliced else ""), "elem_bytes": 8,
                        "source_MB": mb, "per_xcd_MB": mb / 8 if sliced else mb, "gathers": total,
                        "ms": round(t * 1e3, 4), "gathered_GBps": round(total * 8 / t / 1e9, 1),
                        "Ggathers_per_s": round(total / t / 1e9, 2)})
            del src
    return res


def gather_cpol():
    """The 8-byte gathers of gather_probe (whole source) as buffer loads with
    each cache-policy setting (bench_probes.hip, gather_cpol_kernel), from
    1, 4 and 32 MB sources: whether bypassing the L1 (sc0), the streaming
    hint (nt) or system scope (sc1) changes the rate at which random 8-byte
    values come from the L2s or the MALL."""
    import ctypes
    import torch
    lib = probe_lib()
    lib.jlust_probe_gather_cpol_f64.restype = ctypes.c_int
    lib.jlust_probe_gather_cpol_f64.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_int,
                                                ctypes.c_void_p]
    total = 64 * 2**20
    nthreads = total // 8
    idx = torch.empty(total, dtype=torch.int32, device="cuda")
    out = torch.empty(nthreads, dtype=torch.float64, device="cuda")
    stream = torch.cuda.current_stream()
    g = torch.Generator(device="cuda").manual_seed(1)
    names = {0: "default", 1: "sc0", 2: "nt", 3: "sc0 nt", 16: "sc1", 17: "sc0 sc1"}
    res = []
    for mb in (1, 4, 32):
        n = mb * 2**20 // 8
        src = torch.rand(n, dtype=torch.float64, device="cuda")
        idx.random_(0, n, generator=g)
        for cpol, name in names.items():
            call = lambda: lib.jlust_probe_gather_cpol_f64(src.data_ptr(), n, idx.data_ptr(),  # noqa: E731
                                                           out.data_ptr(), nthreads, n, cpol, stream.cuda_stream)
            for _ in range(3):
                assert call() == 0
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            s.record(stream)
            for _ in range(reps):
                call()
            e.record(stream)
            torch.cuda.synchronize()
            t = s.elapsed_time(e) / reps * 1e-3
            res.append({"source_MB": mb, "cpol": name, "gathers": total, "ms": round(t * 1e3, 4),
                        "Ggathers_per_s": round(total / t / 1e9, 2)})
            log(f"{mb} MB, {name}: {t * 1e3:.4f} ms, {total / t / 1e9:.1f} G gathers/s")
        del src
    return res


def _wall_ms(fn, reps=10, warm=3):
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e3


def sweep_spmm():
    """CSR SpMM C = A*B on config 3's matrix (1M x 1M, 32 per row, f32) for
    k = 1 .. 256 (random column-major B), mean wall ms per call, with the
    compulsory-byte rate and the gathered-byte rate (nnz*k*4); then the f32
    SpMV of the same matrix."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    cfg = W.make(3)
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (cfg["m"], cfg["n"]))
    m, n, nnz = cfg["m"], cfg["n"], cfg["colind"].size
    g = torch.Generator(device="cuda").manual_seed(0)
    res = []
    for k in (1, 2, 4, 8, 16, 32, 64, 128, 256):
        B = torch.randn(k, n, device="cuda", generator=g).t()
        C = J.dense_matrix(m, k, dtype=torch.float32)
        ms = _wall_ms(lambda: J.execute(J.SpMMOp, A, B, C))
        alg = 8 * nnz + 4 * (m + 1) + 4 * n * k + 4 * m * k
        res.append({"k": k, "ms": round(ms, 4), "GBps": round(alg / ms / 1e6, 1),
                    "gathered_GBps": round(nnz * k * 4 / ms / 1e6, 1)})
        log(f"SpMM k={k}: {ms:.3f} ms")
        del B, C
    x = torch.randn(n, device="cuda", generator=g)
    y = torch.empty(m, device="cuda")
    res.append({"spmv_f32_ms": round(_wall_ms(lambda: J.execute(J.SpMVOp, A, x, y)), 4)})
    return res


def sweep_sddmm():
    """SDDMM out = S .* (A B^T) at config 4's mask (500k x 500k, 32 per row,
    f32) for K = 1 .. 256 (random column-major A, B), mean wall ms per call."""
    import torch
    import jlust_amd as J
    from jlust_amd import workloads as W
    cfg = W.make(4)
    m, n, nnz = cfg["m"], cfg["n"], cfg["colind"].size
    S = dev(cfg["mask"])
    out = torch.empty_like(S)
    Cs = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), out, (m, n))
    g = torch.Generator(device="cuda").manual_seed(0)
    res = []
    for K in (1, 2, 4, 8, 16, 32, 64, 128, 256):
        Am = torch.randn(K, m, device="cuda", generator=g).t()
        Bm = torch.randn(n, K, device="cuda", generator=g).t()
        ms = _wall_ms(lambda: J.execute(J.SDDMMOp, Am, Bm, Cs, mask=S))
        alg = 4 * (m + 1) + 12 * nnz + 4 * m * K + 4 * n * K
        res.append({"K": K, "ms": round(ms, 4), "GBps": round(alg / ms / 1e6, 1),
                    "gathered_GBps": round(nnz * K * 4 / ms / 1e6, 1)})
        log(f"SDDMM K={K}: {ms:.3f} ms")
        del Am, Bm
    return res


def sweep_spmv():
    """SpMV on random m x n matrices with L uniformly random columns per row
    (f64): the plain call, plans with column slices off (vector kernel where
    the rows allow it), forced XCD slices, forced LDS bins, and the plan's own
    choice, in mean wall ms per call."""
    import torch
    import jlust_amd as J
    rng = np.random.default_rng(0)
    res = []
    for m, n in ((4_000_000, 4_000_000), (1_000_000, 4_000_000), (4_000_000, 1_000_000),
                 (4_000_000, 500_000), (1_000_000, 1_000_000), (2_000_000, 2_000_000)):
        for L in (1, 2, 4, 6, 8, 12, 16):
            rp = (np.arange(m + 1, dtype=np.int64) * L + 1).astype(np.int32)
            ci = rng.integers(0, n, (m, L))
            ci.sort(axis=1)
            A = J.csr_tensor(dev(rp), dev((ci.reshape(-1) + 1).astype(np.int32)),
                             dev(rng.uniform(-1, 1, m * L)), (m, n))
            x = dev(rng.uniform(-1, 1, n))
            y = torch.empty(m, dtype=torch.float64, device="cuda")
            e = {"m": m, "n": n, "per_row": L, "plain_ms": round(_wall_ms(lambda: J.execute(J.SpMVOp, A, x, y)), 4)}
            for key, val in (("unsliced", "0"), ("sliced", "1"), ("binned", "2"), ("auto", None)):
                if val is None:
                    os.environ.pop("JLUST_HIP_SPMV_SLICE", None)
                else:
                    os.environ["JLUST_HIP_SPMV_SLICE"] = val
                h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
                e[f"{key}_ms"] = round(_wall_ms(lambda: J.execute(h, x, y)), 4)
                e[f"{key}_kernel"] = h.kernel()
                del h
            os.environ.pop("JLUST_HIP_SPMV_SLICE", None)
            res.append(e)
            log(f"SpMV {m}x{n} L={L}: {e}")
            del A, x, y
            torch.cuda.empty_cache()
    return res


def _stencil_csr(shape, offsets):
    """CSR (Int32, 1-based) of a grid operator: row i = grid point p, its
    columns p + o for the stencil offsets o that stay inside the grid, values
    uniform in [-1, 1].  Columns are sorted because the offsets are."""
    rng = np.random.default_rng(7)
    dims = np.array(shape)
    m = int(np.prod(dims))
    coords = np.stack(np.unravel_index(np.arange(m), shape), axis=1)
    cols, valid = [], []
    for off in offsets:
        c = coords + np.array(off)
        ok = np.all((c >= 0) & (c < dims), axis=1)
        cols.append(np.ravel_multi_index(tuple(np.clip(c, 0, dims - 1).T), shape))
        valid.append(ok)
    cols, valid = np.stack(cols, axis=1), np.stack(valid, axis=1)
    lens = valid.sum(axis=1)
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    ci = cols[valid]
    return (rp + 1).astype(np.int32), (ci + 1).astype(np.int32), rng.uniform(-1, 1, ci.size), m


def structured_spmv():
    """SpMV (f64) on structured matrices of config 2's size, the kind the
    reference's SuiteSparse benchmark runs (bench_suitesparse.jl): a 2D
    5-point and a 3D 7-point Laplacian, and random columns in a band of
    +-256 around the diagonal (16 per row).  The plain call and the plan's own
    choice, per call from HIP events over 50 back-to-back calls, in effective
    GB/s by the reference's byte formula (12 nnz + 4 (m + 1) + 8 (n + m))."""
    import torch
    import jlust_amd as J
    res = []
    cases = []
    rp, ci, v, m = _stencil_csr((2048, 2048), [(-1, 0), (0, -1), (0, 0), (0, 1), (1, 0)])
    cases.append(("2D 5-point Laplacian 2048^2", rp, ci, v, m, m))
    rp, ci, v, m = _stencil_csr((160, 160, 160), [(-1, 0, 0), (0, -1, 0), (0, 0, -1), (0, 0, 0), (0, 0, 1),
                                                  (0, 1, 0), (1, 0, 0)])
    cases.append(("3D 7-point Laplacian 160^3", rp, ci, v, m, m))
    rng = np.random.default_rng(8)
    m = 4_000_000
    offs = np.sort(rng.choice(513, (m, 16), replace=True) - 256, axis=1)
    cols = np.clip(np.arange(m)[:, None] + offs, 0, m - 1)
    cols = np.sort(cols, axis=1)
    keep = np.ones_like(cols, bool)
    keep[:, 1:] = cols[:, 1:] != cols[:, :-1]          # distinct columns per row
    lens = keep.sum(axis=1)
    rp = np.zeros(m + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    ci = cols[keep]
    cases.append(("random band +-256, 16 per row, 4M", (rp + 1).astype(np.int32), (ci + 1).astype(np.int32),
                  rng.uniform(-1, 1, ci.size), m, m))
    for name, rp, ci, v, m, n in cases:
        nnz = ci.size
        nbytes = 12 * nnz + 4 * (m + 1) + 8 * (n + m)
        A = J.csr_tensor(dev(rp), dev(ci), dev(v), (m, n))
        x = dev(np.random.default_rng(9).uniform(-1, 1, n))
        y = torch.empty(m, dtype=torch.float64, device="cuda")
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        e = {"matrix": name, "m": m, "nnz": int(nnz), "algorithmic_bytes": int(nbytes), "plan_kernel": h.kernel()}
        for key, fn in (("plain", lambda: J.execute(J.SpMVOp, A, x, y)), ("plan", lambda: J.execute(h, x, y))):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(50):
                fn()
            b.record()
            torch.cuda.synchronize()
            ms = a.elapsed_time(b) / 50
            e[f"{key}_us"] = round(ms * 1e3, 1)
            e[f"{key}_GBps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        res.append(e)
        log(f"{name}: {e}")
        del A, x, y, h
        torch.cuda.empty_cache()
    return res


def stream_ceiling():
    """Attainable HBM streaming rates on this box for a 2 GiB f64 tensor: a
    device copy (read + write), a read-only reduction and a fill, in TB/s of
    bytes moved."""
    import torch
    a = torch.empty(1 << 28, dtype=torch.float64, device="cuda").uniform_()
    b = torch.empty_like(a)
    nbytes = a.numel() * 8
    out = {"bytes": nbytes}
    for key, fn, mult in (("copy_TBps", lambda: b.copy_(a), 2), ("read_sum_TBps", lambda: a.sum(), 1),
                          ("write_fill_TBps", lambda: b.fill_(1.0), 1)):
        ms = _wall_ms(fn, reps=20)
        out[key] = round(mult * nbytes / (ms * 1e-3) / 1e12, 3)
    del a, b
    return out


def mfma_peak():
    """Sustained fp32 matrix-core rate (bench_probes.hip,
    mfma_probe_kernel) for 1, 2 and 4 waves per SIMD, beside the published
    dense fp32 MFMA peak."""
    import ctypes
    import torch
    lib = probe_lib()
    lib.jlust_probe_mfma_f32.restype = ctypes.c_int
    lib.jlust_probe_mfma_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream()
    iters, chains = 20000, 4
    res = []
    for waves_per_simd in (1, 2, 4):
        blocks = cus * waves_per_simd          # 4 waves per block = one per SIMD
        out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        call = lambda: lib.jlust_probe_mfma_f32(out.data_ptr(), blocks, iters, stream.cuda_stream)
        assert call() == 0
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        s.record(stream)
        for _ in range(reps):
            call()
        e.record(stream)
        torch.cuda.synchronize()
        t = s.elapsed_time(e) / reps * 1e-3
        flops = blocks * 4 * iters * chains * 2048
        res.append({"waves_per_simd": waves_per_simd, "blocks": blocks, "ms": round(t * 1e3, 3),
                    "TFLOPs": round(flops / t / 1e12, 2),
                    "frac_of_published": round(flops / t / 1e12 / MFMA_F32_PEAK_TFLOPS, 4)})
        del out
    return res


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev(a):
    import torch
    if a.ndim == 2:
        return torch.from_numpy(np.ascontiguousarray(a.T)).cuda().t()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def build_step(cfg, use_plan=False):
    """Returns (step_fn, dominant_kernel_name, bound, algorithmic units)."""
    import torch
    import jlust_amd as J
    kind = cfg["kind"]
    m, n = cfg["m"], cfg["n"]
    if kind == "csr_spmv":
        A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
        x = dev(cfg["x"])
        y = torch.empty(m, dtype=A.dtype, device="cuda")
        if use_plan:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
            torch.cuda.synchronize()
            h.build_ms = (time.perf_counter() - t0) * 1e3
            kname = ("binned_slice_kernel + binned_bin_kernel" if h.kernel() == "binned"
                     else f"csr_spmv_{h.kernel()}_kernel")
            return (lambda: J.execute(h, x, y)), kname, "hbm", (A, x, y, h)
        return (lambda: J.execute(J.SpMVOp, A, x, y)), "csr_spmv_merge_kernel", "hbm", (A, x, y)
    if kind == "csr_spmm":
        A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
        B = dev(cfg["B"])
        C = J.dense_matrix(m, cfg["k"], dtype=A.dtype)
        # One call: transpose_kernel + csr_spmm_kernel per column chunk of B.
        return (lambda: J.execute(J.SpMMOp, A, B, C)), \
            "transpose_kernel + csr_spmm_kernel (per column chunk)", "hbm", (A, B, C)
    if kind == "csr_sddmm":
        S = dev(cfg["mask"])
        out = torch.empty_like(S)
        Cs = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), out, (m, n))
        A, B = dev(cfg["A"]), dev(cfg["B"])
        return (lambda: J.execute(J.SDDMMOp, A, B, Cs, mask=S)), "csr_sddmm_kernel", "hbm", \
            (S, out, Cs, A, B)
    if kind == "bsr_spmm":
        A = J.bsr_tensor(dev(cfg["browptr"]), dev(cfg["bcolind"]), dev(cfg["val"]), (m, n))
        B = dev(cfg["B"])
        C = J.dense_matrix(m, cfg["k"], dtype=torch.float32)
        return (lambda: J.execute(J.SpMMOp, A, B, C)), "bsr16_spmm_wide_strip_kernel", "mfma", (A, B, C)
    raise ValueError(kind)


def cpu_baseline(cfg, budget_s):
    """Time the oracle (C restatement of JLUST's CPU path, OpenMP over 64-row
    chunks) on a bounded sample of the same workload on this host."""
    from oracle import oracle as O
    from jlust_amd import workloads as W
    nt = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or O.default_threads()
    kind = cfg["kind"]
    rows_frac = 1.0
    if kind == "csr_spmv":
        fn = lambda: O.csr_spmv(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"], nthreads=nt)
        sample = "full matrix, repeated"
        sub = cfg
    else:
        # A contiguous block of rows (block-rows for BSR), sized from a probe.
        m_units = cfg["mb"] if kind == "bsr_spmm" else cfg["m"]
        probe = max(1, m_units // 2000)

        def make_sub(units):
            if kind == "bsr_spmm":
                bp = cfg["browptr"][:units + 1]
                q1 = int(bp[-1]) - 1
                return dict(cfg, browptr=bp, bcolind=cfg["bcolind"][:q1],
                            val=cfg["val"][:q1 * 256], mb=units, m=units * 16)
            rp = cfg["rowptr"][:units + 1]
            p1 = int(rp[-1]) - 1
            d = dict(cfg, rowptr=rp, colind=cfg["colind"][:p1], m=units)
            if kind == "csr_spmm":
                d["val"] = cfg["val"][:p1]
            else:
                d["mask"] = cfg["mask"][:p1]
                d["A"] = np.asfortranarray(cfg["A"][:units])
            return d

        def runner(d):
            if kind == "csr_spmm":
                return lambda: O.csr_spmm(d["rowptr"], d["colind"], d["val"], d["B"], nthreads=nt)
            if kind == "csr_sddmm":
                return lambda: O.csr_sddmm(d["rowptr"], d["colind"], d["A"], d["B"],
                                           mask=d["mask"], nthreads=nt)
            return lambda: O.bsr_spmm(d["browptr"], d["bcolind"], d["val"], 16, d["B"],
                                      nthreads=nt)
        t0 = time.perf_counter()
        runner(make_sub(probe))()
        tp = max(time.perf_counter() - t0, 1e-4)
        units = int(min(m_units, max(probe, probe * (budget_s / 4) / tp)))
        sub = make_sub(units)
        fn = runner(sub)
        rows_frac = units / m_units
        sample = f"first {units} of {m_units} {'block-rows' if kind == 'bsr_spmm' else 'rows'}"
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    tmin = min(times)
    nbytes = W.algorithmic_bytes(sub) if kind != "csr_spmv" else W.algorithmic_bytes(cfg)
    return {"value": round(nbytes / tmin / 1e9, 3), "unit": "GB/s", "cores": nt,
            "kind": "port",
            "sample": f"{sample}; min of {len(times)} runs; oracle/jlust_cpu.c "
                      f"(C restatement of JLUST EmitterBackend CPU path, -O3 -ffp-contract=off, "
                      f"OpenMP {nt} threads, 64-row chunks); host nproc={os.cpu_count()}",
            "seconds_per_run": round(tmin, 6), "rows_fraction": round(rows_frac, 6),
            "gflops": round(W.flops(sub) / tmin / 1e9, 3) if kind != "csr_spmv" else
            round(W.flops(cfg) / tmin / 1e9, 3)}


def plain_call_timings(cfg, steps, warmup):
    """The plain call execute(SpMVOp, A, x, y) on the same matrix, as unchanged
    JLUST code makes it: its first call (one synchronised call: the plain
    kernels, no plan yet), its steady state (from the third call on the plan
    cache runs a plan built for this matrix), and the steady state with the
    cache off (the plain kernels every call)."""
    import torch
    from jlust_amd import hip_backend as HB
    from jlust_amd import workloads as W
    nbytes = W.algorithmic_bytes(cfg)
    pstep, pkname, _, pkeep = build_step(cfg, use_plan=False)
    HB.PLAN_CACHE.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    pstep()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1e3
    p_ms, p_launch = timed(pstep, steps, warmup)
    info = HB.PLAN_CACHE.info()
    HB.PLAN_CACHE.clear()
    HB.PLAN_CACHE.enabled = False
    try:
        u_ms, u_launch = timed(pstep, steps, warmup)
    finally:
        HB.PLAN_CACHE.enabled = True
    del pkeep
    return {"value": round(nbytes / (p_ms * 1e-3) / 1e9, 3), "ms_per_step": round(p_ms, 6),
            "per_launch_ms": round(p_launch, 6),
            "kernel": f"cached plan ({info[0]['kernel']})" if info else pkname,
            "first_call_ms": round(first_ms, 4),
            "cache": "calls 1-2 on a matrix run the plain kernels; the 3rd builds a plan for it "
                     "(jlust_amd.hip_backend.PLAN_CACHE, JLUST_HIP_PLAN_CACHE=0 turns it off) and "
                     "later calls run that plan; the warm-up covers the switch",
            "uncached": {"value": round(nbytes / (u_ms * 1e-3) / 1e9, 3), "ms_per_step": round(u_ms, 6),
                         "per_launch_ms": round(u_launch, 6), "kernel": pkname}}


def emitter_handle_timing(cfg, keep, steps, warmup):
    """The emitter-form handle call execute(h, A, x, y) as a binding without
    torch's version counters makes it (a Julia ccall binding): every call
    re-reads A's values into the plan -- a refresh of the copy for the
    copying layouts, a pointer for the others -- then runs the product
    (jlust_hip_csr_spmv_plan_execute_values_*)."""
    import torch
    from jlust_amd import _lib
    from jlust_amd import workloads as W
    A, x, y, h = keep
    import jlust_amd as J
    fn = getattr(_lib.lib(), f"jlust_hip_csr_spmv_plan_execute_values_{h.suf}")
    vp, xp, yp = J.nonzeros(A).data_ptr(), x.data_ptr(), y.data_ptr()
    stream = _lib.stream_handle(x.device)

    def step():
        st = fn(h._plan, vp, 1.0, xp, 0.0, yp, stream)
        if st:
            _lib.check(st, "csr_spmv_plan_execute_values")
    e_ms, e_launch = timed(step, steps, warmup)
    h.update_values(A)                # the handle's own record of the values it holds
    torch.cuda.synchronize()
    nbytes = W.algorithmic_bytes(cfg)
    return {"value": round(nbytes / (e_ms * 1e-3) / 1e9, 3), "ms_per_step": round(e_ms, 6),
            "per_launch_ms": round(e_launch, 6), "kernel": h.kernel(),
            "refresh": "values re-read on every call (the binned layout: CSR values in LDS chunks "
                       "written out by run; the sliced layout: a gather through the plan's "
                       "permutation; nothing to copy for merge and vector plans)"}


def timed(step, steps, warmup):
    """W untimed steps, then exactly K steps bracketed by synchronize() (the
    wall-clock pass), then K more steps between one pair of HIP events
    recorded on the launching stream (the kernel pass: the queue runs the K
    steps back to back, so elapsed / K is the step's kernel time without the
    host).  Returns (wall ms per step, kernel ms per step).  One event pair
    over the whole region rather than one per step: at config 1's size (a
    9 us kernel) each extra record adds about 2 us of queue time."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        torch.distributed.barrier()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    return wall * 1e3 / steps, e0.elapsed_time(e1) / steps


def timed_samples(step, est_ms, n=20, min_sample_ms=0.5):
    """Min and median of n samples (the @belapsed statistics of the
    reference's benchmarks, benchmark/bench_suitesparse.jl:174-177), warm:
    each sample is B back-to-back steps between one pair of HIP events, with
    B chosen so that a sample lasts at least min_sample_ms and the two event
    records (about 2 us) stay a small part of it.  Returns (min, median, B)
    in ms per step."""
    import torch
    b = max(1, int(np.ceil(min_sample_ms / max(est_ms, 1e-6))))
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    pairs = []
    for _ in range(n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(b):
            step()
        e1.record(stream)
        pairs.append((e0, e1))
    torch.cuda.synchronize()
    t = np.array([e0.elapsed_time(e1) / b for e0, e1 in pairs])
    return float(t.min()), float(np.median(t)), b


def timed_cold(step, steps):
    """Each of K steps timed alone (an event pair around it) right after a
    1 GiB read that evicts the operands from the L2s and the 256 MB MALL.
    Returns the mean and minimum step time in ms (the two event records add
    about 2 us to each)."""
    import torch
    flush = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(steps):
        flush.sum()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        step()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    del flush
    return float(np.mean(times)), float(np.min(times))


def counters_for(workload):
    """(traffic bytes, counter readings) of a workload's committed rocprofv3
    --pmc passes (profiles/pmc_traffic.json): L2-miss bytes per step, and the
    L2 hit rate per kernel and MFMA utilisation where they were collected."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        e = d.get(workload)
        if e is None:
            return None, None
        extra = {k: e[k] for k in ("l2_hit_pct", "mfma_busy_pct") if k in e}
        return int(e["traffic_bytes"]), extra or None
    except (OSError, ValueError, KeyError):
        return None, None


def host_info():
    """CPU model, sockets and logical CPUs of this host (from /proc/cpuinfo)."""
    model, sockets, logical = None, set(), 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    sockets.add(v)
                elif k == "processor":
                    logical += 1
    except OSError:
        pass
    return {"cpu_model": model, "sockets": len(sockets) or None, "logical_cpus": logical or None,
            "nproc": os.cpu_count()}


def bench_config(config, steps, warmup, cpu_seconds, no_plan=False, no_cpu=False, cold=False):
    """One configuration: W untimed + K timed steps (wall clock) and K steps
    under HIP events, the plain SpMV call beside a plan, the CPU baseline.
    Returns the result object (the headline keys of the JSON line)."""
    import torch
    from jlust_amd import workloads as W

    t0 = time.perf_counter()
    cfg = W.make(config)
    log(f"generated {cfg['name']} in {time.perf_counter() - t0:.1f}s")
    use_plan = cfg["kind"] == "csr_spmv" and not no_plan
    step, kname, bound, keep = build_step(cfg, use_plan=use_plan)
    ms_per_step, per_launch_ms = timed(step, steps, warmup)
    plain = None
    emitter = None
    if use_plan:
        plain = plain_call_timings(cfg, steps, warmup)
        emitter = emitter_handle_timing(cfg, keep, steps, warmup)
    log(f"config {config}: {steps} steps: wall {ms_per_step:.4f} ms/step, events "
        f"{per_launch_ms:.4f} ms/step")
    s_min, s_med, s_b = timed_samples(step, per_launch_ms)
    samples = {"n": 20, "steps_per_sample": s_b, "min_ms_per_step": round(s_min, 6),
               "median_ms_per_step": round(s_med, 6),
               "cache": "warm: back-to-back steps, operands left in the L2s and the MALL by the "
                        "previous step (--cold times steps after a 1 GiB flush)"}
    log(f"config {config}: 20 samples of {s_b} step(s): min {s_min:.4f}, median {s_med:.4f} ms/step")
    cold_res = None
    if cold:
        c_mean, c_min = timed_cold(step, steps)
        cold_res = {"cold_ms_per_step": round(c_mean, 6), "cold_ms_min": round(c_min, 6),
                    "flush": "1 GiB read before each step (L2s and MALL evicted); one event pair "
                             "around each step"}
        log(f"config {config}: cold {c_mean:.4f} ms/step (min {c_min:.4f})")

    nbytes = W.algorithmic_bytes(cfg)
    nflops = W.flops(cfg)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    k_ms = float(per_launch_ms)
    if bound == "hbm":
        achieved = nbytes / (k_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5)}
    else:
        achieved = nflops / (k_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 3), "peak": MFMA_F32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F32_PEAK_TFLOPS, 5)}
    roof["traffic"], counters = counters_for(cfg["name"] + (":plan" if use_plan else ""))
    if counters:
        roof["counters"] = counters
    roof["traffic_source"] = ("profiles/pmc_traffic.json: the committed rocprofv3 --pmc passes of this "
                              "workload (read by bench.py, not measured in this run)")
    roof["traffic_counts"] = ("L2-miss bytes (FETCH_SIZE x 2.0 + WRITE_SIZE, rocprofv3 --pmc): "
                              "requests leaving the L2s, served by the MALL or by HBM")
    roof["kernel"] = kname
    roof["per_launch_ms"] = round(k_ms, 6)
    plan_build_ms = round(keep[3].build_ms, 2) if use_plan else None

    cpu = None
    if not no_cpu:
        log(f"config {config}: timing the CPU baseline (oracle) ...")
        cpu = cpu_baseline(cfg, cpu_seconds)
        cpu.update(host_info())

    nnz_key = "nnzb" if cfg["kind"] == "bsr_spmm" else "nnz"
    nnz_val = int((cfg["browptr"] if cfg["kind"] == "bsr_spmm" else cfg["rowptr"])[-1]) - 1
    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f64" if np.dtype(cfg["dtype"]) == np.float64 else "f32",
        "data": "synthetic (seeded generator, jlust_amd/csrc/workloads.c)",
        "config": {"workload": cfg["name"], "baseline_config": cfg["config"], "m": cfg["m"],
                   "n": cfg["n"], nnz_key: nnz_val, "seed": cfg["seed"],
                   "index": "Int32, 1-based", "plan": bool(use_plan)},
        "gflops": round(nflops / (ms_per_step * 1e-3) / 1e9, 3),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 3),
        "algorithmic_bytes": int(nbytes), "flops": int(nflops),
        "roofline": roof, "samples": samples, "plain_call": plain, "plan_build_ms": plan_build_ms,
        "emitter_handle": emitter, "cpu_baseline": cpu,
    }
    if cold_res is not None:
        out["cold"] = cold_res
    del keep, step, cfg
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


# Steps per configuration when bench.py runs them all (the driver's default
# run): enough events for a stable mean while the five fit in a few minutes.
ALL_STEPS = {1: 200, 2: 200, 3: 30, 4: 30, 5: 30}
# Configurations timed cold as well by default (config 1's figures are quoted
# in both cache states: its operands fit the L2s and the MALL).
COLD_CONFIGS = (1,)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)
    import torch
    if args.calibrate_copy:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": a.numel() * 4}), flush=True)
        return
    if args.gather_floor:
        print(json.dumps({"gather_floor": gather_floor()}), flush=True)
        return
    if args.structured:
        print(json.dumps({"structured_spmv": structured_spmv()}), flush=True)
        return
    if args.gather_cpol:
        print(json.dumps({"gather_cpol": gather_cpol()}), flush=True)
        return
    if args.bsr_f64:
        print(json.dumps({"bsr_f64": bsr_f64()}), flush=True)
        return
    if args.bsr_spmv:
        print(json.dumps({"bsr_spmv": bsr_spmv_powerlaw()}), flush=True)
        return
    if args.coo_spmm:
        print(json.dumps({"coo_spmm": coo_csc_spmm()}), flush=True)
        return
    if args.bsr_long_rows:
        print(json.dumps({"bsr_long_rows": bsr_long_rows()}), flush=True)
        return
    if args.plan_build:
        print(json.dumps({"plan_build": plan_build()}), flush=True)
        return
    if args.spmv_parts:
        print(json.dumps({"spmv_parts": spmv_parts()}), flush=True)
        return
    if args.gather_overlap:
        print(json.dumps({"gather_overlap": gather_overlap()}), flush=True)
        return
    if args.mall_probe:
        print(json.dumps({"mall_probe": mall_probe()}), flush=True)
        return
    if args.gather_ceiling:
        print(json.dumps({"gather_ceiling": gather_ceiling()}), flush=True)
        return
    if args.mfma_peak:
        print(json.dumps({"mfma_peak": mfma_peak()}), flush=True)
        return
    if args.stream_ceiling:
        print(json.dumps({"stream_ceiling": stream_ceiling()}), flush=True)
        return
    if args.sweep_spmm:
        print(json.dumps({"sweep_spmm": sweep_spmm()}), flush=True)
        return
    if args.sweep_sddmm:
        print(json.dumps({"sweep_sddmm": sweep_sddmm()}), flush=True)
        return
    if args.sweep_spmv:
        print(json.dumps({"sweep_spmv": sweep_spmv()}), flush=True)
        return
    if args.convert:
        print(json.dumps({"convert": convert_bench(args.cpu_seconds)}), flush=True)
        return
    if args.coo:
        print(json.dumps({"coo": coo_bench(args.steps or 50, args.warmup or 3, args.cpu_seconds)}),
              flush=True)
        return
    if args.blocks:
        print(json.dumps({"blocks": blocks_bench(args.steps or 200, args.warmup or 10)}), flush=True)
        return
    steps = args.steps if args.steps is not None else ALL_STEPS[args.config]
    warmup = args.warmup if args.warmup is not None else 5
    # The library's device code loaded once, before anything is timed (what a
    # server does at start-up): otherwise the first plan build of the process
    # also pays the runtime's one-time code-object loading.
    import jlust_amd as J
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    J.preload()
    torch.cuda.synchronize()
    preload_ms = (time.perf_counter() - t0) * 1e3
    log(f"preload {preload_ms:.1f} ms")
    out = bench_config(args.config, steps, warmup, args.cpu_seconds, args.no_plan,
                       args.no_cpu_baseline, args.cold or args.config in COLD_CONFIGS)
    out["preload_ms"] = round(preload_ms, 2)
    if not args.only:
        # Every BASELINE configuration in the same run, the headline first.
        rows = []
        for c in sorted(ALL_STEPS):
            if c == args.config:
                e = out
            else:
                e = bench_config(c, ALL_STEPS[c], warmup, args.other_cpu_seconds,
                                 no_cpu=args.no_cpu_baseline, cold=args.cold or c in COLD_CONFIGS)
            rows.append({k: e[k] for k in ("config", "value", "unit", "ms_per_step", "gflops",
                                           "pct_hbm_peak", "dtype", "algorithmic_bytes", "flops",
                                           "roofline", "samples", "plain_call", "plan_build_ms",
                                           "emitter_handle", "cold", "cpu_baseline") if k in e})
        out["all_configs"] = rows
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
