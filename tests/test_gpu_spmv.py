"""GPU parity of CSR SpMV (and its prepared plan) against the CPU oracle.

Bar: |y - y_ref| <= 1e-12 (fp64) / 1e-5 (fp32) x (|alpha||A||x| + |beta||y0|)
elementwise, y_ref from oracle/ (C restatement of JLUST's CPU walker).
"""
import json
import os
import zlib

import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr, sample_rows

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_fixtures.json")))


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def run_spmv(J, rowptr, colind, val, x, m, n, origin=1, alpha=1.0, beta=0.0, y0=None):
    import torch
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n),
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    y = dev(y0) if y0 is not None else torch.full((m,), float("nan"), dtype=A.dtype,
                                                   device="cuda")
    J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
    return host(y)


@pytest.mark.parametrize("case", [c for c in GOLDEN["spmv"] if c["format"] == "CSR"],
                         ids=lambda c: c["name"])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_reference_fixture(J, case, dtype):
    y = run_spmv(J, np.array(case["rowptr"], np.int32), np.array(case["colind"], np.int32),
                 np.array(case["val"], dtype), np.array(case["x"], dtype), case["m"], case["n"],
                 origin=case["origin"])
    np.testing.assert_array_equal(y, np.array(case["y"], dtype))


def test_mul_bang_and_star(J):
    c = GOLDEN["spmv"][0]
    A = J.csr_tensor(dev(np.array(c["rowptr"], np.int32)), dev(np.array(c["colind"], np.int32)),
                     dev(np.array(c["val"])), (3, 3))
    x = dev(np.array(c["x"]))
    y = J.matmul(A, x)
    np.testing.assert_array_equal(host(y), c["y"])
    y2 = dev(np.ones(3))
    J.mul_(y2, A, x, 2.0, 3.0)
    np.testing.assert_array_equal(host(y2), 2 * np.array(c["y"]) + 3.0)


SHAPES = [
    ("tiny", dict(m=5, n=7, density=0.5)),
    ("empty_rows", dict(m=3000, n=500, density=0.002)),
    ("one_row_long", dict(m=1, n=300_000, lengths=[250_000])),
    ("long_rows_mix", dict(m=4000, n=100_000, lengths=np.r_[np.full(3990, 3), np.full(10, 20_000)])),
    ("all_empty", dict(m=10_000, n=10, lengths=np.zeros(10_000, np.int64))),
    ("dense_rows", dict(m=300, n=300, density=0.9)),
    ("uniform_medium", dict(m=50_000, n=50_000, lengths=np.full(50_000, 16))),
]


@pytest.mark.parametrize("name,kw", SHAPES, ids=[s[0] for s in SHAPES])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("origin", [1, 0])
def test_random_shapes(J, O, name, kw, dtype, origin):
    m, n = kw["m"], kw["n"]
    rowptr, colind, val = random_csr(m, n, density=kw.get("density"), lengths=kw.get("lengths"),
                                     seed=zlib.crc32(name.encode()) % 1000, origin=origin, dtype=dtype)
    x = np.random.default_rng(1).uniform(-1, 1, n).astype(dtype)
    y = run_spmv(J, rowptr, colind, val, x, m, n, origin=origin)
    ref = O.csr_spmv(rowptr, colind, val, x, origin=origin)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, origin=origin)
    assert_within(y, ref, absref, dtype, name)


@pytest.mark.parametrize("alpha,beta", [(2.5, 0.0), (1.0, 1.0), (-0.5, 2.0), (0.0, 3.0)])
def test_alpha_beta(J, O, alpha, beta):
    m, n = 20_000, 20_000
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(3).integers(0, 40, m),
                                     seed=5)
    x = np.random.default_rng(4).uniform(-1, 1, n)
    y0 = np.random.default_rng(5).uniform(-1, 1, m)
    y = run_spmv(J, rowptr, colind, val, x, m, n, alpha=alpha, beta=beta, y0=y0)
    ref = O.csr_spmv(rowptr, colind, val, x, alpha=alpha, beta=beta, y0=y0)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, alpha=alpha, beta=beta, y0=y0)
    assert_within(y, ref, absref, np.float64, f"alpha={alpha} beta={beta}")


def test_beta_zero_is_write_only(J):
    """beta == 0 never reads y: NaN in y does not leak (spmv.jl:167-168)."""
    c = GOLDEN["spmv"][0]
    y = run_spmv(J, np.array(c["rowptr"], np.int32), np.array(c["colind"], np.int32),
                 np.array(c["val"]), np.array(c["x"]), 3, 3,
                 y0=np.full(3, np.nan), beta=0.0)
    np.testing.assert_array_equal(y, c["y"])


def test_deterministic(J):
    import torch
    from jlust_amd import workloads as W
    cfg = W.make(2, scale=8)
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (cfg["m"], cfg["n"]))
    x = dev(cfg["x"])
    y1 = torch.empty(cfg["m"], dtype=torch.float64, device="cuda")
    y2 = torch.empty_like(y1)
    J.execute(J.SpMVOp, A, x, y1)
    J.execute(J.SpMVOp, A, x, y2)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("config", [1, 2])
def test_benchmark_config_full(J, O, config):
    """Full BASELINE configs 1 and 2 against the oracle, every row."""
    from jlust_amd import workloads as W
    cfg = W.make(config)
    y = run_spmv(J, cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"], cfg["m"], cfg["n"])
    ref = O.csr_spmv(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    absref = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    assert_within(y, ref, absref, np.float64, cfg["name"])


def test_plan_execute_and_update_values(J, O):
    import torch
    from jlust_amd import workloads as W
    cfg = W.make(2, scale=16)
    m, n = cfg["m"], cfg["n"]
    A = J.csr_tensor(dev(cfg["rowptr"]), dev(cfg["colind"]), dev(cfg["val"]), (m, n))
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    x = dev(cfg["x"])
    y = torch.empty(m, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, h, x, y)
    ref = O.csr_spmv(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    absref = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    assert_within(host(y), ref, absref, np.float64, "plan")
    # update_values!: same pattern, new values; plan keeps its partition.
    val2 = -2.0 * cfg["val"]
    A2 = J.csr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(val2), (m, n))
    J.update_values_(h, A2)
    J.execute(h, x, y, alpha=1.0, beta=0.0)
    ref2 = O.csr_spmv(cfg["rowptr"], cfg["colind"], val2, cfg["x"])
    absref2 = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], val2, cfg["x"])
    assert_within(host(y), ref2, absref2, np.float64, "plan after update_values!")


def test_power_law_sampled_rows_f32(J, O):
    """fp32 on the power-law pattern (scaled config 2)."""
    from jlust_amd import workloads as W
    cfg = W.make(2, scale=4)
    val = cfg["val"].astype(np.float32)
    x = cfg["x"].astype(np.float32)
    y = run_spmv(J, cfg["rowptr"], cfg["colind"], val, x, cfg["m"], cfg["n"])
    rows = np.random.default_rng(0).choice(cfg["m"], 20_000, replace=False)
    rp, ci, v, _ = sample_rows(cfg["rowptr"], cfg["colind"], val, rows)
    ref = O.csr_spmv(rp, ci, v, x)
    absref = O.csr_spmv_absref(rp, ci, v, x)
    assert_within(y[rows], ref, absref, np.float32, "powerlaw f32")


def test_errors(J):
    import torch
    c = GOLDEN["spmv"][0]
    A = J.csr_tensor(dev(np.array(c["rowptr"], np.int32)), dev(np.array(c["colind"], np.int32)),
                     dev(np.array(c["val"])), (3, 3))
    with pytest.raises(J.IncompatibleExtents):
        J.execute(J.SpMVOp, A, dev(np.ones(4)), dev(np.zeros(3)))
    with pytest.raises(J.UnsupportedValueType):
        J.execute(J.SpMVOp, A, dev(np.ones(3, np.float32)), dev(np.zeros(3, np.float32)))
    y_fn = dev(np.zeros(3))
    J.execute(J.SpMVOp, A, dev(np.ones(3)), y_fn, input_fn=lambda v: 2 * v)   # SpMV takes input_fn
    assert host(y_fn).tolist() == [6.0, 6.0, 18.0]
    with pytest.raises(J.UnsupportedFormat, match="belong to SpMV"):
        J.execute(J.SpMMOp, A, J.dense_matrix(3, 2, fill=1.0), J.dense_matrix(3, 2),
                  input_fn=lambda v: 2 * v)
    # Int64 indices run on their Int32 narrowing (the golden answer); other
    # index types are UnsupportedIndexType
    A64 = J.csr_tensor(dev(np.array(c["rowptr"], np.int64)), dev(np.array(c["colind"], np.int64)),
                       dev(np.array(c["val"])), (3, 3))
    y64 = dev(np.zeros(3))
    J.execute(J.SpMVOp, A64, dev(np.ones(3)), y64)
    assert host(y64).tolist() == [3.0, 3.0, 9.0]
    A16 = J.csr_tensor(dev(np.array(c["rowptr"], np.int16)), dev(np.array(c["colind"], np.int16)),
                       dev(np.array(c["val"])), (3, 3))
    with pytest.raises(J.UnsupportedIndexType):
        J.execute(J.SpMVOp, A16, dev(np.ones(3)), dev(np.zeros(3)))
    Ah = J.csr_tensor(torch.tensor(c["rowptr"], dtype=torch.int32),
                      torch.tensor(c["colind"], dtype=torch.int32), torch.tensor(c["val"]), (3, 3))
    with pytest.raises(J.UnsupportedFormat):
        J.execute(J.SpMVOp, Ah, torch.ones(3, dtype=torch.float64),
                  torch.zeros(3, dtype=torch.float64))
    # C ABI argument checks (status codes -> exceptions)
    L = J._lib.lib()
    st = L.jlust_hip_csr_spmv_f64_i32(-1, 3, 5, 1, None, None, None, 1.0, None, 0.0, None, None)
    assert st == 1 and "negative" in J._lib.last_error()
    st = L.jlust_hip_csr_spmv_f64_i32(3, 3, 5, 2, None, None, None, 1.0, None, 0.0, None, None)
    assert st == 5


def test_device_arch(J):
    import ctypes
    buf = ctypes.create_string_buffer(64)
    assert J._lib.lib().jlust_hip_device_arch(buf, 64) == 0
    assert buf.value.decode().startswith("gfx950")


# ------------------------------------------------- column-sliced SpMV plans

def run_plan(J, rowptr, colind, val, x, m, n, origin=1, alpha=1.0, beta=0.0, y0=None):
    import torch
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n),
                     origin=J.OneBased() if origin == 1 else J.ZeroBased())
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
    y = dev(y0) if y0 is not None else torch.full((m,), float("nan"), dtype=A.dtype,
                                                   device="cuda")
    J.execute(h, dev(x), y, alpha=alpha, beta=beta)
    return host(y), h, A


@pytest.mark.parametrize("name,kw", SHAPES, ids=[s[0] for s in SHAPES])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_plan_sliced_random_shapes(J, O, name, kw, dtype, monkeypatch):
    """JLUST_HIP_SPMV_SLICE=1 forces the 8-column-slice layout on any n >= 8."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "1")
    m, n = kw["m"], kw["n"]
    origin = 0 if name in ("empty_rows", "dense_rows") else 1
    rowptr, colind, val = random_csr(m, n, density=kw.get("density"), lengths=kw.get("lengths"),
                                     seed=zlib.crc32(name.encode()) % 1000 + 7, origin=origin,
                                     dtype=dtype)
    x = np.random.default_rng(2).uniform(-1, 1, n).astype(dtype)
    y, _, _ = run_plan(J, rowptr, colind, val, x, m, n, origin=origin)
    ref = O.csr_spmv(rowptr, colind, val, x, origin=origin)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, origin=origin)
    assert_within(y, ref, absref, dtype, "sliced " + name)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_plan_sliced_auto_alpha_beta_update(J, O, dtype, monkeypatch):
    """Scaled config 2 with n = 1M: x is 8 MB (f64) / 4 MB (f32); the plan
    re-lays A out (LDS bins) when x exceeds 4 MB."""
    monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)
    from jlust_amd import workloads as W
    cfg = W.make(2, scale=4)
    val = cfg["val"].astype(dtype)
    x = cfg["x"].astype(dtype)
    y0 = np.random.default_rng(3).uniform(-1, 1, cfg["m"]).astype(dtype)
    y, h, A = run_plan(J, cfg["rowptr"], cfg["colind"], val, x, cfg["m"], cfg["n"], alpha=1.5,
                       beta=-0.5, y0=y0)
    ref = O.csr_spmv(cfg["rowptr"], cfg["colind"], val, x, 1.5, -0.5, y0)
    absref = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], val, x, 1.5, -0.5, y0)
    assert_within(y, ref, absref, dtype, "sliced auto")
    val2 = (val * -3.0).astype(dtype)
    J.update_values_(h, J.csr_tensor(A.pos_buffers[1], A.crd_buffers[1], dev(val2),
                                     (cfg["m"], cfg["n"])))
    import torch
    yt = torch.empty(cfg["m"], dtype=A.dtype, device="cuda")
    J.execute(h, dev(x), yt)
    ref2 = O.csr_spmv(cfg["rowptr"], cfg["colind"], val2, x)
    absref2 = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], val2, x)
    assert_within(host(yt), ref2, absref2, dtype, "sliced after update_values!")


def test_plan_sliced_full_config2_deterministic(J, O, monkeypatch):
    monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)
    import torch
    from jlust_amd import workloads as W
    cfg = W.make(2)
    y, h, A = run_plan(J, cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"], cfg["m"], cfg["n"])
    ref = O.csr_spmv(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    absref = O.csr_spmv_absref(cfg["rowptr"], cfg["colind"], cfg["val"], cfg["x"])
    assert_within(y, ref, absref, np.float64, "sliced full config 2")
    y2 = torch.empty(cfg["m"], dtype=torch.float64, device="cuda")
    J.execute(h, dev(cfg["x"]), y2)
    np.testing.assert_array_equal(host(y2), y)


@pytest.mark.parametrize("n,per_row,expect", [(3_200_000, 2, "vector"), (3_200_000, 8, "binned"),
                                               (1_000_000, 4, "vector"), (1_000_000, 8, "binned")])
def test_plan_slicing_threshold(J, O, n, per_row, expect, monkeypatch):
    """Random columns, n x n: with x of 25.6 MB the LDS-binned layout pays
    from 7M entries, with x of 8 MB (wide slices shared by several workgroups)
    from 6M; fewer entries keep the vector kernel.  Both plans match the
    oracle."""
    monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)
    monkeypatch.delenv("JLUST_HIP_SPMV_VECTOR", raising=False)
    m = n
    rng = np.random.default_rng(per_row)
    colind = np.sort(rng.integers(0, n, (m, per_row)), axis=1)
    colind = (colind.reshape(-1) + 1).astype(np.int32)
    rowptr = (np.arange(m + 1, dtype=np.int64) * per_row + 1).astype(np.int32)
    val = rng.uniform(-1, 1, colind.size)
    x = rng.uniform(-1, 1, n)
    y, h, _ = run_plan(J, rowptr, colind, val, x, m, n)
    assert h.kernel() == expect
    ref = O.csr_spmv(rowptr, colind, val, x)
    absref = O.csr_spmv_absref(rowptr, colind, val, x)
    assert_within(y, ref, absref, np.float64, f"{per_row} per row")


@pytest.mark.parametrize("lanes", [2, 4])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_plan_vector_kernel_row_lengths(J, O, lanes, dtype, monkeypatch):
    """The vector kernel forced to 2 / 4 lanes per row on rows of 0 .. 16*lanes
    entries: a lane's entries are loaded 4 at a time, so rows end inside, at
    and past those batches; empty rows give beta*y."""
    monkeypatch.setenv("JLUST_HIP_SPMV_VECTOR", str(lanes))
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "0")
    m, n = 20_000, 30_000
    lens = np.random.default_rng(lanes).integers(0, 16 * lanes + 1, m)
    lens[::97] = 0
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=lanes + 40, dtype=dtype)
    x = np.random.default_rng(3).uniform(-1, 1, n).astype(dtype)
    y0 = np.random.default_rng(4).uniform(-1, 1, m).astype(dtype)
    y, h, _ = run_plan(J, rowptr, colind, val, x, m, n, alpha=-1.25, beta=0.5, y0=y0)
    assert h.kernel() == "vector"
    ref = O.csr_spmv(rowptr, colind, val, x, -1.25, 0.5, y0)
    absref = O.csr_spmv_absref(rowptr, colind, val, x, -1.25, 0.5, y0)
    assert_within(y, ref, absref, dtype, f"vector kernel, {lanes} lanes")


@pytest.mark.parametrize("L", [1, 3, 16, 40])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_plan_vector_uniform_rows(J, O, L, dtype, monkeypatch):
    """Rows of exactly L entries: the vector kernel computes the row bounds
    (i*L) instead of loading rowptr, so it is also checked on a pattern whose
    entry count is a multiple of m but whose rows alternate L-1 and L+1 entries
    (the plan must see it is not uniform), and with origin 0."""
    monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", "0")
    monkeypatch.delenv("JLUST_HIP_SPMV_VECTOR", raising=False)
    m, n = 30_000, 50_000
    for lens, origin in ((np.full(m, L), 1), (np.full(m, L), 0),
                         (np.where(np.arange(m) % 2 == 0, L + 1, max(L - 1, 0)), 1)):
        if lens.sum() % m:
            continue
        rowptr, colind, val = random_csr(m, n, lengths=lens, seed=L + 60, origin=origin, dtype=dtype)
        x = np.random.default_rng(L).uniform(-1, 1, n).astype(dtype)
        y0 = np.random.default_rng(L + 1).uniform(-1, 1, m).astype(dtype)
        y, h, _ = run_plan(J, rowptr, colind, val, x, m, n, origin=origin, alpha=0.5, beta=2.0, y0=y0)
        assert h.kernel() == "vector"
        ref = O.csr_spmv(rowptr, colind, val, x, 0.5, 2.0, y0, origin=origin)
        absref = O.csr_spmv_absref(rowptr, colind, val, x, 0.5, 2.0, y0, origin=origin)
        assert_within(y, ref, absref, dtype, f"uniform rows L={L} origin={origin}")


@pytest.mark.parametrize("kind", ["csr", "plan", "coo", "csc", "bsr", "fn"])
def test_spmv_strided_vectors(J, O, kind):
    """x a row of a column-major matrix (stride = its leading dimension) and y
    every other entry of a longer vector, as the reference's ust takes any
    AbstractVector view (src/interop.jl:36-46): the result lands in y's
    entries and the entries between them stay untouched."""
    import torch
    m, n, ld = 700, 600, 5
    if kind == "bsr":
        m, n = 704, 608                        # 44 x 38 blocks of 16 x 16
    rowptr, colind, val = random_csr(m, n, lengths=np.random.default_rng(40).integers(0, 25, m),
                                     seed=41, dtype=np.float32 if kind == "bsr" else np.float64)
    dt = val.dtype
    rng = np.random.default_rng(42)
    xs = rng.uniform(-1, 1, n).astype(dt)
    y0 = rng.uniform(-1, 1, m).astype(dt)
    Xm = np.asfortranarray(np.full((ld, n), 9.0, dt))
    Xm[2] = xs
    Xd = dev(Xm)
    xv = Xd[2]                                 # stride ld
    ybig = dev(np.full(2 * m, 5.0, dt))
    yv = ybig[::2]
    yv.copy_(dev(y0))
    assert xv.stride(0) == ld and yv.stride(0) == 2
    alpha, beta = 1.5, -0.5
    if kind == "bsr":
        # A block pattern and its exact CSR expansion (the oracle's reference).
        mb, nb = m // 16, n // 16
        counts = rng.integers(0, 5, mb)
        bc = np.concatenate([np.sort(rng.choice(nb, c, replace=False)) for c in counts]) + 1
        bp = (np.r_[0, np.cumsum(counts)] + 1).astype(np.int32)
        bv = rng.uniform(-1, 1, bc.size * 256).astype(dt)
        rowptr, colind, val = O.bsr_to_csr(bp, bc.astype(np.int32), bv, 16)
        A = J.bsr_tensor(dev(bp), dev(bc.astype(np.int32)), dev(bv), (m, n))
    elif kind == "coo":
        rows = np.repeat(np.arange(1, m + 1, dtype=np.int32), np.diff(rowptr))
        A = J.coo_tensor(dev(rows), dev(colind), dev(val), (m, n))
    elif kind == "csc":
        cp, ri, cv = O.csr_to_csc(rowptr, colind, val, n)
        A = J.csc_tensor(dev(cp), dev(ri), dev(cv), (m, n))
    else:
        A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    ref = O.csr_spmv(rowptr, colind, val, xs, alpha, beta, y0)
    absref = O.csr_spmv_absref(rowptr, colind, val, xs, alpha, beta, y0)
    if kind == "plan":
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        J.execute(h, xv, yv, alpha=alpha, beta=beta)
    elif kind == "fn":
        # input_fn / output_fn through the same staging: identity-equivalent
        # transforms would not exercise the path, so scale x by 2 on input.
        J.execute(J.SpMVOp, A, xv, yv, alpha=alpha, beta=beta, input_fn=lambda v: 2 * v)
        ref = O.csr_spmv(rowptr, colind, val, 2 * xs, alpha, beta, y0)
        absref = O.csr_spmv_absref(rowptr, colind, val, 2 * xs, alpha, beta, y0)
    else:
        J.execute(J.SpMVOp, A, xv, yv, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    got = host(ybig)
    assert_within(got[::2], ref, absref, dt, f"strided vectors, {kind}")
    assert (got[1::2] == 5.0).all(), "entries between the strided y's entries were written"
    assert (host(Xd) == Xm).all()
