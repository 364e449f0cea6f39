"""Seeded random sweep over every HIP operator path against the CPU oracle.

Each seed draws one sparsity structure and runs on it every path below:

- the shape: up to 4000 rows and columns, every tenth draw 20k-80k;
- the row-length law: uniform, power law, mostly empty, or one dense row;
- the index origin, the value type, alpha and beta.

The paths:

- CSR SpMV plain and as prepared plans of every layout (row order, XCD column
  slices, LDS bins, the plan's own choice);
- COO SpMV (storage order shuffled, some entries duplicated) plain and prepared;
- CSC SpMV;
- CSR SpMM plain and prepared, for a random column count; COO SpMM (shuffled,
  some entries duplicated) and CSC SpMM, plain and prepared;
- SDDMM over the CSR mask, a shuffled COO mask, a DCSR mask of the non-empty
  rows, a CSC mask, and the prepared plans, for a random inner dimension;
- BSR SpMM and SpMV for a random block shape, block order and value type
  (16 x 16 blocks in both precisions), with a block-row of nb blocks in every
  third draw (several SpMV segments).

Every output is compared with the oracle (oracle/jlust_cpu.c) under the parity
bar: |got - ref| <= tol * (|alpha| |A| |x| + |beta| |y0|), tol 1e-12 (f64) and
1e-5 (f32), with the bound computed here in float64 from the same operands.
beta = 0 outputs start as NaN, so a path that reads them fails."""
import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr

pytestmark = pytest.mark.gpu

SEEDS = list(range(40))


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


def _say(seed, what):
    print(f"sweep seed {seed}: {what}", flush=True)


def _lengths(rng, m, n):
    law = int(rng.integers(0, 4))
    if law == 0:
        lens = rng.integers(0, min(n, 24) + 1, m)
    elif law == 1:
        lens = np.minimum((rng.pareto(1.5, m) + 1) * rng.integers(1, 6), n).astype(np.int64)
    elif law == 2:
        lens = np.where(rng.random(m) < 0.8, 0, rng.integers(1, min(n, 40) + 1, m))
    else:
        lens = rng.integers(0, min(n, 6) + 1, m)
        lens[int(rng.integers(0, m))] = n
    return np.asarray(lens, np.int64), law


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    top = 80000 if seed % 10 == 9 else 4000          # every tenth draw: many tiles and blocks
    m = int(np.exp(rng.uniform(0 if top == 4000 else np.log(20000), np.log(top))))
    n = int(np.exp(rng.uniform(0 if top == 4000 else np.log(20000), np.log(top))))
    lens, law = _lengths(rng, m, n)
    origin = int(rng.integers(0, 2))
    dtype = np.float64 if rng.random() < 0.5 else np.float32
    alpha = float(rng.choice([1.0, -0.75, 2.5]))
    beta = float(rng.choice([0.0, 0.0, 0.5, -1.25]))
    rowptr, colind, val = random_csr(m, n, lengths=lens, seed=seed, origin=origin, dtype=dtype)
    return rng, m, n, law, origin, dtype, alpha, beta, rowptr, colind, val


def _org(J, origin):
    return J.OneBased() if origin == 1 else J.ZeroBased()


def _spmv_absref(rows0, cols0, val, x, m, alpha, beta, y0):
    """|alpha| sum |v| |x[col]| per row (+ |beta| |y0|), rows0/cols0 0-based."""
    a = np.zeros(m, np.float64)
    np.add.at(a, rows0, np.abs(val.astype(np.float64)) * np.abs(x.astype(np.float64)[cols0]))
    a *= abs(alpha)
    if beta != 0.0:
        a += abs(beta) * np.abs(y0.astype(np.float64))
    return a


def _y(m, dtype, beta, y0):
    import torch
    if beta == 0.0:
        return torch.full((m,), float("nan"), dtype=torch.float64 if dtype == np.float64 else torch.float32,
                          device="cuda")
    return dev(y0)


@pytest.mark.parametrize("seed", SEEDS)
def test_sweep_spmv(J, O, seed, monkeypatch):
    rng, m, n, law, origin, dtype, alpha, beta, rowptr, colind, val = _draw(seed)
    x = rng.uniform(-1, 1, n).astype(dtype)
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    rows0 = np.repeat(np.arange(m), np.diff(rowptr))
    cols0 = colind.astype(np.int64) - origin
    ref = O.csr_spmv(rowptr, colind, val, x, alpha, beta, y0 if beta else None, origin=origin)
    absref = _spmv_absref(rows0, cols0, val, x, m, alpha, beta, y0)
    what = f"m={m} n={n} nnz={val.size} law={law} origin={origin} {np.dtype(dtype).name} a={alpha} b={beta}"

    _say(seed, f"CSR SpMV plain {what}")
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n), origin=_org(J, origin))
    y = _y(m, dtype, beta, y0)
    J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
    assert_within(host(y), ref, absref, dtype, f"seed {seed} CSR SpMV plain {what}")

    for layout in (None, "0", "1", "2"):
        if layout is None:
            monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)
        else:
            monkeypatch.setenv("JLUST_HIP_SPMV_SLICE", layout)
        _say(seed, f"CSR SpMV plan layout={layout} {what}")
        h = J.prepare(J.HIPBackend(), J.SpMVOp, A)
        y = _y(m, dtype, beta, y0)
        J.execute(h, dev(x), y, alpha=alpha, beta=beta)
        assert_within(host(y), ref, absref, dtype,
                      f"seed {seed} CSR SpMV plan layout={layout} ({h.kernel()}) {what}")
    monkeypatch.delenv("JLUST_HIP_SPMV_SLICE", raising=False)

    # COO: storage order shuffled, a few entries stored twice.
    dup = rng.random(val.size) < 0.05
    r = np.concatenate([rows0, rows0[dup]])
    c = np.concatenate([cols0, cols0[dup]])
    v = np.concatenate([val, val[dup] * dtype(0.5)]).astype(dtype)
    perm = rng.permutation(v.size)
    r, c, v = r[perm], c[perm], v[perm]
    rows_o = (r + origin).astype(np.int32)
    cols_o = (c + origin).astype(np.int32)
    cref = O.coo_spmv(rows_o, cols_o, v, x, m, alpha, beta, y0 if beta else None, origin=origin)
    cabs = _spmv_absref(r, c, v, x, m, alpha, beta, y0)
    _say(seed, f"COO SpMV plain nnz={v.size} {what}")
    Ac = J.coo_tensor(dev(rows_o), dev(cols_o), dev(v), (m, n), origin=_org(J, origin))
    y = _y(m, dtype, beta, y0)
    J.execute(J.SpMVOp, Ac, dev(x), y, alpha=alpha, beta=beta)
    assert_within(host(y), cref, cabs, dtype, f"seed {seed} COO SpMV plain {what}")
    _say(seed, f"COO SpMV plan {what}")
    hc = J.prepare(J.HIPBackend(), J.SpMVOp, Ac)
    y = _y(m, dtype, beta, y0)
    J.execute(hc, dev(x), y, alpha=alpha, beta=beta)
    assert_within(host(y), cref, cabs, dtype, f"seed {seed} COO SpMV plan {what}")

    # CSC (scatter with atomics).
    colptr, rowind, cval = O.csr_to_csc(rowptr, colind, val, n, origin=origin)
    sref = O.csc_spmv(colptr, rowind, cval, x, m, alpha, beta, y0 if beta else None, origin=origin)
    _say(seed, f"CSC SpMV {what}")
    As = J.csc_tensor(dev(colptr), dev(rowind), dev(cval), (m, n), origin=_org(J, origin))
    y = _y(m, dtype, beta, y0)
    J.execute(J.SpMVOp, As, dev(x), y, alpha=alpha, beta=beta)
    assert_within(host(y), sref, absref, dtype, f"seed {seed} CSC SpMV {what}")


@pytest.mark.parametrize("seed", SEEDS)
def test_sweep_spmm(J, O, seed):
    rng, m, n, law, origin, dtype, alpha, beta, rowptr, colind, val = _draw(seed)
    k = int(rng.integers(1, 71))
    B = np.asfortranarray(rng.uniform(-1, 1, (n, k)).astype(dtype))
    C0 = np.asfortranarray(rng.uniform(-1, 1, (m, k)).astype(dtype))
    c0 = C0 if beta else np.zeros((m, k), dtype, order="F")
    ref, _ = O.csr_spmm(rowptr, colind, val, B, alpha, beta, c0, origin=origin)
    absref = O.csr_spmm_absref(rowptr, colind, val, B, alpha, beta, c0, origin=origin)
    what = f"m={m} n={n} k={k} nnz={val.size} law={law} origin={origin} {np.dtype(dtype).name} a={alpha} b={beta}"
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n), origin=_org(J, origin))
    tdt = A.dtype

    def out():
        return dev(C0) if beta else J.dense_matrix(m, k, dtype=tdt, fill=float("nan"))

    _say(seed, f"CSR SpMM plain {what}")
    C = out()
    J.execute(J.SpMMOp, A, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), ref, absref, dtype, f"seed {seed} CSR SpMM plain {what}")
    _say(seed, f"CSR SpMM plan {what}")
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    C = out()
    J.execute(h, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), ref, absref, dtype, f"seed {seed} CSR SpMM plan {what}")

    # COO: storage order shuffled, a few entries stored twice (their scale in
    # the bound counts each stored copy).
    rows0 = np.repeat(np.arange(m), np.diff(rowptr))
    cols0 = colind.astype(np.int64) - origin
    dup = rng.random(val.size) < 0.05
    r = np.concatenate([rows0, rows0[dup]])
    c = np.concatenate([cols0, cols0[dup]])
    v = np.concatenate([val, val[dup] * dtype(0.5)]).astype(dtype)
    perm = rng.permutation(v.size)
    r, c, v = r[perm], c[perm], v[perm]
    rows_o, cols_o = (r + origin).astype(np.int32), (c + origin).astype(np.int32)
    cref = O.coo_spmm(rows_o, cols_o, v, B, m, alpha, beta, c0, origin=origin)
    crp = np.r_[0, np.cumsum(np.bincount(r, minlength=m))].astype(np.int64)
    order = np.argsort(r, kind="stable")
    cabs = O.csr_spmm_absref((crp + origin).astype(np.int32), cols_o[order], v[order], B, alpha, beta, c0,
                             origin=origin)
    Ac = J.coo_tensor(dev(rows_o), dev(cols_o), dev(v), (m, n), origin=_org(J, origin))
    _say(seed, f"COO SpMM plain nnz={v.size} {what}")
    C = out()
    J.execute(J.SpMMOp, Ac, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), cref, cabs, dtype, f"seed {seed} COO SpMM plain {what}")
    _say(seed, f"COO SpMM plan {what}")
    hc = J.prepare(J.HIPBackend(), J.SpMMOp, Ac, n_cols=k)
    C = out()
    J.execute(hc, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), cref, cabs, dtype, f"seed {seed} COO SpMM plan {what}")

    colptr, rowind, cval = O.csr_to_csc(rowptr, colind, val, n, origin=origin)
    sref = O.csc_spmm(colptr, rowind, cval, B, m, alpha, beta, c0, origin=origin)
    As = J.csc_tensor(dev(colptr), dev(rowind), dev(cval), (m, n), origin=_org(J, origin))
    _say(seed, f"CSC SpMM plain {what}")
    C = out()
    J.execute(J.SpMMOp, As, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), sref, absref, dtype, f"seed {seed} CSC SpMM plain {what}")
    _say(seed, f"CSC SpMM plan {what}")
    hs = J.prepare(J.HIPBackend(), J.SpMMOp, As, n_cols=k)
    C = out()
    J.execute(hs, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), sref, absref, dtype, f"seed {seed} CSC SpMM plan {what}")


@pytest.mark.parametrize("seed", SEEDS)
def test_sweep_sddmm(J, O, seed):
    rng, m, n, law, origin, dtype, alpha, beta, rowptr, colind, val = _draw(seed)
    K = int(rng.integers(1, 71))
    A = np.asfortranarray(rng.uniform(-1, 1, (m, K)).astype(dtype))
    Bm = np.asfortranarray(rng.uniform(-1, 1, (K, n)).astype(dtype))
    c0 = rng.uniform(-1, 1, val.size).astype(dtype)
    rows0 = np.repeat(np.arange(m), np.diff(rowptr))
    cols0 = colind.astype(np.int64) - origin
    what = f"m={m} n={n} K={K} nnz={val.size} law={law} origin={origin} {np.dtype(dtype).name} a={alpha} b={beta}"
    ref = O.csr_sddmm(rowptr, colind, A, Bm, alpha, beta, c0 if beta else None, origin=origin)
    absref = O.csr_sddmm_absref(rowptr, colind, A, Bm, alpha, beta, c0 if beta else None, origin=origin)

    def cvals(v0):
        import torch
        if beta:
            return dev(v0)
        return torch.full((v0.size,), float("nan"), dtype=torch.float64 if dtype == np.float64
                          else torch.float32, device="cuda")

    _say(seed, f"SDDMM CSR mask {what}")
    cv = cvals(c0)
    Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n), origin=_org(J, origin))
    J.execute(J.SDDMMOp, dev(A), dev(Bm), Cs, alpha=alpha, beta=beta)
    assert_within(host(cv), ref, absref, dtype, f"seed {seed} SDDMM CSR {what}")

    _say(seed, f"SDDMM plan {what}")
    cv = cvals(c0)
    Cs = J.csr_tensor(dev(rowptr), dev(colind), cv, (m, n), origin=_org(J, origin))
    h = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
    J.execute(J.SDDMMOp, h, dev(A), dev(Bm), Cs, alpha=alpha, beta=beta)
    assert_within(host(cv), ref, absref, dtype, f"seed {seed} SDDMM plan {what}")

    perm = rng.permutation(val.size)
    r_o = (rows0[perm] + origin).astype(np.int32)
    c_o = (cols0[perm] + origin).astype(np.int32)
    cref = O.coo_sddmm(r_o, c_o, A, Bm, alpha, beta, c0[perm] if beta else None, origin=origin)
    _say(seed, f"SDDMM COO mask (shuffled) {what}")
    cv = cvals(c0[perm])
    Cc = J.coo_tensor(dev(r_o), dev(c_o), cv, (m, n), origin=_org(J, origin))
    J.execute(J.SDDMMOp, dev(A), dev(Bm), Cc, alpha=alpha, beta=beta)
    assert_within(host(cv), cref, absref[perm], dtype, f"seed {seed} SDDMM COO {what}")

    # DCSR: the non-empty rows of the CSR mask, entries in the same order.
    keep = np.flatnonzero(np.diff(rowptr) > 0)
    outer = (keep + origin).astype(np.int32)
    dpos = (np.r_[0, np.cumsum(np.diff(rowptr)[keep])] + origin).astype(np.int32)
    dref = O.dcsr_sddmm(outer, dpos, colind, A, Bm, alpha, beta, c0 if beta else None, origin=origin)
    _say(seed, f"SDDMM DCSR mask {what}")
    cv = cvals(c0)
    Cd = J.dcsr_tensor(dev(outer), dev(dpos), dev(colind), cv, (m, n), origin=_org(J, origin))
    J.execute(J.SDDMMOp, dev(A), dev(Bm), Cd, alpha=alpha, beta=beta)
    assert_within(host(cv), dref, absref, dtype, f"seed {seed} SDDMM DCSR {what}")
    _say(seed, f"SDDMM DCSR plan {what}")
    cv = cvals(c0)
    Cd = J.dcsr_tensor(dev(outer), dev(dpos), dev(colind), cv, (m, n), origin=_org(J, origin))
    hd = J.prepare(J.HIPBackend(), J.SDDMMOp, Cd, n_inner=K)
    J.execute(hd, dev(A), dev(Bm), alpha=alpha, beta=beta)
    assert_within(host(cv), dref, absref, dtype, f"seed {seed} SDDMM DCSR plan {what}")

    # CSC: the mask's entries in column order.
    idx = np.arange(val.size, dtype=np.float64) + 1.0
    cp, ri, ci = O.csr_to_csc(rowptr, colind, idx, n, origin=origin)
    cperm = (ci - 1.0).astype(np.int64)
    sref = O.csc_sddmm(cp, ri, A, Bm, alpha, beta, c0[cperm] if beta else None, origin=origin)
    _say(seed, f"SDDMM CSC mask {what}")
    cv = cvals(c0[cperm])
    Cs = J.csc_tensor(dev(cp), dev(ri), cv, (m, n), origin=_org(J, origin))
    J.execute(J.SDDMMOp, dev(A), dev(Bm), Cs, alpha=alpha, beta=beta)
    assert_within(host(cv), sref, absref[cperm], dtype, f"seed {seed} SDDMM CSC {what}")
    _say(seed, f"SDDMM CSC plan {what}")
    cv = cvals(c0[cperm])
    Cs = J.csc_tensor(dev(cp), dev(ri), cv, (m, n), origin=_org(J, origin))
    hs = J.prepare(J.HIPBackend(), J.SDDMMOp, Cs, n_inner=K)
    J.execute(hs, dev(A), dev(Bm), alpha=alpha, beta=beta)
    assert_within(host(cv), sref, absref[cperm], dtype, f"seed {seed} SDDMM CSC plan {what}")


@pytest.mark.parametrize("seed", SEEDS)
def test_sweep_bsr(J, O, seed):
    rng = np.random.default_rng(5000 + seed)
    b1, b2 = [(16, 16), (16, 16), (1, 1), (2, 3), (4, 4), (3, 5), (8, 2), (1, 7)][seed % 8]
    if (b1, b2) == (16, 16):
        dtype = np.float64 if seed % 16 >= 8 else np.float32
    else:
        dtype = np.float32 if rng.random() < 0.5 else np.float64
    row_major = bool(rng.random() < 0.75)
    origin = int(rng.integers(0, 2))
    mb, nb = int(rng.integers(1, 60)), int(rng.integers(1, 60))
    counts = np.minimum(rng.integers(0, 12, mb), nb)
    if seed % 3 == 0:                                 # one block-row of nb blocks
        counts[int(rng.integers(0, mb))] = nb
    bcols = [np.sort(rng.choice(nb, int(cn), replace=False)) for cn in counts]
    browptr = (np.r_[0, np.cumsum(counts)] + origin).astype(np.int32)
    bcolind = ((np.concatenate(bcols) if counts.sum() else np.zeros(0, np.int64)) + origin).astype(np.int32)
    bval = rng.uniform(-1, 1, bcolind.size * b1 * b2).astype(dtype)
    k = int(rng.integers(1, 50))
    alpha = float(rng.choice([1.0, 0.5, -2.0]))
    beta = float(rng.choice([0.0, 1.5]))
    B = np.asfortranarray(rng.uniform(-1, 1, (nb * b2, k)).astype(dtype))
    C0 = np.asfortranarray(rng.uniform(-1, 1, (mb * b1, k)).astype(dtype))
    c0 = C0 if beta else np.zeros_like(C0)
    rp, ci, v = O.bsr_to_csr(browptr, bcolind, bval, b1, origin, row_major, b2)
    ref = O.bsr_spmm(browptr, bcolind, bval, b1, B, alpha, beta, c0, origin, row_major, b2=b2)
    absref = O.csr_spmm_absref(rp, ci, v, B, alpha, beta, c0, origin=origin)
    what = (f"mb={mb} nb={nb} block={b1}x{b2} nnzb={bcolind.size} k={k} origin={origin} "
            f"{'row' if row_major else 'col'}-major blocks {np.dtype(dtype).name} a={alpha} b={beta}")
    A = J.bsr_tensor(dev(browptr), dev(bcolind), dev(bval), (mb * b1, nb * b2), (b1, b2),
                     row_major_blocks=row_major, origin=_org(J, origin))
    tdt = A.dtype

    def out():
        return dev(C0) if beta else J.dense_matrix(mb * b1, k, dtype=tdt, fill=float("nan"))

    _say(seed, f"BSR SpMM plain {what}")
    C = out()
    J.execute(J.SpMMOp, A, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), ref, absref, dtype, f"seed {seed} BSR SpMM plain {what}")
    _say(seed, f"BSR SpMM plan {what}")
    h = J.prepare(J.HIPBackend(), J.SpMMOp, A, n_cols=k)
    C = out()
    J.execute(h, dev(B), C, alpha=alpha, beta=beta)
    assert_within(host(C), ref, absref, dtype, f"seed {seed} BSR SpMM plan {what}")

    x = rng.uniform(-1, 1, nb * b2).astype(dtype)
    y0 = rng.uniform(-1, 1, mb * b1).astype(dtype)
    yref = O.csr_spmv(rp, ci, v, x, alpha, beta, y0 if beta else None, origin=origin)
    rows0 = np.repeat(np.arange(mb * b1), np.diff(rp))
    yabs = _spmv_absref(rows0, ci.astype(np.int64) - origin, v, x, mb * b1, alpha, beta, y0)
    _say(seed, f"BSR SpMV {what}")
    y = _y(mb * b1, dtype, beta, y0)
    J.execute(J.SpMVOp, A, dev(x), y, alpha=alpha, beta=beta)
    assert_within(host(y), yref, yabs, dtype, f"seed {seed} BSR SpMV {what}")
