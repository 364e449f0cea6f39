"""SpMV's input_fn / output_fn on the GPU: the reference's known answers
(test/test_emitter_cuda.jl:188-258: [14, 12], [8, 7], [15, 13]) with named
Python functions as in the reference and with the device transforms, and
random CSR / COO / ShiftedDiag cases against numpy within the parity
tolerance."""
import numpy as np
import pytest

from tests._util import assert_within, dev, host, random_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def J():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import jlust_amd
    return jlust_amd


def _fuse_double(x):
    return 2.0 * x


def _fuse_addone(x):
    return x + 1.0


def fixture_A(J):
    return J.csr_tensor(dev(np.int32([1, 3, 4])), dev(np.int32([1, 3, 2])),
                        dev(np.float64([1.0, 2.0, 3.0])), (2, 3))


@pytest.mark.parametrize("kind", ["callable", "device"])
def test_reference_fused_cases(J, kind):
    import torch
    dbl = _fuse_double if kind == "callable" else J.affine_fn(2.0)
    add1 = _fuse_addone if kind == "callable" else J.affine_fn(1.0, 1.0)
    A = fixture_A(J)
    x = dev(np.float64([1.0, 2.0, 3.0]))
    y = torch.zeros(2, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, A, x, y, input_fn=dbl)
    assert host(y).tolist() == [14.0, 12.0]
    y.zero_()
    J.execute(J.SpMVOp, A, x, y, output_fn=add1)
    assert host(y).tolist() == [8.0, 7.0]
    h = J.prepare(J.HIPBackend(), J.SpMVOp, A, input_fn=dbl, output_fn=add1)
    y.zero_()
    J.execute(J.SpMVOp, h, A, x, y)
    assert host(y).tolist() == [15.0, 13.0]
    y.zero_()
    J.execute(J.SpMVOp, h, A, x, y)                  # second call: stable
    assert host(y).tolist() == [15.0, 13.0]
    y.zero_()
    J.execute(h, x, y)                               # cuSPARSE-style form
    assert host(y).tolist() == [15.0, 13.0]


FNS = {
    "identity": (lambda J: J.identity_fn, lambda v: v),
    "affine": (lambda J: J.affine_fn(-1.5, 0.25), lambda v: -1.5 * v + 0.25),
    "abs": (lambda J: J.abs_fn, np.abs),
    "square": (lambda J: J.square_fn, lambda v: v * v),
    "sqrt": (lambda J: J.sqrt_fn, lambda v: np.sqrt(np.abs(v))),
    "exp": (lambda J: J.exp_fn, np.exp),
    "log": (lambda J: J.log_fn, lambda v: np.log(np.abs(v))),
    "relu": (lambda J: J.relu_fn, lambda v: np.maximum(v, 0)),
}


@pytest.mark.parametrize("name", list(FNS))
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_input_fn_kinds(J, name, dtype):
    m, n = 300, 200
    rowptr, colind, val = random_csr(m, n, density=0.05, seed=3, dtype=dtype)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    rng = np.random.default_rng(4)
    xs = rng.uniform(-2, 2, n).astype(dtype)
    if name in ("sqrt", "log"):
        xs = np.abs(xs) + dtype(0.1)
    dfn, npfn = FNS[name]
    fx = npfn(xs.astype(np.float64))
    D = np.zeros((m, n))
    for r in range(m):
        D[r, colind[rowptr[r] - 1:rowptr[r + 1] - 1] - 1] = val[rowptr[r] - 1:rowptr[r + 1] - 1]
    y0 = rng.uniform(-1, 1, m).astype(dtype)
    y = dev(y0)
    J.execute(J.SpMVOp, A, dev(xs), y, alpha=2.0, beta=-0.5, input_fn=dfn(J))
    ref = 2.0 * (D @ fx) - 0.5 * y0
    bound = 2.0 * (np.abs(D) @ np.abs(fx)) + 0.5 * np.abs(y0)
    assert_within(host(y), ref, bound, dtype, f"input_fn {name}")


@pytest.mark.parametrize("name", ["affine", "abs", "square", "relu", "identity"])
def test_output_fn_kinds(J, name):
    m, n = 257, 190
    rowptr, colind, val = random_csr(m, n, density=0.04, seed=5)
    A = J.csr_tensor(dev(rowptr), dev(colind), dev(val), (m, n))
    rng = np.random.default_rng(6)
    xs = rng.uniform(-1, 1, n)
    D = np.zeros((m, n))
    for r in range(m):
        D[r, colind[rowptr[r] - 1:rowptr[r + 1] - 1] - 1] = val[rowptr[r] - 1:rowptr[r + 1] - 1]
    dfn, npfn = FNS[name]
    acc = D @ xs
    y0 = rng.uniform(-1, 1, m)
    for prepared in (False, True):
        y = dev(y0)
        if prepared:
            h = J.prepare(J.HIPBackend(), J.SpMVOp, A, output_fn=dfn(J))
            J.execute(h, dev(xs), y, alpha=1.5, beta=0.25)
        else:
            J.execute(J.SpMVOp, A, dev(xs), y, alpha=1.5, beta=0.25, output_fn=dfn(J))
        ref = 1.5 * npfn(acc) + 0.25 * y0
        lip = 2 * np.abs(acc) + 1 if name == "square" else 1.5     # |f'| on the error interval
        bound = 1.5 * lip * (np.abs(D) @ np.abs(xs)) + 0.25 * np.abs(y0) + np.abs(ref)
        assert_within(host(y), ref, bound, np.float64, f"output_fn {name} prepared={prepared}")


def test_coo_and_shifted_diag(J):
    import torch
    rows = np.int32([1, 1, 2, 3, 3])
    cols = np.int32([1, 3, 2, 1, 3])
    vals = np.float64([1.0, 2.0, 3.0, 4.0, 5.0])
    C = J.coo_tensor(dev(rows), dev(cols), dev(vals), (3, 3))
    x = dev(np.float64([1.0, 2.0, 3.0]))
    y = torch.zeros(3, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, C, x, y, input_fn=_fuse_double)
    assert host(y).tolist() == [14.0, 12.0, 38.0]
    with pytest.raises(J.UnsupportedFormat, match="output_fn"):
        J.execute(J.SpMVOp, C, x, y, output_fn=_fuse_addone)
    S = J.shifted_diag_tensor(torch.float64, 3, 4, shift=1, val=-2.0)
    y4 = torch.zeros(3, dtype=torch.float64, device="cuda")
    J.execute(J.SpMVOp, S, dev(np.float64([1.0, 2.0, 3.0, 4.0])), y4, input_fn=J.square_fn,
              output_fn=_fuse_addone)
    assert host(y4).tolist() == [-7.0, -17.0, -31.0]


def test_callable_must_keep_shape(J):
    A = fixture_A(J)
    import torch
    y = torch.zeros(2, dtype=torch.float64, device="cuda")
    with pytest.raises(ValueError):
        J.execute(J.SpMVOp, A, dev(np.float64([1.0, 2.0, 3.0])), y, input_fn=lambda v: v[:2])
