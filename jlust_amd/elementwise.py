"""input_fn / output_fn of SpMV (execute(::EmitterBackend, ::Op{:SpMV};
input_fn, output_fn), ext/KernelAbstractionsExt/ops/spmv.jl:371-374):

    y = alpha * output_fn(A * input_fn.(x)) + beta * y

The reference compiles the two Julia functions into its kernel.  Here a
transform is either

  * an ElementwiseFn (identity, affine a*v + b, abs, square, sqrt, exp, log,
    relu), applied on the device by jlust_hip_apply_fn_{f64,f32}; or
  * any Python callable, called once on the whole device vector (a torch
    tensor) and expected to return a tensor of the same shape and dtype, the
    counterpart of the reference's arbitrary `input_fn::IF`.

The SpMV itself always runs in the HIP kernels: in_fn.(x) is formed first,
the product is taken with alpha = 1, beta = 0 into a row-sum vector when an
output_fn is given, and the row write alpha*out_fn(t) + beta*y follows.  A
product scaled by 1 and a beta = 0 store are exact, so this equals the fused
form.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

FN_IDENTITY, FN_AFFINE, FN_ABS, FN_SQUARE, FN_SQRT, FN_EXP, FN_LOG, FN_RELU = range(8)
_NAMES = {FN_IDENTITY: "identity", FN_AFFINE: "affine", FN_ABS: "abs", FN_SQUARE: "square",
          FN_SQRT: "sqrt", FN_EXP: "exp", FN_LOG: "log", FN_RELU: "relu"}


@dataclass(frozen=True)
class ElementwiseFn:
    """f(v) of one jlust_fn_kind (include/jlust_hip.h)."""
    kind: int
    a: float = 1.0
    b: float = 0.0

    def __repr__(self):
        if self.kind == FN_AFFINE:
            return f"affine({self.a}*v + {self.b})"
        return _NAMES.get(self.kind, f"fn{self.kind}")

    def __call__(self, v: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(v)
        apply_fn(self, v, out)
        return out


identity_fn = ElementwiseFn(FN_IDENTITY)
abs_fn = ElementwiseFn(FN_ABS)
square_fn = ElementwiseFn(FN_SQUARE)
sqrt_fn = ElementwiseFn(FN_SQRT)
exp_fn = ElementwiseFn(FN_EXP)
log_fn = ElementwiseFn(FN_LOG)
relu_fn = ElementwiseFn(FN_RELU)


def affine_fn(a: float, b: float = 0.0) -> ElementwiseFn:
    """v -> a*v + b (products and sums not contracted into FMAs)."""
    return ElementwiseFn(FN_AFFINE, float(a), float(b))


def is_identity(fn) -> bool:
    return fn is None or (isinstance(fn, ElementwiseFn) and fn.kind == FN_IDENTITY)


def apply_fn(fn, src: torch.Tensor, dst: torch.Tensor, alpha=1.0, beta=0.0) -> torch.Tensor:
    """dst = alpha*fn(src) + beta*dst on the device (beta == 0: dst write-only)."""
    if src.device.type != "cuda" or dst.device != src.device or src.dtype != dst.dtype or \
            src.numel() != dst.numel() or not src.is_contiguous() or not dst.is_contiguous():
        raise ValueError("apply_fn: contiguous device vectors of one dtype and length")
    if isinstance(fn, ElementwiseFn) or fn is None:
        f = fn or identity_fn
        suf = {torch.float64: "f64", torch.float32: "f32"}.get(src.dtype)
        if suf is None:
            from .errors import UnsupportedValueType
            raise UnsupportedValueType(src.dtype, "HIPBackend")
        with _lib.on_device(src.device):
            st = getattr(_lib.lib(), f"jlust_hip_apply_fn_{suf}")(
                src.numel(), f.kind, f.a, f.b, src.data_ptr() if src.numel() else None,
                float(alpha), float(beta), dst.data_ptr() if dst.numel() else None,
                _lib.stream_handle(src.device))
        _lib.check(st, "apply_fn")
        return dst
    v = fn(src)                                   # user callable on the device vector
    if not isinstance(v, torch.Tensor) or v.shape != src.shape or v.dtype != src.dtype or \
            v.device != src.device:
        raise ValueError("input_fn/output_fn callables must map a device vector to one of the "
                         "same shape, dtype and device")
    return apply_fn(identity_fn, v.contiguous(), dst, alpha, beta)
