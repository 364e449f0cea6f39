"""Level formats of the JLUST tensor-format DSL, restricted to the formats on
the sparse hot path (src/formats.jl, src/named_formats.jl).

A format is an ordered tuple of levels, each mapping a level coordinate to an
expression of the dimension coordinates (i, j):

  CSR   (i : dense, j : compressed)                      named_formats.jl:25
  CSC   (j : dense, i : compressed)                      named_formats.jl:26
  COO   (i : compressed(nonunique), j : singleton)       named_formats.jl:24
  DCSR  (i : compressed, j : compressed)                 named_formats.jl:27
  BSRRight((b1,b2))  (i÷b1 : dense, j÷b2 : compressed, i%b1 : dense(b1),
                      j%b2 : dense(b2))                  named_formats.jl:106-116
  BSRLeft((b1,b2))   same with the two inner levels swapped, :118-128
  DensedRight(N)     N dense levels (plain column-major arrays), :219-227
  ShiftedDiag(T; shift, val)  (i : dense, j : shifted diagonal): row r holds
                     val at column r + shift, no buffers, :53-61
  PeriodicCSR(T, br, nc)  (i÷br : periodic, i%br : dense(br), j : compressed):
                     T copies of one br x nc CSR block on the diagonal, :77-88

Only the level *types* drive operator dispatch (dense outer + compressed
inner = CSR-shaped, compressed non-unique + singleton = COO-shaped, blocked =
BSR), exactly as in the reference's backends.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Tuple

from .errors import InvalidTensorFormat


@dataclass(frozen=True)
class DenseLevel:
    size: Optional[int] = None

    def __repr__(self):
        return "DenseLevel" if self.size is None else f"DenseLevel({self.size})"


@dataclass(frozen=True)
class CompressedLevel:
    unique: bool = True
    ordered: bool = True

    def __repr__(self):
        return "CompressedLevel" if self.unique else "CompressedLevel(nonunique)"


@dataclass(frozen=True)
class SingletonLevel:
    def __repr__(self):
        return "SingletonLevel"


@dataclass(frozen=True)
class ShiftedDiagLevel:
    """src/formats.jl:47-74: row r holds one entry at column r + shift with
    the constant value val; the level stores no buffers."""
    shift: int = 0
    val: float = 1.0

    def __repr__(self):
        return f"ShiftedDiagLevel(shift={self.shift}, val={self.val})"


@dataclass(frozen=True)
class PeriodicLevel:
    """src/formats.jl:87-107: the period index i ÷ block_rows of a T-fold
    block-diagonal replica; each period shifts columns by n_cols."""
    periods: int
    n_cols: int

    def __post_init__(self):
        if not (isinstance(self.periods, int) and self.periods > 0 and
                isinstance(self.n_cols, int) and self.n_cols > 0):
            raise InvalidTensorFormat(
                f"PeriodicLevel needs positive integers, got T={self.periods}, n_cols={self.n_cols}")

    def __repr__(self):
        return f"PeriodicLevel({self.periods}, {self.n_cols})"


@dataclass(frozen=True, eq=False)
class TensorFormat:
    """Levels plus the dim->level coordinate maps; equality is structural."""
    name: str
    levels: Tuple
    family: str
    ndims: int
    _d2l: Callable = None          # dims -> level coords
    _d2l_size: Callable = None     # dim extents -> level extents
    _l2d: Callable = None          # level coords -> dims

    def __eq__(self, other):
        return isinstance(other, TensorFormat) and self.name == other.name and \
            self.levels == other.levels

    def __hash__(self):
        return hash((self.name, self.levels))

    def __repr__(self):
        return self.name

    @property
    def is_dense(self) -> bool:
        return all(isinstance(lv, DenseLevel) for lv in self.levels)


def dim2lvl(fmt: TensorFormat, dim_indices, as_size: bool = False):
    """Level coordinates (or level extents when as_size) of dimension
    coordinates (src/formats.jl:429-431)."""
    if len(dim_indices) != fmt.ndims:
        raise InvalidTensorFormat(f"{fmt}: expected {fmt.ndims} coordinates")
    f = fmt._d2l_size if as_size else fmt._d2l
    return list(f(*dim_indices))


def lvl2dim(fmt: TensorFormat, lvl_indices):
    """Inverse of dim2lvl (src/formats.jl:433-440)."""
    if len(lvl_indices) != len(fmt.levels):
        raise InvalidTensorFormat(f"{fmt}: expected {len(fmt.levels)} level coordinates")
    return list(fmt._l2d(*lvl_indices))


def _ident2():
    return (lambda i, j: (i, j)), (lambda i, j: (i, j)), (lambda a, b: (a, b))


def _swap2():
    return (lambda i, j: (j, i)), (lambda i, j: (j, i)), (lambda a, b: (b, a))


def _make2(name, levels, family, maps):
    d2l, d2ls, l2d = maps
    return TensorFormat(name, tuple(levels), family, 2, d2l, d2ls, l2d)


_DENSE = {}


class Formats:
    """Named formats (src/named_formats.jl)."""

    CSR = _make2("CSR", [DenseLevel(), CompressedLevel()], "CSR", _ident2())
    CSC = _make2("CSC", [DenseLevel(), CompressedLevel()], "CSC", _swap2())
    COO = _make2("COO", [CompressedLevel(unique=False), SingletonLevel()], "COO", _ident2())
    DCSR = _make2("DCSR", [CompressedLevel(), CompressedLevel()], "DCSR", _ident2())

    @staticmethod
    def DensedRight(n: int) -> TensorFormat:
        """One shared (immutable) format object per n: every dense wrapper
        of an operand reuses it."""
        f = _DENSE.get(n)
        if f is None:
            if n < 1:
                raise InvalidTensorFormat("DensedRight needs at least one dimension")
            ident = lambda *c: tuple(c)  # noqa: E731
            f = _DENSE[n] = TensorFormat(f"DensedRight({n})", tuple(DenseLevel() for _ in range(n)),
                                         "Dense", n, ident, ident, ident)
        return f

    @staticmethod
    def ShiftedDiag(dtype=None, shift: int = 0, val=1.0) -> TensorFormat:
        """src/named_formats.jl:53-61; val is rounded to dtype (Float64 by default)."""
        import torch
        dtype = torch.float64 if dtype is None else dtype
        v = float(torch.tensor(float(val), dtype=dtype).item())
        return _make2(f"ShiftedDiag(shift={int(shift)},val={v})",
                      [DenseLevel(), ShiftedDiagLevel(int(shift), v)], "ShiftedDiag", _ident2())

    @staticmethod
    def PeriodicCSR(periods: int, block_rows: int, n_cols: int) -> TensorFormat:
        """src/named_formats.jl:77-88: (i ÷ block_rows : periodic, i % block_rows :
        dense(block_rows), j : compressed), T copies of one CSR block along the
        diagonal sharing its buffers."""
        br, nc = int(block_rows), int(n_cols)
        return TensorFormat(
            f"PeriodicCSR(T={int(periods)},br={br},nc={nc})",
            (PeriodicLevel(int(periods), nc), DenseLevel(br), CompressedLevel()), "PeriodicCSR", 2,
            (lambda i, j: (i // br, i % br, j)),
            (lambda m, n: (int(periods), br, n)),
            (lambda t, r, j: (t * br + r, j)))

    @staticmethod
    def BSRRight(blocksize) -> TensorFormat:
        b1, b2 = blocksize
        return _make2(
            f"BSRRight{b1}x{b2}",
            [DenseLevel(), CompressedLevel(), DenseLevel(b1), DenseLevel(b2)], "BSR",
            ((lambda i, j: (i // b1, j // b2, i % b1, j % b2)),
             (lambda m, n: (-(-m // b1), -(-n // b2), b1, b2)),
             (lambda bi, bj, ii, jj: (bi * b1 + ii, bj * b2 + jj))))

    @staticmethod
    def BSRLeft(blocksize) -> TensorFormat:
        b1, b2 = blocksize
        return _make2(
            f"BSRLeft{b1}x{b2}",
            [DenseLevel(), CompressedLevel(), DenseLevel(b2), DenseLevel(b1)], "BSR",
            ((lambda i, j: (i // b1, j // b2, j % b2, i % b1)),
             (lambda m, n: (-(-m // b1), -(-n // b2), b2, b1)),
             (lambda bi, bj, jj, ii: (bi * b1 + ii, bj * b2 + jj))))


def is_csr_shaped(fmt: TensorFormat) -> bool:
    """Dense outer over rows + unique compressed inner (spmv.jl:487-491)."""
    lv = fmt.levels
    return fmt.family == "CSR" and len(lv) == 2 and isinstance(lv[0], DenseLevel) and \
        isinstance(lv[1], CompressedLevel) and lv[1].unique


def is_csc_shaped(fmt: TensorFormat) -> bool:
    """Dense outer over columns + unique compressed inner over rows: the
    column-outer shape the reference walks in scatter mode (spmv.jl:104-112)."""
    lv = fmt.levels
    return fmt.family == "CSC" and len(lv) == 2 and isinstance(lv[0], DenseLevel) and \
        isinstance(lv[1], CompressedLevel) and lv[1].unique


def is_coo_shaped(fmt: TensorFormat) -> bool:
    """Non-unique compressed outer + singleton inner (spmv.jl:382-384)."""
    lv = fmt.levels
    return len(lv) >= 2 and isinstance(lv[0], CompressedLevel) and not lv[0].unique and \
        isinstance(lv[1], SingletonLevel)


def is_shifted_diag(fmt: TensorFormat) -> bool:
    """(Dense, ShiftedDiag): the shape the block compile recognises
    (ext/CUDAExt/ops/block_mul.jl:60-69)."""
    lv = fmt.levels
    return len(lv) == 2 and isinstance(lv[0], DenseLevel) and isinstance(lv[1], ShiftedDiagLevel)


def is_periodic_csr(fmt: TensorFormat) -> bool:
    return fmt.family == "PeriodicCSR"


def is_bsr(fmt: TensorFormat) -> bool:
    return fmt.family == "BSR"


def bsr_blocksize(fmt: TensorFormat):
    lv = fmt.levels
    if fmt.name.startswith("BSRRight"):
        return lv[2].size, lv[3].size, True
    return lv[3].size, lv[2].size, False
