"""Op vocabulary and output rules.

Mirrors src/nn/primitive.rs (``Op``, ``output``, the shape rules at :146-367)
and src/nn/dtype.rs / shape.rs: the reference's nine Ops (``Unary``,
``Binary``, ``Reduce``, ``Matmul``, ``Copy``, ``ToDtype``, ``IndexSelect``,
``Cat``, ``SliceScatter``), extended with the two quantized ops the reference
lacks:

- ``QuantizedMatmul(bits=4, group=64)``: inputs ``[x, wq, scales, biases]``,
  ``x`` float ``[rows, K]``, ``wq`` U32 ``[N, K/8]``, ``scales``/``biases``
  BF16 ``[N, K/group]`` -> ``[rows, N]`` in x's dtype. The q4 form of
  ``Op::Matmul`` with the transposed-weight right operand that
  ``Linear::forward`` builds (src/nn/linear.rs:22-35).
- ``QuantizedIndexSelect(dim=0, bits=4, group=64)``: inputs
  ``[wq, scales, biases, ids]``, ``ids`` U32 1-D ``[n]`` -> BF16
  ``[n, K]``. The q4 form of ``Op::IndexSelect`` (src/nn/primitive.rs:258-289).

Validation raises ``TensorError`` with the reference's variant names before
any device call, as ``Tensor::apply`` does (src/nn/tensor.rs:362-372).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

MAX_RANK = 4  # src/nn/shape.rs:11
MAX_NUMEL = 0x7FFF_FFFF  # src/nn/shape.rs:13


class DType(enum.IntEnum):
    """src/nn/dtype.rs:6-10; values match fh_dtype."""

    F32 = 0
    BF16 = 1
    U32 = 2

    @property
    def itemsize(self) -> int:
        return 2 if self is DType.BF16 else 4

    @property
    def is_float(self) -> bool:
        return self in (DType.F32, DType.BF16)


class TensorError(Exception):
    """Validation error; ``kind`` is the reference's TensorError variant."""

    def __init__(self, kind: str, message: str = ""):
        self.kind = kind
        super().__init__(f"{kind}: {message}" if message else kind)


def check_shape(dims) -> tuple[int, ...]:
    """src/nn/shape.rs: rank <= 4 and numel <= 2^31 - 1."""
    dims = tuple(int(d) for d in dims)
    if len(dims) > MAX_RANK:
        raise TensorError("RankTooLarge", f"{dims}")
    numel = 1
    for d in dims:
        if d < 0:
            raise TensorError("NumelOverflow", f"negative dim in {dims}")
        numel *= d
    if numel > MAX_NUMEL:
        raise TensorError("NumelOverflow", f"{dims} has {numel} elements")
    return dims


class UnaryOp(enum.IntEnum):
    """src/nn/primitive.rs:14-24; values match fh_unary_op."""

    NEG = 0
    EXP = 1
    SQRT = 2
    RECIPROCAL = 3


class BinaryOp(enum.IntEnum):
    """src/nn/primitive.rs:26-36; values match fh_binary_op."""

    ADD = 0
    SUB = 1
    MUL = 2
    DIV = 3


class ReduceOp(enum.IntEnum):
    """src/nn/primitive.rs:38-46; values match fh_reduce_op."""

    SUM = 0
    AMAX = 1
    ARGMAX = 2


@dataclass(frozen=True)
class Unary:
    op: UnaryOp
    name = "unary"


@dataclass(frozen=True)
class Binary:
    op: BinaryOp
    name = "binary"


@dataclass(frozen=True)
class Reduce:
    op: ReduceOp
    dim: int
    name = "reduce"


@dataclass(frozen=True)
class Matmul:
    name = "matmul"


@dataclass(frozen=True)
class Copy:
    name = "copy"


@dataclass(frozen=True)
class ToDtype:
    dtype: "DType"
    name = "to_dtype"


@dataclass(frozen=True)
class IndexSelect:
    dim: int
    name = "index_select"


@dataclass(frozen=True)
class Cat:
    dim: int
    name = "cat"


@dataclass(frozen=True)
class SliceScatter:
    dim: int
    start: int
    name = "slice_scatter"


def size(shape, dim: int) -> int:
    """Shape::size (src/nn/shape.rs:41-53)."""
    if not 0 <= dim < len(shape):
        raise TensorError("DimOutOfRange", f"dim {dim} of {shape}")
    return shape[dim]


def with_dim(shape, dim: int, n: int) -> tuple[int, ...]:
    """Shape::with_dim (src/nn/shape.rs:96-108)."""
    size(shape, dim)
    return check_shape(shape[:dim] + (n,) + shape[dim + 1:])


def broadcast(lhs, rhs) -> tuple[int, ...]:
    """Shape::broadcast (src/nn/shape.rs:62-94): right-aligned; equal sizes
    or a size of one."""
    nd = max(len(lhs), len(rhs))
    out = []
    for i in range(1, nd + 1):
        a = lhs[-i] if i <= len(lhs) else 1
        b = rhs[-i] if i <= len(rhs) else 1
        if a == b or b == 1:
            out.append(a)
        elif a == 1:
            out.append(b)
        else:
            raise TensorError("BroadcastIncompatible", f"{lhs} and {rhs}")
    return check_shape(tuple(reversed(out)))


def _require_same_float(a: DType, b: DType) -> DType:
    if a != b:
        raise TensorError("DTypeMismatch", f"{DType(a).name} and {DType(b).name}")
    return _require_float(a)


def _dims_equal_except(a, b, dim: int) -> bool:
    return len(a) == len(b) and all(i == dim or x == y for i, (x, y) in enumerate(zip(a, b)))


def _output_standard(op, inputs):
    """src/nn/primitive.rs:146-207 for the reference's own Ops."""
    def arity(n):
        if len(inputs) != n:
            raise TensorError("OperandCount", f"{op.name} takes {n} operands, got {len(inputs)}")
    if isinstance(op, Unary):
        arity(1)
        return inputs[0][1], _require_float(inputs[0][0])
    if isinstance(op, Binary):
        arity(2)
        dtype = _require_same_float(inputs[0][0], inputs[1][0])
        return broadcast(inputs[0][1], inputs[1][1]), dtype
    if isinstance(op, Reduce):
        arity(1)
        dtype, shape = inputs[0]
        dtype = _require_float(dtype)
        n = size(shape, op.dim)
        if op.op in (ReduceOp.AMAX, ReduceOp.ARGMAX) and n == 0:
            raise TensorError("EmptyReduction", f"{ReduceOp(op.op).name} over dim {op.dim} of {shape}")
        return with_dim(shape, op.dim, 1), (DType.U32 if op.op == ReduceOp.ARGMAX else dtype)
    if isinstance(op, Matmul):
        arity(2)
        dtype = _require_same_float(inputs[0][0], inputs[1][0])
        lhs, rhs = inputs[0][1], inputs[1][1]
        if len(lhs) < 2 or len(rhs) < 2 or lhs[:-2] != rhs[:-2] or lhs[-1] != rhs[-2]:
            raise TensorError("MatmulIncompatible", f"{lhs} x {rhs}")
        return with_dim(lhs, len(lhs) - 1, rhs[-1]), dtype
    if isinstance(op, Copy):
        arity(1)
        return inputs[0][1], inputs[0][0]
    if isinstance(op, ToDtype):
        arity(1)
        _require_float(inputs[0][0])
        return inputs[0][1], _require_float(op.dtype)
    if isinstance(op, IndexSelect):
        arity(2)
        (t_dt, table), (i_dt, ids) = inputs
        dtype = _require_float(t_dt)
        if i_dt is not DType.U32:
            raise TensorError("IndicesNotU32", f"{DType(i_dt).name}")
        if op.dim != 0 or len(table) != 2 or len(ids) != 1:
            raise TensorError("IndexSelectIncompatible", f"dim {op.dim}, table {table}, indices {ids}")
        return check_shape((ids[0], table[1])), dtype
    if isinstance(op, Cat):
        arity(2)
        dtype = _require_same_float(inputs[0][0], inputs[1][0])
        lhs, rhs = inputs[0][1], inputs[1][1]
        a, b = size(lhs, op.dim), size(rhs, op.dim)
        if not _dims_equal_except(lhs, rhs, op.dim):
            raise TensorError("CatIncompatible", f"{lhs} and {rhs} along {op.dim}")
        return with_dim(lhs, op.dim, a + b), dtype
    if isinstance(op, SliceScatter):
        arity(2)
        dtype = _require_same_float(inputs[0][0], inputs[1][0])
        target, src = inputs[0][1], inputs[1][1]
        t, n = size(target, op.dim), size(src, op.dim)
        if op.start < 0 or op.start + n > t or not _dims_equal_except(target, src, op.dim):
            raise TensorError("SliceScatterOutOfBounds", f"{src} into {target} at {op.start} along {op.dim}")
        return target, dtype
    return None


@dataclass(frozen=True)
class QuantizedMatmul:
    bits: int = 4
    group: int = 64

    @property
    def name(self) -> str:
        return "q4matmul"


@dataclass(frozen=True)
class QuantizedIndexSelect:
    dim: int = 0
    bits: int = 4
    group: int = 64

    @property
    def name(self) -> str:
        return "q4index_select"


def _require_float(dtype: DType) -> DType:
    if not DType(dtype).is_float:
        raise TensorError("DTypeNotFloat", f"{DType(dtype).name}")
    return DType(dtype)


def _check_q4_weight(op, wq, scales, biases, incompatible: str) -> tuple[int, int]:
    """Returns (rows, K) of a q4 weight triplet or raises."""
    (wq_dt, wq_shape), (s_dt, s_shape), (b_dt, b_shape) = wq, scales, biases
    if op.bits != 4:
        raise TensorError(incompatible, f"{op.bits}-bit weights are not supported")
    if op.group <= 0 or op.group % 8 != 0:
        raise TensorError(incompatible, f"group {op.group} is not a positive multiple of 8")
    if DType(wq_dt) is not DType.U32:
        raise TensorError("DTypeMismatch", f"packed weights are {DType(wq_dt).name}, not U32")
    if DType(s_dt) is not DType.BF16 or DType(b_dt) is not DType.BF16:
        raise TensorError("DTypeMismatch", "scales and biases must be BF16")
    if len(wq_shape) != 2 or len(s_shape) != 2 or len(b_shape) != 2:
        raise TensorError(incompatible, "q4 weights, scales and biases are 2-D")
    rows, words = wq_shape
    k = words * 8
    if k % op.group != 0:
        raise TensorError(incompatible, f"K={k} is not a multiple of the group {op.group}")
    expect = (rows, k // op.group)
    if tuple(s_shape) != expect or tuple(b_shape) != expect:
        raise TensorError(incompatible, f"scales/biases {s_shape}/{b_shape}, expected {expect}")
    return rows, k


def output(op, inputs) -> tuple[tuple[int, ...], DType]:
    """src/nn/primitive.rs:146-207: (output shape, dtype) of any Op."""
    inputs = [(DType(dt), check_shape(shape)) for dt, shape in inputs]
    std = _output_standard(op, inputs)
    if std is not None:
        return std
    if isinstance(op, QuantizedMatmul):
        if len(inputs) != 4:
            raise TensorError("OperandCount", f"{op.name} takes 4 operands, got {len(inputs)}")
        (x_dt, x_shape), wq, s, b = inputs
        dtype = _require_float(x_dt)
        n, k = _check_q4_weight(op, wq, s, b, "MatmulIncompatible")
        if len(x_shape) != 2 or x_shape[1] != k:
            raise TensorError("MatmulIncompatible", f"x {x_shape} cannot multiply [{k}, {n}]")
        return check_shape((x_shape[0], n)), dtype
    if isinstance(op, QuantizedIndexSelect):
        if len(inputs) != 4:
            raise TensorError("OperandCount", f"{op.name} takes 4 operands, got {len(inputs)}")
        wq, s, b, (ids_dt, ids_shape) = inputs
        if ids_dt is not DType.U32:
            raise TensorError("IndicesNotU32", f"{ids_dt.name}")
        if op.dim != 0:
            raise TensorError("IndexSelectIncompatible", f"dim {op.dim}")
        _, k = _check_q4_weight(op, wq, s, b, "IndexSelectIncompatible")
        if len(ids_shape) != 1:
            raise TensorError("IndexSelectIncompatible", f"indices {ids_shape} are not 1-D")
        return check_shape((ids_shape[0], k)), DType.BF16
    raise TensorError("OperandCount", f"unknown op {op!r}")


def profile_key(op, rows: int, k: int, n: int) -> str:
    """Dispatch key in the style of MatmulGeometry::profile_key
    (src/metal/args.rs:196-204), e.g. ``q4matmul b1 m1 k3072 n8192 g64``."""
    if isinstance(op, QuantizedMatmul):
        return f"q4matmul b1 m{rows} k{k} n{n} g{op.group}"
    return f"q4index_select n{rows} k{k} g{op.group}"
