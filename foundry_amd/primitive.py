"""Op vocabulary and output rules for the q4 path.

Mirrors src/nn/primitive.rs (``Op``, ``output``, the shape rules at :146-289)
and src/nn/dtype.rs / shape.rs, extended with the two quantized ops the
reference lacks:

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
    """src/nn/primitive.rs:146-207 for the q4 ops: (output shape, dtype)."""
    inputs = [(DType(dt), check_shape(shape)) for dt, shape in inputs]
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
