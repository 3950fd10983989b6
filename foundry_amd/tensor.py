"""Tensor: a strided view of HipStorage, mirroring src/nn/tensor.rs.

Views (``reshape``, ``permute``, ``narrow``, ``expand``) share storage; every
op validates with ``primitive.output`` and runs through ``Device::run`` into a
fresh contiguous tensor (``Tensor::apply``, src/nn/tensor.rs:362-372);
``slice_scatter`` writes in place through ``Device::run_in_place``.

bf16 data crosses the host boundary as uint16 bit patterns.
"""
from __future__ import annotations

import numpy as np

from .device import HipDevice, HipStorage, Layout, Operand
from .primitive import (Binary, BinaryOp, Cat, Copy, DType, IndexSelect, Matmul, Reduce, ReduceOp, SliceScatter,
                        TensorError, ToDtype, Unary, UnaryOp, broadcast, check_shape, output)

_NP = {DType.F32: np.float32, DType.BF16: np.uint16, DType.U32: np.uint32}


class Tensor:
    def __init__(self, storage: HipStorage, layout: Layout, dtype: DType):
        self.storage = storage
        self.layout = layout
        self.dtype = DType(dtype)
        storage.views += 1

    def __del__(self):
        st = getattr(self, "storage", None)
        if st is not None:
            st.views -= 1

    @property
    def shape(self) -> tuple:
        return self.layout.shape

    def _view(self, layout: Layout) -> "Tensor":
        return Tensor(self.storage, layout, self.dtype)

    # ---- construction and bytes ----
    @staticmethod
    def from_bytes(device: HipDevice, data: bytes, dtype: DType, shape) -> "Tensor":
        """src/nn/tensor.rs:60-81: byte length must match shape and dtype."""
        shape = check_shape(shape)
        numel = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if len(data) != numel * DType(dtype).itemsize:
            raise TensorError("ByteLengthMismatch", f"{len(data)} bytes for {shape} {DType(dtype).name}")
        return Tensor(device.storage_from_bytes(data), Layout.contiguous(shape), dtype)

    @staticmethod
    def from_numpy(device: HipDevice, array: np.ndarray, dtype: DType) -> "Tensor":
        arr = np.ascontiguousarray(array, dtype=_NP[DType(dtype)])
        return Tensor.from_bytes(device, arr.tobytes(), dtype, arr.shape)

    @staticmethod
    def scalar_f32(device: HipDevice, value: float) -> "Tensor":
        """src/nn/tensor.rs:83-93: an F32 tensor of shape [1]."""
        return Tensor.from_bytes(device, np.float32(value).tobytes(), DType.F32, (1,))

    @staticmethod
    def zeros(device: HipDevice, dtype: DType, shape) -> "Tensor":
        shape = check_shape(shape)
        n = Layout.contiguous(shape).numel
        return Tensor(device.zeros(n * DType(dtype).itemsize), Layout.contiguous(shape), dtype)

    def to_bytes(self, device: HipDevice) -> bytes:
        if not self.layout.is_contiguous():
            raise TensorError("ToBytesNonContiguous")
        return device.storage_to_bytes(self.operand())

    def to_numpy(self, device: HipDevice) -> np.ndarray:
        return np.frombuffer(self.to_bytes(device), dtype=_NP[self.dtype]).reshape(self.shape).copy()

    def operand(self) -> Operand:
        return Operand(self.storage, self.layout, self.dtype)

    # ---- views ----
    def reshape(self, shape) -> "Tensor":
        return self._view(self.layout.reshape(shape))

    def permute(self, dims) -> "Tensor":
        return self._view(self.layout.permute(dims))

    def narrow(self, dim: int, start: int, length: int) -> "Tensor":
        return self._view(self.layout.narrow(dim, start, length))

    def expand(self, shape) -> "Tensor":
        return self._view(self.layout.expand(shape))

    # ---- ops (src/nn/tensor.rs:155-330) ----
    def neg(self, device):
        return self.apply(device, Unary(UnaryOp.NEG), [])

    def exp(self, device):
        return self.apply(device, Unary(UnaryOp.EXP), [])

    def sqrt(self, device):
        return self.apply(device, Unary(UnaryOp.SQRT), [])

    def reciprocal(self, device):
        return self.apply(device, Unary(UnaryOp.RECIPROCAL), [])

    def _binary(self, device, op: BinaryOp, rhs: "Tensor") -> "Tensor":
        """Tensor::binary (src/nn/tensor.rs:332-344): both sides expanded to
        the broadcast shape first."""
        shape = broadcast(self.shape, rhs.shape)
        return self.expand(shape).apply(device, Binary(op), [rhs.expand(shape)])

    def add(self, device, rhs):
        return self._binary(device, BinaryOp.ADD, rhs)

    def sub(self, device, rhs):
        return self._binary(device, BinaryOp.SUB, rhs)

    def mul(self, device, rhs):
        return self._binary(device, BinaryOp.MUL, rhs)

    def div(self, device, rhs):
        return self._binary(device, BinaryOp.DIV, rhs)

    def sum_keepdim(self, device, dim: int):
        return self.apply(device, Reduce(ReduceOp.SUM, dim), [])

    def amax_keepdim(self, device, dim: int):
        return self.apply(device, Reduce(ReduceOp.AMAX, dim), [])

    def argmax_keepdim(self, device, dim: int):
        return self.apply(device, Reduce(ReduceOp.ARGMAX, dim), [])

    def matmul(self, device, rhs):
        return self.apply(device, Matmul(), [rhs])

    def contiguous(self, device):
        if self.layout.is_contiguous():
            return self._view(self.layout)
        return self.apply(device, Copy(), [])

    def to_dtype(self, device, dtype: DType):
        if DType(dtype) == self.dtype and self.dtype.is_float:
            return self._view(self.layout)
        return self.apply(device, ToDtype(DType(dtype)), [])

    def index_select(self, device, dim: int, indices: "Tensor"):
        return self.apply(device, IndexSelect(dim), [indices])

    @staticmethod
    def cat(device, tensors, dim: int) -> "Tensor":
        a, b = tensors
        return a.apply(device, Cat(dim), [b])

    def slice_scatter(self, device: HipDevice, src: "Tensor", dim: int, start: int) -> None:
        """src/nn/tensor.rs:297-330: validate, require a contiguous target
        that no other tensor shares, then Device::run_in_place."""
        op = SliceScatter(dim, start)
        output(op, [(self.dtype, self.shape), (src.dtype, src.shape)])
        if not self.layout.is_contiguous():
            raise TensorError("SliceScatterNonContiguous")
        if self.storage.views != 1:
            raise TensorError("SharedStorage")
        device.run_in_place(op, self.operand(), [src.operand()])

    def apply(self, device: HipDevice, op, inputs) -> "Tensor":
        """src/nn/tensor.rs:362-372: validate, then Device::run."""
        tensors = [self, *inputs]
        shape, dtype = output(op, [(t.dtype, t.shape) for t in tensors])
        storage = device.run(op, [t.operand() for t in tensors], shape, dtype)
        return Tensor(storage, Layout.contiguous(shape), dtype)
