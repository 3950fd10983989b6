"""Tensor: a strided view of HipStorage, the subset of src/nn/tensor.rs the
q4 path uses (``from_bytes``, ``to_bytes``, ``reshape``, ``apply``).

bf16 data crosses the host boundary as uint16 bit patterns.
"""
from __future__ import annotations

import numpy as np

from .device import HipDevice, HipStorage, Layout, Operand
from .primitive import DType, TensorError, check_shape, output

_NP = {DType.F32: np.float32, DType.BF16: np.uint16, DType.U32: np.uint32}


class Tensor:
    def __init__(self, storage: HipStorage, layout: Layout, dtype: DType):
        self.storage = storage
        self.layout = layout
        self.dtype = DType(dtype)

    @property
    def shape(self) -> tuple:
        return self.layout.shape

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

    def to_bytes(self, device: HipDevice) -> bytes:
        return device.storage_to_bytes(self.operand())

    def to_numpy(self, device: HipDevice) -> np.ndarray:
        return np.frombuffer(self.to_bytes(device), dtype=_NP[self.dtype]).reshape(self.shape).copy()

    def operand(self) -> Operand:
        return Operand(self.storage, self.layout, self.dtype)

    def reshape(self, shape) -> "Tensor":
        """Contiguous-only reshape (TensorError::ReshapeNonContiguous otherwise)."""
        shape = check_shape(shape)
        if int(np.prod(shape, dtype=np.int64)) != self.layout.numel:
            raise TensorError("NumelMismatch", f"{self.shape} -> {shape}")
        if not self.layout.is_contiguous():
            raise TensorError("ReshapeNonContiguous")
        lay = Layout.contiguous(shape)
        return Tensor(self.storage, Layout(lay.shape, lay.strides, self.layout.offset), self.dtype)

    def apply(self, device: HipDevice, op, inputs) -> "Tensor":
        """src/nn/tensor.rs:362-372: validate, then Device::run."""
        tensors = [self, *inputs]
        shape, dtype = output(op, [(t.dtype, t.shape) for t in tensors])
        storage = device.run(op, [t.operand() for t in tensors], shape, dtype)
        return Tensor(storage, Layout.contiguous(shape), dtype)
