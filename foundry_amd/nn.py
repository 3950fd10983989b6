"""q4 forms of the reference's weight-consuming modules (src/nn/linear.rs).

``Q4Linear.forward`` keeps Linear::forward's shape handling
(src/nn/linear.rs:22-35): flatten every leading dim into rows, multiply by
the transposed weight, restore ``[..., out_features]``.
``Q4Embedding.forward`` keeps Embedding::forward's (src/nn/linear.rs:53-69):
flatten the ids, select rows, reshape to ``[...ids.dims, hidden]``.
"""
from __future__ import annotations

from dataclasses import dataclass

from .device import HipDevice
from .primitive import DType, QuantizedIndexSelect, QuantizedMatmul, TensorError
from .tensor import Tensor


@dataclass
class Q4Weight:
    """A q4 weight triplet: wq U32 [N, K/8], scales/biases BF16 [N, K/group]."""

    wq: Tensor
    scales: Tensor
    biases: Tensor
    group: int = 64

    @property
    def out_features(self) -> int:
        return self.wq.shape[0]

    @property
    def in_features(self) -> int:
        return self.wq.shape[1] * 8


class Q4Linear:
    def __init__(self, weight: Q4Weight):
        self.weight = weight

    def forward(self, device: HipDevice, x: Tensor) -> Tensor:
        if len(x.shape) == 0:
            raise TensorError("DimOutOfRange", "x has no last dim")
        in_features = x.shape[-1]
        rows = 1
        for d in x.shape[:-1]:
            rows *= d
        out_shape = (*x.shape[:-1], self.weight.out_features)
        op = QuantizedMatmul(bits=4, group=self.weight.group)
        w = self.weight
        return x.reshape((rows, in_features)).apply(device, op, [w.wq, w.scales, w.biases]).reshape(out_shape)


class Q4Embedding:
    def __init__(self, weight: Q4Weight):
        self.weight = weight

    def forward(self, device: HipDevice, input_ids: Tensor) -> Tensor:
        if input_ids.dtype is not DType.U32:
            raise TensorError("IndicesNotU32", input_ids.dtype.name)
        numel = 1
        for d in input_ids.shape:
            numel *= d
        flat = input_ids.reshape((numel,))
        w = self.weight
        op = QuantizedIndexSelect(dim=0, bits=4, group=w.group)
        rows = w.wq.apply(device, op, [w.scales, w.biases, flat])
        return rows.reshape((*input_ids.shape, w.in_features))
