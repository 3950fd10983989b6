"""foundry_amd: MI355X (gfx950) backend for Foundry's 4-bit quantized weight path.

The compute lives in libfoundry_hip.so (hand-written HIP for gfx950) behind
the C-ABI in include/foundry_hip.h. This package is the host side above that
boundary: a ctypes binding (``_lib``), the reference's Device/Op interface for
the q4 ops (``device``, ``primitive``, ``tensor``), the q4 Linear/Embedding
modules (``nn``) and a seeded synthetic-input generator (``synth``).
"""
from .primitive import DType, QuantizedIndexSelect, QuantizedMatmul, TensorError  # noqa: F401

__all__ = ["DType", "QuantizedIndexSelect", "QuantizedMatmul", "TensorError"]
