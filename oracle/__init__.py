"""CPU oracle for the q4 weight path: TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
path (``foundry_amd``) never imports it and has no CPU fallback.

Two parts:
- ``liboracle.so`` (oracle.c): the reference's arithmetic restated in C.
  SplitMix64 (src/bench/rng.rs:13-43), bf16 codec
  (src/metal/kernels/common.metal:29-43), gather with zero rows for
  out-of-range ids (src/metal/kernels/index_select.metal:11-29), and the
  fp32 sequential-k matmul (src/metal/kernels/matmul.metal:29-65), composed
  with the q4 dequant w = s*q + b.
- ``linear_f64``: fp64 dequant-then-matmul, the tolerance oracle for the
  GEMV and GEMM.

Parity status per function (how each is pinned) is listed in the module
docstring of tests/test_oracle.py.
"""
from .oracle import *  # noqa: F401,F403
