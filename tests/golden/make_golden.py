"""Writes tests/golden/q4_small.npz from the CPU oracle.

    python tests/golden/make_golden.py

The fixture freezes the oracle's outputs on small seeded cases so that a later
change to the oracle (or to the generators) shows up as a diff, and so GPU
tests have expected values without re-running the oracle. It holds data only:
inputs and expected outputs.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

CASES = {
    # name: (weight seed, rows, k, x seed, m)
    "gemv": (11, 40, 128, 12, 3),
    "gemm": (21, 72, 256, 22, 20),
}
EMBED_IDS = np.array([3, 0, 39, 40, 1000, 7, 39], dtype=np.uint32)  # 40 and 1000 are out of range


def build() -> dict:
    out = {}
    for name, (wseed, rows, k, xseed, m) in CASES.items():
        wq, s, b = O.gen_q4(wseed, rows, k)
        x = O.gen_bf16_normal(xseed, (m, k))
        y32, y16 = O.q4_linear(x, wq, s, b)
        out[f"{name}_wq"] = wq
        out[f"{name}_s"] = s
        out[f"{name}_b"] = b
        out[f"{name}_x"] = x
        out[f"{name}_deq"] = O.q4_dequant_bf16(wq, s, b)
        out[f"{name}_y32"] = y32
        out[f"{name}_y16"] = y16
        out[f"{name}_y64"] = O.linear_f64(x, wq, s, b)
    out["embed_ids"] = EMBED_IDS
    out["embed_rows"] = O.q4_embed(out["gemv_wq"], out["gemv_s"], out["gemv_b"], EMBED_IDS)
    return out


def main() -> None:
    path = os.path.join(HERE, "q4_small.npz")
    np.savez_compressed(path, **build())
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
