"""Seeded synthetic inputs for the q4 path (the task's config distributions).

SplitMix64 is the reference's generator (src/bench/rng.rs:13-25). Draw ``i``
of a stream seeded with ``seed`` has state ``seed + (i + 1) * gamma``, so a
whole stream is generated at once with numpy.

Derivations (the reference has no float sampler; these are this build's):
- uniform: ``u = (d >> 40) * 2^-24`` in [0, 1)
- normal: Box-Muller on two draws,
  ``sqrt(-2 ln u1) * cos(2 pi u2)``, ``u1 = ((d0 >> 40) + 1) * 2^-24``
- q4 weights from one stream: packed words first (each draw gives two
  words, low half first: 16 uniform nibbles), then one draw per scale,
  ``s = RNE_bf16(0.004 + 0.016 u)``, then two per bias,
  ``b = RNE_bf16(f32(-8 s + 1e-3 n))``
- bf16 activations ``x = RNE_bf16(f32(n))``, two draws per element
- token ids: ``below(vocab)`` per id, the reference's rejection sampler
  (src/bench/rng.rs:27-42), drawn in order as src/bench/mod.rs:203-241 does.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK64 = (1 << 64) - 1


def mix(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        z ^= z >> np.uint64(30)
        z *= _M1
        z ^= z >> np.uint64(27)
        z *= _M2
        z ^= z >> np.uint64(31)
    return z


def draws(seed: int, start: int, count: int) -> np.ndarray:
    """Draws start .. start+count-1 of the stream seeded with ``seed``."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        state = np.uint64(seed & _MASK64) + idx * GAMMA
    return mix(state)


def bf16_rne(values: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, nearest-even, NaN made quiet
    (src/metal/kernels/common.metal:37-43)."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _unit(d: np.ndarray) -> np.ndarray:
    return (d >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)


def _normal(d0: np.ndarray, d1: np.ndarray) -> np.ndarray:
    u1 = ((d0 >> np.uint64(40)) + np.uint64(1)).astype(np.float64) * (1.0 / 16777216.0)
    u2 = _unit(d1)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)


def q4_weights(seed: int, rows: int, k: int, group: int = 64, centre: float = 8.0):
    """Returns (wq u32[rows, k/8], scales bf16[rows, k/group], biases bf16[...]).
    ``centre`` 8 is the task's distribution (b = -8 s + N(0, 1e-3), so the
    weights have mean -s/2); 7.5 gives zero-mean weights."""
    words = rows * (k // 8)
    word_draws = (words + 1) // 2
    ngroups = rows * (k // group)
    d = draws(seed, 0, word_draws)
    wq = d.view(np.uint32)[:words].reshape(rows, k // 8).copy()  # little-endian: low half first
    s = bf16_rne((0.004 + 0.016 * _unit(draws(seed, word_draws, ngroups))).astype(np.float32))
    db = draws(seed, word_draws + ngroups, 2 * ngroups)
    z = _normal(db[0::2], db[1::2])
    bias = (-centre * bf16_to_f32(s).astype(np.float64) + 1e-3 * z).astype(np.float32)
    b = bf16_rne(bias)
    return wq, s.reshape(rows, k // group), b.reshape(rows, k // group)


def bf16_normal(seed: int, shape) -> np.ndarray:
    count = int(np.prod(shape, dtype=np.int64))
    d = draws(seed, 0, 2 * count)
    return bf16_rne(_normal(d[0::2], d[1::2]).astype(np.float32)).reshape(shape)


class SplitMix64:
    """Sequential form, for ``below`` (src/bench/rng.rs:8-43)."""

    def __init__(self, seed: int):
        self.state = seed & _MASK64

    def next_u64(self) -> int:
        self.state = (self.state + int(GAMMA)) & _MASK64
        z = self.state
        z = ((z ^ (z >> 30)) * int(_M1)) & _MASK64
        z = ((z ^ (z >> 27)) * int(_M2)) & _MASK64
        return z ^ (z >> 31)

    def below(self, bound: int):
        if bound <= 0:
            return None
        rejected = ((_MASK64 % bound) + 1) % bound
        max_accepted = _MASK64 - rejected
        for _ in range(64):
            d = self.next_u64()
            if d <= max_accepted:
                return d % bound
        return None


def token_ids(seed: int, count: int, vocab: int) -> np.ndarray:
    rng = SplitMix64(seed)
    out = np.empty(count, dtype=np.uint32)
    for i in range(count):
        v = rng.below(vocab)
        if v is None:
            raise RuntimeError("token id draw failed")
        out[i] = v
    return out
