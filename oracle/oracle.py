"""ctypes wrapper over liboracle.so plus the fp64 tolerance oracle.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64

_lib = None


def lib() -> ctypes.CDLL:
    """Load liboracle.so, failing loudly if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle not built: {_LIB_PATH} missing (run `make -C oracle`)")
    L = ctypes.CDLL(_LIB_PATH)
    sig = {
        "or_splitmix_next": (ctypes.c_uint64, [_u64p]),
        "or_splitmix_below": (ctypes.c_int, [_u64p, ctypes.c_uint32, _u32p]),
        "or_splitmix_mix": (ctypes.c_uint64, [ctypes.c_uint64]),
        "or_splitmix_at": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
        "or_unit": (ctypes.c_double, [ctypes.c_uint64]),
        "or_normal": (ctypes.c_double, [ctypes.c_uint64, ctypes.c_uint64]),
        "or_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "or_bf16_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
        "or_q4_get": (ctypes.c_uint32, [_u32p, _i64, _i64, _i64]),
        "or_q4_pack": (None, [_u8p, _i64, _i64, _u32p]),
        "or_q4_unpack": (None, [_u32p, _i64, _i64, _u8p]),
        "or_q4_dequant_one": (ctypes.c_float, [ctypes.c_uint16, ctypes.c_uint32, ctypes.c_uint16]),
        "or_q4_dequant_bf16": (None, [_u32p, _u16p, _u16p, _i64, _i64, _i64, _u16p]),
        "or_q4_dequant_f32": (None, [_u32p, _u16p, _u16p, _i64, _i64, _i64, _f32p]),
        "or_q4_embed": (None, [_u32p, _u16p, _u16p, _i64, _i64, _i64, _u32p, _i64, _u16p]),
        "or_matmul_f32": (None, [_f32p, _i64, _i64, _i64, _f32p, _i64, _f32p]),
        "or_q4_linear": (None, [_u16p, _i64, _i64, _i64, _u32p, _u16p, _u16p, _i64, _i64,
                                 _f32p, _u16p, ctypes.c_int]),
        "or_gen_q4": (None, [ctypes.c_uint64, _i64, _i64, _i64, _u32p, _u16p, _u16p]),
        "or_gen_bf16_normal": (None, [ctypes.c_uint64, _i64, _u16p]),
        "or_gen_token_ids": (ctypes.c_int, [ctypes.c_uint64, _i64, ctypes.c_uint32, _u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray, ptype):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ptype)


class SplitMix64:
    """src/bench/rng.rs:8-43, through the C restatement."""

    def __init__(self, seed: int):
        self._state = ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        return lib().or_splitmix_next(ctypes.byref(self._state))

    def below(self, bound: int):
        out = ctypes.c_uint32(0)
        rc = lib().or_splitmix_below(ctypes.byref(self._state), bound, ctypes.byref(out))
        return None if rc != 0 else out.value


def splitmix_at(seed: int, index: int) -> int:
    return lib().or_splitmix_at(seed, index)


def bf16_from_f32(values) -> np.ndarray:
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32)).ravel()
    return np.array([lib().or_bf16_from_f32(float(x)) for x in v], dtype=np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def q4_pack(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows, k = q.shape
    out = np.empty((rows, k // 8), dtype=np.uint32)
    lib().or_q4_pack(_p(q, _u8p), rows, k, _p(out, _u32p))
    return out


def q4_unpack(wq: np.ndarray, k: int) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    rows = wq.shape[0]
    out = np.empty((rows, k), dtype=np.uint8)
    lib().or_q4_unpack(_p(wq, _u32p), rows, k, _p(out, _u8p))
    return out


def q4_dequant_one(s: int, q: int, b: int) -> float:
    return lib().or_q4_dequant_one(s, q, b)


def q4_dequant_bf16(wq, s, b, group: int = 64) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    rows, k = wq.shape[0], wq.shape[1] * 8
    out = np.empty((rows, k), dtype=np.uint16)
    lib().or_q4_dequant_bf16(_p(wq, _u32p), _p(s, _u16p), _p(b, _u16p), rows, k, group, _p(out, _u16p))
    return out


def q4_dequant_f32(wq, s, b, group: int = 64) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    rows, k = wq.shape[0], wq.shape[1] * 8
    out = np.empty((rows, k), dtype=np.float32)
    lib().or_q4_dequant_f32(_p(wq, _u32p), _p(s, _u16p), _p(b, _u16p), rows, k, group, _p(out, _f32p))
    return out


def q4_embed(wq, s, b, ids, group: int = 64) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.uint32).ravel()
    rows, k = wq.shape[0], wq.shape[1] * 8
    out = np.empty((ids.size, k), dtype=np.uint16)
    lib().or_q4_embed(_p(wq, _u32p), _p(s, _u16p), _p(b, _u16p), rows, k, group,
                      _p(ids, _u32p), ids.size, _p(out, _u16p))
    return out


def matmul_f32(lhs: np.ndarray, rhs_t: np.ndarray) -> np.ndarray:
    lhs = np.ascontiguousarray(lhs, dtype=np.float32)
    rhs_t = np.ascontiguousarray(rhs_t, dtype=np.float32)
    m, k = lhs.shape
    n = rhs_t.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().or_matmul_f32(_p(lhs, _f32p), m, k, k, _p(rhs_t, _f32p), n, _p(out, _f32p))
    return out


def q4_linear(x_bf16, wq, s, b, group: int = 64, threads: int = 1):
    """Reference arithmetic: returns (y_f32, y_bf16)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = x.shape
    n = wq.shape[0]
    y32 = np.empty((m, n), dtype=np.float32)
    y16 = np.empty((m, n), dtype=np.uint16)
    lib().or_q4_linear(_p(x, _u16p), m, k, k, _p(wq, _u32p), _p(s, _u16p), _p(b, _u16p), n, group,
                       _p(y32, _f32p), _p(y16, _u16p), threads)
    return y32, y16


def linear_f64(x_bf16, wq, s, b, group: int = 64, rows=None) -> np.ndarray:
    """fp64 dequant-then-matmul: y[m, n] = sum_k x[m,k] * (s*q + b) in float64.

    ``rows`` optionally restricts the weight rows (output columns) computed.
    """
    x = bf16_to_f32(np.asarray(x_bf16, dtype=np.uint16)).astype(np.float64)
    wq = np.asarray(wq, dtype=np.uint32)
    s = np.asarray(s, dtype=np.uint16)
    b = np.asarray(b, dtype=np.uint16)
    if rows is not None:
        wq, s, b = wq[rows], s[rows], b[rows]
    n, kw = wq.shape
    k = kw * 8
    shifts = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    q = ((wq[:, :, None] >> shifts) & 0xF).reshape(n, k).astype(np.float64)
    sf = np.repeat(bf16_to_f32(s).astype(np.float64), group, axis=1)
    bf = np.repeat(bf16_to_f32(b).astype(np.float64), group, axis=1)
    w = sf * q + bf
    return x @ w.T


def gen_q4(seed: int, rows: int, k: int, group: int = 64):
    wq = np.empty((rows, k // 8), dtype=np.uint32)
    s = np.empty((rows, k // group), dtype=np.uint16)
    b = np.empty((rows, k // group), dtype=np.uint16)
    lib().or_gen_q4(seed, rows, k, group, _p(wq, _u32p), _p(s, _u16p), _p(b, _u16p))
    return wq, s, b


def gen_bf16_normal(seed: int, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().or_gen_bf16_normal(seed, out.size, _p(out, _u16p))
    return out


def gen_token_ids(seed: int, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    rc = lib().or_gen_token_ids(seed, count, vocab, _p(out, _u32p))
    if rc != 0:
        raise RuntimeError("token id draw failed")
    return out
