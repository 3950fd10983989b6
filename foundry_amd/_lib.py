"""ctypes binding of libfoundry_hip.so (include/foundry_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback for any op.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfoundry_hip.so")

# fh_status
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_DEVICE_UNAVAILABLE = 2
ERR_ALLOCATION = 3
ERR_FOREIGN_STORAGE = 4
ERR_OUT_OF_BOUNDS = 5
ERR_LAUNCH = 6
ERR_FAILED = 7
ERR_INDEX_TOO_LARGE = 8
ERR_DTYPE = 9
ERR_UNSUPPORTED = 10
ERR_CAPTURE = 11

STATUS_NAMES = {
    OK: "OK",
    ERR_INVALID_ARGUMENT: "InvalidArgument",
    ERR_DEVICE_UNAVAILABLE: "DeviceUnavailable",
    ERR_ALLOCATION: "BufferAllocation",
    ERR_FOREIGN_STORAGE: "ForeignStorage",
    ERR_OUT_OF_BOUNDS: "OutOfBounds",
    ERR_LAUNCH: "Launch",
    ERR_FAILED: "CommandBufferFailed",
    ERR_INDEX_TOO_LARGE: "KernelIndexTooLarge",
    ERR_DTYPE: "DType",
    ERR_UNSUPPORTED: "Unsupported",
    ERR_CAPTURE: "Capture",
}

# fh_dtype
F32 = 0
BF16 = 1
U32 = 2

# fh_profile_mode
PROFILE_OFF = 0
PROFILE_STEPS = 1
PROFILE_KERNELS = 2


class AllocatedMemory(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint64), ("source", ctypes.c_char_p)]


class Profile(ctypes.Structure):
    _fields_ = [
        ("dispatches", ctypes.c_uint64),
        ("allocations", ctypes.c_uint64),
        ("allocated_bytes", ctypes.c_uint64),
        ("gpu_busy_ns", ctypes.c_uint64),
    ]


class Q4Weight(ctypes.Structure):
    """fh_q4_weight."""
    _fields_ = [("wq", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("n", ctypes.c_int64), ("k", ctypes.c_int64), ("sb", ctypes.c_void_p), ("wt", ctypes.c_void_p)]


class LlamaLayer(ctypes.Structure):
    """fh_llama_layer."""
    _fields_ = [("qkv", Q4Weight), ("o", Q4Weight), ("gate_up", Q4Weight), ("down", Q4Weight),
                ("input_norm", ctypes.c_void_p), ("post_norm", ctypes.c_void_p),
                ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p)]


class LlamaModel(ctypes.Structure):
    """fh_llama_model."""
    _fields_ = [(name, ctypes.c_int64) for name in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
                                                    "ffn", "vocab", "batch", "max_len", "max_tokens")] + [
        ("rms_norm_eps", ctypes.c_float), ("scale", ctypes.c_float),
        ("layers", ctypes.POINTER(LlamaLayer)), ("embed", Q4Weight),
        ("final_norm", ctypes.c_void_p), ("cos_tab", ctypes.c_void_p), ("sin_tab", ctypes.c_void_p),
    ] + [(name, ctypes.c_void_p) for name in ("h", "h2", "x", "qkv", "q", "attn", "o", "gate_up", "act",
                                              "logits")] + [
        ("attn_workspace", ctypes.c_void_p), ("attn_workspace_bytes", ctypes.c_uint64),
        ("decode_workspace", ctypes.c_void_p), ("decode_workspace_bytes", ctypes.c_uint64),
    ]


class View(ctypes.Structure):
    """fh_view: a strided view (src/metal/args.rs:22-29), in elements."""
    _fields_ = [("offset", ctypes.c_int64), ("ndim", ctypes.c_int32), ("dims", ctypes.c_int64 * 4),
                ("strides", ctypes.c_int64 * 4)]

    @staticmethod
    def of(shape, strides, offset: int = 0) -> "View":
        v = View()
        v.offset, v.ndim = int(offset), len(shape)
        for d, (n, st) in enumerate(zip(shape, strides)):
            v.dims[d], v.strides[d] = int(n), int(st)
        return v


class HipError(RuntimeError):
    """An fh_status other than OK, with the library's message."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, f"status {status}")
        super().__init__(f"{self.kind}: {message}")


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> argument types; every function returns int (fh_status)
SIGNATURES = {
    "fh_abi_version": [],
    "fh_device_count": [ctypes.POINTER(_int)],
    "fh_device_create": [_int, ctypes.POINTER(_vp)],
    "fh_device_create_profiled": [_int, _int, ctypes.POINTER(_vp)],
    "fh_device_destroy": [_vp],
    "fh_device_name": [_vp, ctypes.c_char_p, _sz],
    "fh_synchronize": [_vp],
    "fh_device_stream": [_vp, ctypes.POINTER(_vp)],
    "fh_alloc": [_vp, _sz, _int, ctypes.POINTER(_vp)],
    "fh_free": [_vp, _vp],
    "fh_upload": [_vp, _vp, _vp, _sz],
    "fh_download": [_vp, _vp, _vp, _sz],
    "fh_max_memory_allocated": [_vp, ctypes.POINTER(AllocatedMemory)],
    "fh_reset_run_memory_peak": [_vp],
    "fh_run_memory_peak": [_vp, ctypes.POINTER(AllocatedMemory)],
    "fh_take_profile": [_vp, ctypes.POINTER(Profile)],
    "fh_capture_begin": [_vp],
    "fh_capture_end": [_vp, ctypes.POINTER(_vp)],
    "fh_graph_launch": [_vp, _vp],
    "fh_graph_destroy": [_vp],
    "fh_read_probe_blocks": [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)],
    "fh_read_probe": [_vp, _vp, ctypes.c_uint64, _vp],
    "fh_timer_begin": [_vp],
    "fh_timer_end": [_vp, ctypes.POINTER(ctypes.c_double)],
    "fh_q4_embed": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp],
    "fh_q4_matmul": [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _int],
    "fh_q4_dequant": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "fh_rms_norm": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp],
    "fh_rope_kv": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp],
    "fh_attention_workspace": [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_uint64)],
    "fh_attention": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _vp,
                     ctypes.c_uint64, _vp],
    "fh_decode_attention_workspace": [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_uint64)],
    "fh_decode_attention": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64,
                            ctypes.c_float, _vp, ctypes.c_uint64, _vp],
    "fh_decode_attention_noalloc": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64,
                                    ctypes.c_float, _vp],
    "fh_q4_matmul_rmsnorm": [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
                             _vp, _int],
    "fh_q4_gate_up_silu": [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp],
    "fh_q4_interleave": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "fh_q4_tile": [_vp, _vp, _i64, _i64, _i64, _int, _vp],
    "fh_silu_mul": [_vp, _vp, _i64, _i64, _vp],
    "fh_argmax": [_vp, _vp, _i64, _i64, _vp],
    "fh_advance_positions": [_vp, _vp, _i64, _i64],
    "fh_append_token": [_vp, _vp, _i64, _vp, _vp, _i64, _i64],
    "fh_append_token_advance": [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64],
    "fh_llama_forward": [_vp, _vp, _i64, _vp, _vp, _vp],
    "fh_copy_strided": [_vp, _int, _vp, ctypes.POINTER(View), _vp],
    "fh_to_dtype": [_vp, _int, _vp, ctypes.POINTER(View), _int, _vp],
    "fh_unary": [_vp, _int, _int, _vp, ctypes.POINTER(View), _vp],
    "fh_binary": [_vp, _int, _int, _vp, ctypes.POINTER(View), _vp, ctypes.POINTER(View), _vp],
    "fh_reduce": [_vp, _int, _int, _vp, ctypes.POINTER(View), ctypes.c_int32, _vp],
    "fh_matmul": [_vp, _int, _vp, ctypes.POINTER(View), _vp, ctypes.POINTER(View), _vp],
    "fh_index_select": [_vp, _int, _vp, ctypes.POINTER(View), _vp, ctypes.POINTER(View), _vp],
    "fh_cat": [_vp, _int, ctypes.c_int32, _vp, ctypes.POINTER(View), _vp, ctypes.POINTER(View), _vp],
    "fh_slice_scatter": [_vp, _int, ctypes.c_int32, _i64, _vp, ctypes.POINTER(View), _vp, ctypes.POINTER(View)],
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads the library once; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m foundry_amd.build` "
            "(the q4 ops have no CPU fallback)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _int
    lib.fh_last_error.argtypes = []
    lib.fh_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().fh_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise HipError(status, last_error())


def attention_workspace_bytes(tokens: int, n_heads: int, n_kv: int, head_dim: int, max_len: int) -> int:
    out = ctypes.c_uint64()
    call("fh_attention_workspace", tokens, n_heads, n_kv, head_dim, max_len, ctypes.byref(out))
    return out.value


def decode_attention_workspace_bytes(batch: int, n_heads: int, n_kv: int, head_dim: int, max_len: int) -> int:
    out = ctypes.c_uint64()
    call("fh_decode_attention_workspace", batch, n_heads, n_kv, head_dim, max_len, ctypes.byref(out))
    return out.value


def call(name: str, *args) -> None:
    """Calls an fh_* function and raises HipError on a non-OK status."""
    check(getattr(load(), name)(*args))
