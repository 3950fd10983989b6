"""fh_decode_attention_noalloc against fh_decode_attention through the C-ABI:
the same kernels on the same inputs, so outputs and cache writes must be
bit-identical. Two calls in a row share the static workspace; the second is
smaller than the first (fewer sequences, heads and keys), so stale contents
of the first call must not leak into it."""
import ctypes

import numpy as np
import pytest

from foundry_amd import _lib, synth
from foundry_amd.device import HipDevice
from foundry_amd.llama import LlamaConfig, rope_tables

pytestmark = pytest.mark.gpu


def _up(dev, arr):
    arr = np.ascontiguousarray(arr)
    return dev.storage_from_bytes(arr.tobytes())


def _down(dev, st, dtype, count):
    out = np.empty(count, dtype=dtype)
    _lib.call("fh_download", dev.handle, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(st.ptr), out.nbytes)
    return out


def _case(dev, seed, batch, n_heads, n_kv, head_dim, max_len):
    """Runs both entry points on identical copies of one decode step's inputs;
    returns (out, k, v) of each."""
    cfg = LlamaConfig(1, n_heads * head_dim, n_heads, n_kv, head_dim, 64, 64)
    width = (n_heads + 2 * n_kv) * head_dim
    qkv = synth.bf16_normal(seed, (batch, width))
    cache_elems = batch * n_kv * max_len * head_dim
    k0 = synth.bf16_normal(seed + 1, (cache_elems,))
    v0 = synth.bf16_normal(seed + 2, (cache_elems,))
    pos = (max_len - 1 - np.arange(batch) * 37 % (max_len // 2)).astype(np.uint32)
    cos, sin = rope_tables(cfg, max_len)
    s_qkv, s_cos, s_sin, s_pos = _up(dev, qkv), _up(dev, cos), _up(dev, sin), _up(dev, pos)
    scale = ctypes.c_float(float(np.float32(1.0) / np.sqrt(np.float32(head_dim))))
    results = []
    for noalloc in (False, True):
        kc, vc = _up(dev, k0), _up(dev, v0)
        out = dev.empty(batch * n_heads * head_dim * 2)
        common = (dev.handle, ctypes.c_void_p(s_qkv.ptr), batch, n_heads, n_kv, head_dim, ctypes.c_void_p(s_cos.ptr),
                  ctypes.c_void_p(s_sin.ptr), max_len, ctypes.c_void_p(s_pos.ptr), ctypes.c_void_p(kc.ptr),
                  ctypes.c_void_p(vc.ptr), max_len, scale)
        if noalloc:
            _lib.call("fh_decode_attention_noalloc", *common, ctypes.c_void_p(out.ptr))
        else:
            ws_bytes = _lib.decode_attention_workspace_bytes(batch, n_heads, n_kv, head_dim, max_len)
            ws = dev.empty(ws_bytes)
            _lib.call("fh_decode_attention", *common, ctypes.c_void_p(ws.ptr), ws_bytes, ctypes.c_void_p(out.ptr))
        results.append((_down(dev, out, np.uint16, batch * n_heads * head_dim),
                        _down(dev, kc, np.uint16, cache_elems), _down(dev, vc, np.uint16, cache_elems)))
    return results


def test_decode_attention_noalloc_equals_the_workspace_entry_point():
    dev = HipDevice(0)
    try:
        # config 5's decode shape (chunked P.V, then the combine), then a smaller one
        for seed, shape in ((1, (8, 32, 8, 128, 4096)), (2, (2, 24, 8, 128, 2048))):
            print(f"[no-alloc] decode attention batch/heads/kv/head_dim/max_len {shape}", flush=True)
            ws_bytes = _lib.decode_attention_workspace_bytes(*shape)
            assert ws_bytes <= 32 << 20
            (o1, k1, v1), (o2, k2, v2) = _case(dev, seed * 10, *shape)
            assert np.array_equal(o1, o2) and np.array_equal(k1, k2) and np.array_equal(v1, v2), shape
            assert np.any(o1 != 0)
        # a request larger than the static workspace is refused on the host
        big = (8, 64, 8, 128, 65536)
        assert _lib.decode_attention_workspace_bytes(*big) > 32 << 20
        buf = dev.empty(64)
        rc = _lib.load().fh_decode_attention_noalloc(dev.handle, ctypes.c_void_p(buf.ptr), 8, 64, 8, 128,
                                                     ctypes.c_void_p(buf.ptr), ctypes.c_void_p(buf.ptr), 65536,
                                                     ctypes.c_void_p(buf.ptr), ctypes.c_void_p(buf.ptr),
                                                     ctypes.c_void_p(buf.ptr), 65536, ctypes.c_float(0.1),
                                                     ctypes.c_void_p(buf.ptr))
        assert rc == _lib.ERR_UNSUPPORTED and "static one holds" in _lib.last_error()
    finally:
        dev.close()
