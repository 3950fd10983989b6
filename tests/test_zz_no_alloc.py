"""fh_decode_attention_noalloc against fh_decode_attention through the C-ABI:
the same kernels on the same inputs, so outputs and cache writes must be
bit-identical. Two calls in a row share the static workspace; the second is
smaller than the first (fewer sequences, heads and keys), so stale contents
of the first call must not leak into it. The entry point's defining
property is checked too: the device's byte counters and (on a profiled
device) its allocation counter do not move across a call, and the call
gives the same bytes when profiled per kernel and when captured into a
graph that is replayed several times."""
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


class _Step:
    """One decode step's inputs on a device, with fresh cache copies per run."""

    def __init__(self, dev, seed, batch, n_heads, n_kv, head_dim, max_len):
        self.dev, self.shape = dev, (batch, n_heads, n_kv, head_dim, max_len)
        cfg = LlamaConfig(1, n_heads * head_dim, n_heads, n_kv, head_dim, 64, 64)
        width = (n_heads + 2 * n_kv) * head_dim
        self.cache_elems = batch * n_kv * max_len * head_dim
        self.out_elems = batch * n_heads * head_dim
        self.k0 = synth.bf16_normal(seed + 1, (self.cache_elems,))
        self.v0 = synth.bf16_normal(seed + 2, (self.cache_elems,))
        pos = (max_len - 1 - np.arange(batch) * 37 % (max_len // 2)).astype(np.uint32)
        cos, sin = rope_tables(cfg, max_len)
        self.inputs = [_up(dev, synth.bf16_normal(seed, (batch, width))), _up(dev, cos), _up(dev, sin),
                       _up(dev, pos)]
        self.scale = ctypes.c_float(float(np.float32(1.0) / np.sqrt(np.float32(head_dim))))

    def buffers(self):
        kc, vc = _up(self.dev, self.k0), _up(self.dev, self.v0)
        out = _up(self.dev, np.full(self.out_elems, 0x7FC1, np.uint16))  # a sentinel the call must overwrite
        return kc, vc, out

    def call(self, noalloc, kc, vc, out, ws=None):
        batch, n_heads, n_kv, head_dim, max_len = self.shape
        s_qkv, s_cos, s_sin, s_pos = self.inputs
        common = (self.dev.handle, ctypes.c_void_p(s_qkv.ptr), batch, n_heads, n_kv, head_dim,
                  ctypes.c_void_p(s_cos.ptr), ctypes.c_void_p(s_sin.ptr), max_len, ctypes.c_void_p(s_pos.ptr),
                  ctypes.c_void_p(kc.ptr), ctypes.c_void_p(vc.ptr), max_len, self.scale)
        if noalloc:
            _lib.call("fh_decode_attention_noalloc", *common, ctypes.c_void_p(out.ptr))
        else:
            ws_bytes = _lib.decode_attention_workspace_bytes(*self.shape)
            _lib.call("fh_decode_attention", *common, ctypes.c_void_p(ws.ptr), ws_bytes, ctypes.c_void_p(out.ptr))

    def read(self, kc, vc, out):
        return (_down(self.dev, out, np.uint16, self.out_elems), _down(self.dev, kc, np.uint16, self.cache_elems),
                _down(self.dev, vc, np.uint16, self.cache_elems))

    def run(self, noalloc):
        kc, vc, out = self.buffers()
        ws = None if noalloc else self.dev.empty(_lib.decode_attention_workspace_bytes(*self.shape))
        self.dev.synchronize()
        before = (self.dev.max_memory_allocated()["bytes"], self.dev.run_memory_peak()["bytes"])
        self.dev.take_profile()
        self.call(noalloc, kc, vc, out, ws)
        self.dev.synchronize()
        prof = self.dev.take_profile()
        after = (self.dev.max_memory_allocated()["bytes"], self.dev.run_memory_peak()["bytes"])
        if noalloc:
            assert after == before, f"byte counters moved across the no-alloc call: {before} -> {after}"
            assert prof is None or prof["allocations"] == 0, prof
        return self.read(kc, vc, out)


SHAPES = ((1, (8, 32, 8, 128, 4096)), (2, (2, 24, 8, 128, 2048)))


def _equal(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


def test_decode_attention_noalloc_equals_the_workspace_entry_point():
    dev = HipDevice(0)
    try:
        # config 5's decode shape (chunked P.V, then the combine), then a smaller one
        for seed, shape in SHAPES:
            print(f"[no-alloc] decode attention batch/heads/kv/head_dim/max_len {shape}", flush=True)
            assert _lib.decode_attention_workspace_bytes(*shape) <= 32 << 20
            step = _Step(dev, seed * 10, *shape)
            want, got = step.run(False), step.run(True)
            assert _equal(want, got), shape
            assert np.any(want[0] != 0)
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


def test_decode_attention_noalloc_profiled_and_captured():
    """On a device profiled per kernel, and inside a captured graph replayed
    three times with eager work between the replays, the no-alloc call gives
    the eager workspace entry point's bytes."""
    dev = HipDevice.profiled(_lib.PROFILE_KERNELS)
    try:
        for seed, shape in SHAPES:
            print(f"[no-alloc] profiled + captured, shape {shape}", flush=True)
            step = _Step(dev, seed * 10 + 3, *shape)
            want = step.run(False)
            assert _equal(want, step.run(True)), shape
            kc, vc, out = step.buffers()
            dev.capture_begin()
            step.call(True, kc, vc, out)
            graph = dev.capture_end()
            for replay in range(3):
                # reset the outputs, then eager work of the same entry point between replays
                _lib.call("fh_upload", dev.handle, ctypes.c_void_p(out.ptr),
                          np.full(step.out_elems, 0x7FC1, np.uint16).ctypes.data_as(ctypes.c_void_p),
                          step.out_elems * 2)
                graph.launch()
                assert _equal(want, step.read(kc, vc, out)), (shape, replay)
                k2, v2, o2 = step.buffers()
                step.call(True, k2, v2, o2)
                dev.synchronize()
            del graph
    finally:
        dev.close()
