"""Benchmark of the q4 weight path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--quick]

Headline (``value``): q4 decode GEMV HBM GB/s at the task's config 1,
x bf16[1,3072] . W q4[8192,3072]^T, over ``--copies`` distinct weight copies
(48 x 14.2 MB = 680 MB, larger than the 256 MB MALL), so every launch streams
its weights from HBM. One step = one pass over all copies (48 launches),
replayed as one HIP graph; event timing on the device's stream brackets the K
timed steps. Algorithmic bytes per launch: 12,582,912 (nibbles) + 1,572,864
(scales + biases) + 6,144 (x) + 16,384 (y) = 14,178,304.

Every graph is also replayed MEDIAN_REPLAYS more times, each replay timed
on its own with a pair of HIP events on the device's stream (the replays are
enqueued back to back), and the median replay is reported per launch
(``median_us_per_launch``).

Secondary lines (same method): the GEMV warm (one weight copy, which stays in
the eight 4 MB L2s);
the LM-head GEMV (N=128256, K=3072) cold (3 copies, 665 MB) and warm (one);
the q4 embedding gather at B = 4096, 64 and 1, cold (3 tables, distinct ids)
and warm (one table, the same ids); the two config-3 prefill GEMMs; the
launch and read floors (an almost empty kernel; fh_read_probe reading a
GEMV's bytes per launch, and 1 GiB); config 4 (Llama-3.2-3B shape: prefill
and greedy decode tok/s, with greedy agreement and first-step logits against
the CPU restatement, whose own tok/s is reported) and config 5 (8B shape,
batch 8 at context 4096, with batch-invariance and 2-layer restatement
logits checks).

cpu_baseline: the reference arithmetic (oracle/liboracle.so: fp32 dequant,
sequential-k fp32 accumulation, bf16 RNE) on the config-1 GEMV, on this
host's cores, for a bounded number of calls.

Single legs, for kernel traces and counters: --gemm-only, --floors-only,
--lm-head-only, --copy-sweep-only (the GEMV over 1 .. 48 weight copies),
--decode-only, --batched-only, and --eager-steps N (config 4, or config 5
with --batched-only: the decode steps launched op by op).
"""
from __future__ import annotations

import argparse
import gc
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from foundry_amd import _lib, synth  # noqa: E402
from foundry_amd.device import HipDevice  # noqa: E402

METRIC = "q4 GEMV HBM GB/s (% of peak); decode tok/s, Llama-3.2-3B-shape q4, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def embed_bytes(b: int, k: int) -> int:
    # per id: packed row, its scales and biases, the id, the bf16 row written
    return b * (k // 2 + 2 * 2 * (k // 64) + 4 + 2 * k)


class Weights:
    """Device copies of one q4 weight shape, each from its own seed."""

    def __init__(self, dev: HipDevice, n: int, k: int, copies: int, seed: int):
        self.n, self.k = n, k
        self.ptrs = []
        self._keep = []
        base = synth.q4_weights(seed, n, k)
        for c in range(copies):
            # distinct bytes per copy: xor the packed words with a per-copy pattern
            wq = base[0] ^ np.uint32((0x9E3779B9 * (c + 1)) & 0xFFFFFFFF) if c else base[0]
            arrs = (np.ascontiguousarray(wq), base[1], base[2])
            sts = [dev.storage_from_bytes(a.tobytes()) for a in arrs]
            self._keep.append(sts)
            self.ptrs.append(tuple(st.ptr for st in sts))


def q4_matmul(dev, x_ptr, m, k, w_ptrs, n, y_ptr, y_dtype=_lib.BF16):
    _lib.call("fh_q4_matmul", dev.handle, ctypes.c_void_p(x_ptr), m, k, k,
              ctypes.c_void_p(w_ptrs[0]), ctypes.c_void_p(w_ptrs[1]), ctypes.c_void_p(w_ptrs[2]),
              n, 64, ctypes.c_void_p(y_ptr), y_dtype)


class StreamEvents:
    """HIP event pairs recorded on the device's own stream around individual
    graph replays that are enqueued back to back (no host wait between them),
    so each span is one replay's GPU time."""

    def __init__(self, dev: HipDevice, pairs: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.stream = ctypes.c_void_p()
        _lib.call("fh_device_stream", dev.handle, ctypes.byref(self.stream))
        self.events = []
        for _ in range(2 * pairs):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.events.append(e)

    def record(self, i: int) -> None:
        if self.hip.hipEventRecord(self.events[i], self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def spans_ms(self, pairs: int) -> list:
        out = []
        for i in range(pairs):
            ms = ctypes.c_float()
            if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.events[2 * i], self.events[2 * i + 1]) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            out.append(ms.value)
        return out

    def close(self) -> None:
        for e in self.events:
            self.hip.hipEventDestroy(e)
        self.events = []


def median_replay_ms(dev: HipDevice, graph, replays: int) -> float:
    """Median GPU time of `replays` individually timed replays of a graph."""
    ev = StreamEvents(dev, replays)
    try:
        for i in range(replays):
            ev.record(2 * i)
            graph.launch()
            ev.record(2 * i + 1)
        dev.synchronize()
        spans = sorted(ev.spans_ms(replays))
    finally:
        ev.close()
    return spans[len(spans) // 2]


MEDIAN_REPLAYS = 60


def timed_graph(dev: HipDevice, enqueue, steps: int, warmup: int, median_replays: int = MEDIAN_REPLAYS):
    """Captures enqueue() as one graph. Returns (ms per replay over `steps`
    timed together, median ms of `median_replays` individually timed
    replays)."""
    dev.capture_begin()
    enqueue()
    graph = dev.capture_end()
    for _ in range(warmup):
        graph.launch()
    dev.synchronize()
    dev.timer_begin()
    for _ in range(steps):
        graph.launch()
    ms = dev.timer_end()
    dev.synchronize()
    med = median_replay_ms(dev, graph, median_replays) if median_replays else None
    return ms / steps, med


def bench_gemv(dev, n, k, copies, steps, warmup, seed, launches=None):
    """`launches` GEMVs per replay (default one per copy), cycling through
    `copies` distinct weight copies: cold when the copies exceed the 256 MB
    last-level cache (MALL), warm with one copy (held in the L2s)."""
    w = Weights(dev, n, k, copies, seed)
    x = dev.storage_from_bytes(synth.bf16_normal(seed + 1, (1, k)).tobytes())
    y = dev.empty(2 * n)
    launches = launches or copies

    def enqueue():
        for i in range(launches):
            q4_matmul(dev, x.ptr, 1, k, w.ptrs[i % copies], n, y.ptr)

    ms_step, med_step = timed_graph(dev, enqueue, steps, warmup)
    per_launch_ms = ms_step / launches
    gbs = gemv_bytes(1, n, k) / (per_launch_ms * 1e-3) / 1e9
    med_us = med_step / launches * 1e3
    return {"n": n, "k": k, "copies": copies, "launches_per_replay": launches,
            "distinct_weight_bytes": copies * gemv_bytes(1, n, k),
            "us_per_launch": per_launch_ms * 1e3, "GB_per_s": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
            "median_us_per_launch": med_us, "median_GB_per_s": gemv_bytes(1, n, k) / (med_us * 1e-6) / 1e9,
            "median_over_replays": MEDIAN_REPLAYS, "ms_per_step": ms_step}


def bench_lm_head(dev, steps, warmup):
    """The LM-head GEMV (128256 x 3072, 222 MB per launch). Cold: 3 weight
    copies cycled, so each launch's weights were last read two launches (444
    MB) earlier, more than the 256 MB MALL holds; warm: one copy. 12 launches
    per replay, so the individually timed replays' medians carry one graph
    launch per 12 GEMVs rather than per 3."""
    return {"lm_head_gemv_cold": bench_gemv(dev, 128256, 3072, 3, steps, warmup, seed=3, launches=12),
            "lm_head_gemv_warm": bench_gemv(dev, 128256, 3072, 1, steps, warmup, seed=3, launches=12)}


_TABLES: dict = {}


def bench_embed(dev, batch, steps, warmup, seed, tables=1, reps=12):
    """Config 2: the q4 gather of `batch` ids from a [128256, 3072] table.
    Each replay runs `reps` gathers, gather i from table i % tables with its
    own ids: cold with 3 tables (663 MB, more than the MALL holds), warm with
    one table and one id set repeated."""
    rows, k = 128256, 3072
    if (seed, rows, k) not in _TABLES:
        _TABLES[(seed, rows, k)] = synth.q4_weights(seed, rows, k)
    base = _TABLES[(seed, rows, k)]
    tabs = []
    for c in range(tables):
        wq = base[0] ^ np.uint32((0x9E3779B9 * (c + 1)) & 0xFFFFFFFF) if c else base[0]
        tabs.append([dev.storage_from_bytes(np.ascontiguousarray(a).tobytes()) for a in (wq, base[1], base[2])])
    id_sets = [dev.storage_from_bytes(synth.token_ids(seed + (i if tables > 1 else 0), batch, rows).tobytes())
               for i in range(reps if tables > 1 else 1)]
    out = dev.empty(batch * k * 2)

    def enqueue():
        for i in range(reps):
            sts = tabs[i % tables]
            ids = id_sets[i % len(id_sets)]
            _lib.call("fh_q4_embed", dev.handle, *[ctypes.c_void_p(st.ptr) for st in sts], rows, k, 64,
                      ctypes.c_void_p(ids.ptr), batch, ctypes.c_void_p(out.ptr))

    ms_step, med_step = timed_graph(dev, enqueue, steps, warmup)
    ms, med = ms_step / reps, med_step / reps
    gbs = embed_bytes(batch, k) / (ms * 1e-3) / 1e9
    return {"batch": batch, "tables": tables, "us_per_launch": ms * 1e3, "GB_per_s": gbs,
            "frac_hbm_peak": gbs / HBM_PEAK_GBS, "median_us_per_launch": med * 1e3,
            "median_GB_per_s": embed_bytes(batch, k) / (med * 1e-3) / 1e9,
            "cache": "cold (3 tables, distinct ids per launch)" if tables > 1 else "warm (one table, same ids)"}


def bench_gemm(dev, m, n, k, steps, warmup, seed):
    w = Weights(dev, n, k, 1, seed)
    x = dev.storage_from_bytes(synth.bf16_normal(seed + 1, (m, k)).tobytes())
    y = dev.empty(2 * m * n)
    reps = 4

    def enqueue():
        for _ in range(reps):
            q4_matmul(dev, x.ptr, m, k, w.ptrs[0], n, y.ptr)

    ms_step, med_step = timed_graph(dev, enqueue, steps, warmup)
    ms, med = ms_step / reps, med_step / reps
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"m": m, "n": n, "k": k, "us_per_launch": ms * 1e3, "TFLOP_per_s": tflops,
            "frac_bf16_peak": tflops / BF16_PEAK_TFLOPS, "median_us_per_launch": med * 1e3,
            "median_TFLOP_per_s": 2.0 * m * n * k / (med * 1e-3) / 1e12}


def bench_copy_sweep(dev, steps, warmup):
    """Where the warm GEMV's speed comes from: 48 launches per replay cycling
    through 1 .. 48 weight copies, for the config-1 shape (14.2 MB a copy)
    and the config-4 gate/up shape (16384 x 3072, 28.3 MB). One or two copies
    fit the eight 4 MB L2s; 8 copies of the first shape (113 MB) and of the
    second (227 MB) fit only the 256 MB MALL; 48 and 24 copies fit neither."""
    out = {}
    for n, counts in ((8192, (1, 2, 4, 8, 16, 48)), (16384, (1, 2, 4, 8, 16, 24))):
        for copies in counts:
            r = bench_gemv(dev, n, 3072, copies, steps, warmup, seed=1, launches=48)
            out[f"n{n}_copies{copies}"] = {"distinct_weight_MB": r["distinct_weight_bytes"] / 1e6,
                                           "us_per_launch": r["us_per_launch"],
                                           "median_us_per_launch": r["median_us_per_launch"]}
            print(f"[bench] n={n} copies={copies}: median {r['median_us_per_launch']:.2f} us", flush=True)
    return out


def bench_floors(dev, steps, warmup):
    """What one launch costs before its bytes: an almost empty kernel
    (fh_advance_positions on one word) replayed 200 times per graph, and
    fh_read_probe (16-byte loads, nothing else) reading one config-1 GEMV's
    worth of bytes (14,178,304) per launch over 48 distinct buffers, and a
    1 GiB buffer per launch (the sustained read rate)."""
    pos = dev.zeros(4)

    def tiny():
        for _ in range(200):
            _lib.call("fh_advance_positions", dev.handle, ctypes.c_void_p(pos.ptr), 1, 1)

    tiny_ms, tiny_med = timed_graph(dev, tiny, steps, warmup)
    out = {"empty_kernel_us": tiny_ms / 200 * 1e3, "empty_kernel_median_us": tiny_med / 200 * 1e3}
    for label, nbytes, copies in (("gemv_bytes", gemv_bytes(1, 8192, 3072) // 16 * 16, 48), ("1GiB", 1 << 30, 2)):
        blocks = ctypes.c_uint64()
        _lib.call("fh_read_probe_blocks", nbytes, ctypes.byref(blocks))
        bufs = [dev.zeros(nbytes) for _ in range(copies)]
        sink = dev.empty(blocks.value * 4)

        def reads():
            for b in bufs:
                _lib.call("fh_read_probe", dev.handle, ctypes.c_void_p(b.ptr), nbytes, ctypes.c_void_p(sink.ptr))

        ms, med = timed_graph(dev, reads, steps, warmup)
        out[f"read_{label}"] = {"bytes_per_launch": nbytes, "buffers": copies, "us_per_launch": ms / copies * 1e3,
                                "GB_per_s": nbytes / (ms / copies * 1e-3) / 1e9,
                                "median_us_per_launch": med / copies * 1e3}
        del bufs
    return out


def cpu_baseline(seconds: float = 12.0):
    """Reference arithmetic of the config-1 GEMV on the host (oracle)."""
    import oracle as O  # checker only: the bench's CPU baseline leg

    n, k = 8192, 3072
    wq, s, b = synth.q4_weights(1, n, k)
    x = synth.bf16_normal(2, (1, k))
    out = {}
    cores = os.cpu_count() or 1
    for label, threads, budget in (("1_thread", 1, seconds * 0.5), ("all_cores", cores, seconds * 0.5)):
        calls, t0 = 0, time.perf_counter()
        while True:
            O.q4_linear(x, wq, s, b, threads=threads)
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget:
                break
        ms = el / calls * 1e3
        out[label] = {"threads": threads, "calls": calls, "ms_per_call": ms,
                      "GB_per_s": gemv_bytes(1, n, k) / (ms * 1e-3) / 1e9}
    cpu = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return out, cpu


def decode_step_bytes(cfg, context: float, batch: int = 1) -> int:
    """HBM bytes one decode step must read at a given context: every q4 linear
    (weights + scales/biases, read once for the whole batch), the LM head
    (tied table), the norm weights and each sequence's K/V cache rows
    attended to."""
    def q4(n, k):
        return n * k // 2 + 4 * n * (k // 64)

    per_layer = (q4(cfg.qkv_rows, cfg.hidden) + q4(cfg.hidden, cfg.n_heads * cfg.head_dim)
                 + q4(2 * cfg.ffn, cfg.hidden) + q4(cfg.hidden, cfg.ffn) + 2 * 2 * cfg.hidden
                 + int(batch * 2 * cfg.n_kv_heads * cfg.head_dim * 2 * context))
    return cfg.n_layers * per_layer + q4(cfg.vocab, cfg.hidden) + 2 * cfg.hidden


def bench_decode(dev, new_tokens: int, agreement: int, seed: int = 0):
    """Config 4: Llama-3.2-3B-shaped random-init q4 decoder, the reference's
    512 seeded prompt ids (SplitMix64 seed 0, vocab 128256), greedy decode
    through the captured step."""
    from foundry_amd.llama import LlamaConfig, Q4Llama

    cfg = LlamaConfig.llama_3_2_3b()
    prompt = synth.token_ids(0, 512, cfg.vocab)
    max_len = len(prompt) + max(new_tokens, agreement)
    t0 = time.perf_counter()
    model = Q4Llama(dev, cfg, seed, max_len, max_tokens=len(prompt) + agreement)
    build_s = time.perf_counter() - t0
    # one untimed run of the same prompt first, as the reference's bench runs
    # whole warm-up runs before its measured ones (src/bench/mod.rs:157-170)
    model.generate(prompt, min(4, max_len - len(prompt)))
    gc.collect()
    dev.timer_begin()
    model.prefill(prompt)
    prefill_ms = dev.timer_end()
    log = dev.zeros(4 * new_tokens)
    first = np.empty(1, dtype=np.uint32)
    _lib.call("fh_download", dev.handle, first.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(model.buf["next"].ptr), 4)
    graph = model.capture_decode(log, new_tokens)
    dev.timer_begin()
    for _ in range(new_tokens - 1):
        graph.launch()
    decode_ms = dev.timer_end()
    tokens = np.empty(new_tokens, dtype=np.uint32)
    _lib.call("fh_download", dev.handle, tokens.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(log.ptr), tokens.nbytes)
    tokens[0] = first[0]
    steps = new_tokens - 1
    step_ms = decode_ms / steps
    # step i feeds position len(prompt) + i and attends to that many keys + 1
    mean_ctx = len(prompt) + (steps + 1) / 2
    step_bytes = decode_step_bytes(cfg, mean_ctx)
    out = {
        "config": "Llama-3.2-3B shape (28 layers, hidden 3072, 24/8 heads, head_dim 128, FFN 8192, vocab 128256), "
                  "q4 group 64, tied embedding/LM head, random init",
        "prompt_tokens": len(prompt), "new_tokens": new_tokens,
        "prefill_ms": prefill_ms, "prefill_tok_s": len(prompt) / (prefill_ms * 1e-3),
        "decode_ms_per_step": step_ms, "decode_tok_s": 1e3 / step_ms,
        "decode_bytes_per_step": step_bytes,
        "decode_GB_per_s": step_bytes / (step_ms * 1e-3) / 1e9,
        "decode_frac_hbm_peak": step_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "decode_ceiling_tok_s_at_peak": HBM_PEAK_GBS * 1e9 / step_bytes,
        "model_build_s": build_s,
        "first_tokens": tokens[:8].tolist(),
    }
    if agreement:
        out["agreement"] = greedy_agreement(model, cfg, seed, prompt, tokens, agreement)
    return out


def config5_parity(dev, cfg, seed, depth_ids, prompt_ids, first8, max_len):
    """Config 5's logits against two references, for sequence 0:
    - batch invariance: the bench model's prefill logits at batch 8 against
      the same sequence run alone at batch 1 (all 32 layers; rows of a batch
      are independent in the reference);
    - the restatement (oracle/llama_ref.py): a 2-layer model of the same
      shapes at batch 8 and context 4096, its decode step's logits."""
    from foundry_amd.llama import LlamaConfig, Q4Llama, embed_weights, final_norm_weight, layer_weights
    from oracle import llama_ref as R  # checker only

    def err(a, b):
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))

    d, p = depth_ids.shape[1], prompt_ids.shape[1]
    t0 = time.perf_counter()
    one = Q4Llama(dev, cfg, seed, max_len, max_tokens=p, batch=1)
    one.generate(prompt_ids[:1], 1, depth=depth_ids[:1])
    first1 = R.from_bf16(one.logits())
    del one
    out = {"batch_invariance_seq0_prefill_logits_err": err(first8[0], first1),
           "batch_invariance_bit_identical_fraction": float(np.mean(first8[0] == first1))}
    batch = depth_ids.shape[0]
    two = LlamaConfig(2, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab)
    m2 = Q4Llama(dev, two, seed, max_len, max_tokens=p, batch=batch)
    # greedy through the captured batch-8 decode step, reading sequence 0's
    # logits after the prefill and after every step
    m2.generate(prompt_ids, 1, depth=depth_ids)
    gpu_logits = [R.from_bf16(m2.logits())[0]]
    gpu_tokens = [int(m2.next_tokens()[0])]
    graph = m2.capture_step()
    for _ in range(CONFIG5_GREEDY - 1):
        graph.launch()
        gpu_logits.append(R.from_bf16(m2.logits())[0])
        gpu_tokens.append(int(m2.next_tokens()[0]))
    del graph, m2
    ref = R.RefLlama(two, embed_weights(two, seed), [layer_weights(two, seed, l) for l in range(2)],
                     final_norm_weight(two, seed), max_len)
    logits = ref.forward(list(np.concatenate([depth_ids[0], prompt_ids[0]])), np.arange(d + p), batch=batch)
    exp_tokens, exp_tops = [], []
    for i in range(CONFIG5_GREEDY):
        exp_tokens.append(R.argmax(logits))
        exp_tops.append(R.top_ids(logits, 5))
        # step 1 is fed the GPU's token, so its logits compare like with like
        # (the greedy rule below then follows the restatement's own tokens
        # only while both agree)
        feed = gpu_tokens[0] if i == 0 else exp_tokens[-1]
        if i + 1 < CONFIG5_GREEDY:
            logits = ref.forward([feed], np.array([d + p + i]), batch=batch)
            if i == 0:
                out["restatement_2_layer_decode_step_logits_err"] = err(gpu_logits[1], logits)
                out["restatement_2_layer_top5_equal"] = R.top_ids(gpu_logits[1], 5) == R.top_ids(logits, 5)
                if gpu_tokens[0] != exp_tokens[0]:
                    break
    n = len(exp_tokens)
    gpu_tops = [R.top_ids(l, 5) for l in gpu_logits[:n]]
    out["restatement_2_layer_greedy_seq0"] = {
        **R.compare_generation(np.array(gpu_tokens[:n]), gpu_tops, np.array(exp_tokens), exp_tops),
        "gpu_tokens": gpu_tokens[:n], "reference_arithmetic_tokens": exp_tokens}
    out["s"] = time.perf_counter() - t0
    return out


# greedy steps of config 5's 2-layer restatement comparison (sequence 0)
CONFIG5_GREEDY = 8


def bench_decode_batched(dev, new_tokens: int, seed: int = 0, batch: int = 8, depth: int = 2048,
                         prompt_len: int = 2048, parity: bool = True):
    """Config 5: Llama-3.1-8B-shaped random-init q4 decoder (32 layers,
    hidden 4096, 32/8 heads, FFN 14336, vocab 128256; the q4 table is tied as
    the reference's model requires, src/models/llama/config.rs:177-180) over
    `batch` sequences, run as the reference's bench runs depth rows
    (src/bench/mod.rs:203-300): depth ids fill every cache untimed, the
    prompt step is the timed prefill, then greedy decode steps start at
    context depth + prompt_len. Ids come from one SplitMix64 stream, every
    depth row then every prompt row (draw_inputs, src/bench/mod.rs:203-241).
    Rates follow the reference's report: P / Tp with P = batch * prompt
    tokens, and D / Td with D = decode steps * batch
    (tools/reference/README.md:83-108)."""
    from foundry_amd.llama import LlamaConfig, Q4Llama

    cfg = LlamaConfig.llama_3_1_8b()
    ids = synth.token_ids(seed, batch * (depth + prompt_len), cfg.vocab)
    depth_ids = ids[:batch * depth].reshape(batch, depth)
    prompt_ids = ids[batch * depth:].reshape(batch, prompt_len)
    max_len = depth + prompt_len + new_tokens
    t0 = time.perf_counter()
    model = Q4Llama(dev, cfg, seed, max_len, max_tokens=prompt_len, batch=batch)
    build_s = time.perf_counter() - t0
    model.generate(prompt_ids[:, :16], 3)  # warm the prefill and decode kernels (positions later overwritten)
    t0 = time.perf_counter()
    for s0 in range(0, depth, prompt_len):
        model.step(depth_ids[:, s0:s0 + prompt_len], s0)
    dev.synchronize()
    depth_s = time.perf_counter() - t0
    gc.collect()
    dev.timer_begin()
    model.step(prompt_ids, depth)
    prefill_ms = dev.timer_end()
    first8 = (model.logits().astype(np.uint32) << 16).view(np.float32) if parity else None
    first = np.empty(batch, dtype=np.uint32)
    _lib.call("fh_download", dev.handle, first.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(model.buf["next"].ptr),
              first.nbytes)
    log = dev.zeros(4 * batch * new_tokens)
    graph = model.capture_decode(log, new_tokens)
    dev.timer_begin()
    for _ in range(new_tokens - 1):
        graph.launch()
    decode_ms = dev.timer_end()
    tokens = np.empty((batch, new_tokens), dtype=np.uint32)
    _lib.call("fh_download", dev.handle, tokens.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(log.ptr), tokens.nbytes)
    tokens[:, 0] = first
    steps = new_tokens - 1
    step_ms = decode_ms / steps
    ctx0 = depth + prompt_len
    step_bytes = decode_step_bytes(cfg, ctx0 + (steps + 1) / 2, batch)
    gbs = step_bytes / (step_ms * 1e-3) / 1e9
    return {
        "config": "Llama-3.1-8B shape (32 layers, hidden 4096, 32/8 heads, head_dim 128, FFN 14336, vocab 128256), "
                  "q4 group 64, tied q4 embedding/LM head, random init",
        "batch": batch, "depth_tokens": depth, "prompt_tokens": prompt_len, "new_tokens": new_tokens,
        "decode_context_first_step": ctx0,
        "prefill_ms": prefill_ms, "prompt_tokens_per_s": batch * prompt_len / (prefill_ms * 1e-3),
        "depth_s_untimed": depth_s,
        "decode_ms_per_step": step_ms, "decode_tokens_per_s": batch * 1e3 / step_ms,
        "decode_bytes_per_step": step_bytes, "decode_GB_per_s": gbs, "decode_frac_hbm_peak": gbs / HBM_PEAK_GBS,
        "decode_ceiling_tokens_per_s_at_peak": batch * HBM_PEAK_GBS * 1e9 / step_bytes,
        "model_build_s": build_s,
        "first_tokens": tokens[:, :4].tolist(),
        **({"parity": config5_parity(dev, cfg, seed, depth_ids, prompt_ids, first8, max_len)} if parity else {}),
    }


def eager_decode_steps(dev, steps: int, batched: bool, seed: int = 0):
    """Config 4 (or config 5 when `batched`) set up as bench_decode /
    bench_decode_batched do (the depth rows of config 5 are left out: the
    caches hold the prompt), then `steps` decode steps launched op by op
    (Q4Llama.eager_step): the same kernels as the captured step, for kernel
    traces taken without graph replay."""
    from foundry_amd.llama import LlamaConfig, Q4Llama

    if batched:
        cfg, batch = LlamaConfig.llama_3_1_8b(), 8
        ids = synth.token_ids(seed, batch * 4096, cfg.vocab).reshape(batch, 4096)
        prompt = ids[:, 2048:]
        model = Q4Llama(dev, cfg, seed, 4096 + steps + 1, max_tokens=2048, batch=batch)
        model.step(ids[:, :2048], 0)  # depth rows: context 4096 at the first step
        model.step(prompt, 2048)
    else:
        cfg, batch = LlamaConfig.llama_3_2_3b(), 1
        prompt = synth.token_ids(0, 512, cfg.vocab)
        model = Q4Llama(dev, cfg, seed, len(prompt) + steps + 1, max_tokens=len(prompt))
        model.prefill(prompt)
    dev.synchronize()
    dev.timer_begin()
    for _ in range(steps):
        model.eager_step()
    ms = dev.timer_end()
    return {"config": "Llama-3.1-8B shape, batch 8, context 4096" if batched else "Llama-3.2-3B shape, batch 1",
            "eager_steps": steps, "ms_per_eager_step": ms / steps,
            "next_tokens": model.next_tokens()[:4].tolist()}


def greedy_agreement(model, cfg, seed, prompt, tokens, n):
    """Greedy agreement with the CPU restatement of the reference's forward
    (oracle/llama_ref.py) over the first n new tokens, by the reference's rule
    (src/eval/generation.rs:132-176) with top-k 5."""
    from foundry_amd.llama import embed_weights, final_norm_weight, layer_weights
    from oracle import llama_ref as R  # checker only

    t0 = time.perf_counter()
    layers = [layer_weights(cfg, seed, l) for l in range(cfg.n_layers)]
    ref = R.RefLlama(cfg, embed_weights(cfg, seed), layers, final_norm_weight(cfg, seed), len(prompt) + n)
    build_s = time.perf_counter() - t0
    exp_tokens, exp_tops = ref.generate(prompt, n)
    got = tokens[:n]
    # first-step logits after the prompt, beside the token rule (random-init
    # weights whose mean is -s/2 make greedy decode repeat a few tokens)
    model.prefill(prompt)
    gpu_logits = R.from_bf16(model.logits()).astype(np.float64)
    ref_logits = ref.first_logits.astype(np.float64)
    first_step = {"logits_max_abs_err_rel": float(np.max(np.abs(gpu_logits - ref_logits)) / np.max(np.abs(ref_logits))),
                  "top5_gpu": R.top_ids(gpu_logits.astype(np.float32), 5),
                  "top5_reference_arithmetic": R.top_ids(ref_logits.astype(np.float32), 5),
                  "distinct_greedy_tokens": int(len(set(got.tolist())))}
    # the batch-1 decode step itself (the captured graph the bench replays:
    # dot2 GEMVs with the RMSNorm prologue and SiLU epilogue, the one-launch
    # attention) from the prefill's token, against the restatement's step
    # from the same token (its step_logits[1])
    decode_step = None
    if n > 1 and int(got[0]) == int(exp_tokens[0]):
        graph = model.capture_step()
        graph.launch()
        step = R.from_bf16(model.logits()).astype(np.float64)
        want = ref.step_logits[1].astype(np.float64)
        decode_step = {"logits_max_abs_err_rel": float(np.max(np.abs(step - want)) / np.max(np.abs(want))),
                       "top5_gpu": R.top_ids(step.astype(np.float32), 5),
                       "top5_reference_arithmetic": R.top_ids(want.astype(np.float32), 5)}
    # what the prefill GEMM's bf16 weight tiles cost against fp32 dequantised
    # weights throughout (BASELINE's dequant arithmetic): the restatement's
    # first-step logits both ways, and the GPU's against the fp32 one
    saved = R.GEMV_MAX_ROWS
    try:
        R.GEMV_MAX_ROWS = 1 << 30
        ref.reset()
        f32_logits = ref.forward(list(int(i) for i in prompt), np.arange(len(prompt))).astype(np.float64)
    finally:
        R.GEMV_MAX_ROWS = saved
    scale = np.max(np.abs(f32_logits))
    drift = {"restatement_bf16_vs_fp32_weights_logits_err": float(np.max(np.abs(ref_logits - f32_logits)) / scale),
             "gpu_vs_fp32_weight_restatement_logits_err": float(np.max(np.abs(gpu_logits - f32_logits)) / scale),
             "top5_fp32_weights": R.top_ids(f32_logits.astype(np.float32), 5)}
    report = R.compare_generation(got, [[]] * n, exp_tokens, exp_tops)
    if report["first_divergence"] is not None:
        d = report["first_divergence"]
        model.prefill(np.concatenate([prompt, got[:d]]).astype(np.uint32))
        gpu_tops = [[]] * n
        gpu_tops[d] = R.top_ids(R.from_bf16(model.logits()), 5)
        report = R.compare_generation(got, gpu_tops, exp_tokens, exp_tops)
    report["first_step"] = first_step
    report["decode_step"] = decode_step
    report["prefill_weight_rounding_drift"] = drift
    report["cpu_s"] = time.perf_counter() - t0
    # the restatement's own speed on this host (numpy fp32, one process)
    report["cpu_reference"] = {"threads": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                               "build_s": build_s, "prefill_s": ref.prefill_s,
                               "prefill_tok_s": len(prompt) / ref.prefill_s,
                               "decode_tok_s": (n - 1) / ref.decode_s if n > 1 else None}
    report["gpu_tokens"] = got.tolist()
    report["reference_arithmetic_tokens"] = exp_tokens.tolist()
    return report


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_8192x3072_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the headline GEMV, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (copy-calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_dispatch="):
                    return int(float(line.split("=", 1)[1].split()[0]))
    except OSError:
        return None
    return None


def calibrate_copy() -> int:
    """One device-to-device copy of a known size on the device's stream: the
    plain copy kernel that scales the FETCH_SIZE / WRITE_SIZE counters."""
    from foundry_amd.profiling import CALIBRATION_BYTES

    dev = HipDevice(0)
    src = dev.zeros(CALIBRATION_BYTES)
    dst = dev.empty(CALIBRATION_BYTES)
    hip = ctypes.CDLL("libamdhip64.so")
    stream = ctypes.c_void_p()
    _lib.call("fh_device_stream", dev.handle, ctypes.byref(stream))
    hip.hipMemcpyDtoDAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    rc = hip.hipMemcpyDtoDAsync(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), CALIBRATION_BYTES, stream)
    if rc != 0:
        raise RuntimeError(f"hipMemcpyDtoDAsync failed: {rc}")
    dev.synchronize()
    dev.close()
    print(f"[bench] copied {CALIBRATION_BYTES} bytes device to device", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only, no secondary lines")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one device copy of known size (counter calibration)")
    ap.add_argument("--decode-tokens", type=int, default=256, help="config-4 greedy steps (0 skips)")
    ap.add_argument("--agreement", type=int, default=16,
                    help="compare the first N config-4 tokens with the CPU restatement (0 skips)")
    ap.add_argument("--no-parity", action="store_true", help="skip config 5's logits checks")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the config-4 decode (for a kernel trace of the step); prints its JSON")
    ap.add_argument("--batched-tokens", type=int, default=32,
                    help="config-5 greedy steps per sequence (8B shape, batch 8, context 4096; 0 skips)")
    ap.add_argument("--batched-only", action="store_true", help="only the config-5 run; prints its JSON")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the two config-3 GEMMs (for kernel traces and counters); prints their JSON")
    ap.add_argument("--floors-only", action="store_true",
                    help="only the launch and read floors; prints their JSON")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="only the LM-head GEMV (128256 x 3072) cold and warm legs; prints their JSON")
    ap.add_argument("--copy-sweep-only", action="store_true",
                    help="only the decode GEMV over 1 .. 48 weight copies (L2-, MALL- and HBM-resident "
                         "weights); prints their JSON")
    ap.add_argument("--eager-steps", type=int, default=0,
                    help="only config 4 (or with --batched-only config 5): the prompt, then this many decode "
                         "steps launched op by op instead of as a graph (for kernel traces: the profiler's "
                         "graph interception has crashed on the replayed legs); prints their JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the q4 path has no multi-GPU form here)", file=sys.stderr)
        return 2

    if args.calibrate_copy:
        calibrate_copy()
    dev = HipDevice(0)
    small = max(5, args.steps // 5)
    if args.eager_steps > 0:
        d = eager_decode_steps(dev, args.eager_steps, batched=args.batched_only)
        dev.close()
        print(json.dumps(d), flush=True)
        return 0
    if (args.decode_only or args.batched_only or args.gemm_only or args.floors_only or args.lm_head_only
            or args.copy_sweep_only):
        if args.decode_only:
            d = bench_decode(dev, max(2, args.decode_tokens), args.agreement)
        elif args.batched_only:
            d = bench_decode_batched(dev, max(2, args.batched_tokens), parity=not args.no_parity)
        elif args.gemm_only:
            d = {"gemm_gate_up": bench_gemm(dev, 2048, 8192, 3072, args.steps, args.warmup, seed=7),
                 "gemm_down": bench_gemm(dev, 2048, 3072, 8192, args.steps, args.warmup, seed=9)}
        elif args.lm_head_only:
            d = bench_lm_head(dev, args.steps, args.warmup)
        elif args.copy_sweep_only:
            d = bench_copy_sweep(dev, args.steps, args.warmup)
        else:
            d = bench_floors(dev, args.steps, args.warmup)
        dev.close()
        print(json.dumps(d), flush=True)
        return 0
    head = bench_gemv(dev, 8192, 3072, args.copies, args.steps, args.warmup, seed=1)
    print(f"[bench] gemv 8192x3072: {head['us_per_launch']:.2f} us/launch, {head['GB_per_s']:.0f} GB/s "
          f"(median {head['median_us_per_launch']:.2f} us)", flush=True)
    secondary = {}
    if not args.quick:
        secondary["gemv_warm"] = bench_gemv(dev, 8192, 3072, 1, small, 2, seed=1, launches=args.copies)
        secondary.update(bench_lm_head(dev, small, 2))
        print(f"[bench] gemv warm {secondary['gemv_warm']['GB_per_s']:.0f} GB/s; lm head cold "
              f"{secondary['lm_head_gemv_cold']['GB_per_s']:.0f}, warm {secondary['lm_head_gemv_warm']['GB_per_s']:.0f} GB/s",
              flush=True)
        for b in (4096, 64, 1):
            for tables, tag in ((3, "cold"), (1, "warm")):
                secondary[f"embed_b{b}_{tag}"] = bench_embed(dev, b, small, 2, seed=5, tables=tables)
        print(f"[bench] embed B=4096: cold {secondary['embed_b4096_cold']['GB_per_s']:.0f}, warm "
              f"{secondary['embed_b4096_warm']['GB_per_s']:.0f} GB/s; B=64 cold "
              f"{secondary['embed_b64_cold']['median_us_per_launch']:.2f} us", flush=True)
        # the compute-bound GEMMs get the full warmup: their first replays after
        # the HBM-bound legs run slower and would weigh on the mean
        secondary["gemm_gate_up"] = bench_gemm(dev, 2048, 8192, 3072, small, args.warmup, seed=7)
        secondary["gemm_down"] = bench_gemm(dev, 2048, 3072, 8192, small, args.warmup, seed=9)
        print(f"[bench] gemm: mean {secondary['gemm_gate_up']['TFLOP_per_s']:.0f} / "
              f"{secondary['gemm_down']['TFLOP_per_s']:.0f} TFLOP/s, median "
              f"{secondary['gemm_gate_up']['median_TFLOP_per_s']:.0f} / "
              f"{secondary['gemm_down']['median_TFLOP_per_s']:.0f} TFLOP/s", flush=True)
        secondary["floors"] = bench_floors(dev, small, 2)
        f = secondary["floors"]
        print(f"[bench] floors: empty kernel {f['empty_kernel_us']:.2f} us; read 14.2 MB "
              f"{f['read_gemv_bytes']['us_per_launch']:.2f} us ({f['read_gemv_bytes']['GB_per_s']:.0f} GB/s); "
              f"read 1 GiB {f['read_1GiB']['GB_per_s']:.0f} GB/s", flush=True)
    if not args.quick and args.decode_tokens > 1:
        secondary["decode_llama_3_2_3b"] = bench_decode(dev, args.decode_tokens, args.agreement)
        d = secondary["decode_llama_3_2_3b"]
        print(f"[bench] decode: {d['decode_tok_s']:.0f} tok/s ({d['decode_frac_hbm_peak']*100:.1f}% of HBM roofline), "
              f"prefill {d['prefill_tok_s']:.0f} tok/s", flush=True)
    if not args.quick and args.batched_tokens > 1:
        secondary["decode_llama_3_1_8b_b8"] = bench_decode_batched(dev, args.batched_tokens, parity=not args.no_parity)
        d = secondary["decode_llama_3_1_8b_b8"]
        print(f"[bench] 8B batch 8 at context 4096: decode {d['decode_tokens_per_s']:.0f} tok/s "
              f"({d['decode_frac_hbm_peak']*100:.1f}% of HBM roofline), prefill {d['prompt_tokens_per_s']:.0f} tok/s",
              flush=True)
    dev.close()

    cpu = None
    if not args.no_cpu:
        base, model = cpu_baseline()
        cpu = {"value": base["1_thread"]["GB_per_s"], "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": (f"config-1 GEMV x[1,3072].W[8192,3072]^T, reference arithmetic "
                          f"(oracle/liboracle.so), {base['1_thread']['calls']} calls single-threaded; "
                          f"all {base['all_cores']['threads']} cores: {base['all_cores']['GB_per_s']:.2f} GB/s"),
               "cpu_model": model, "all_cores": base["all_cores"]}
        dec = secondary.get("decode_llama_3_2_3b", {}).get("agreement", {}).get("cpu_reference")
        if dec:
            cpu["config4_restatement"] = dec

    per_launch_bytes = gemv_bytes(1, 8192, 3072)
    line = {
        "metric": METRIC,
        "value": round(head["GB_per_s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (SplitMix64-seeded, task config distributions)",
        "config": {"workload": f"q4 decode GEMV x[1,3072].W[8192,3072]^T over {args.copies} weight copies per step",
                   "m": 1, "n": 8192, "k": 3072, "group": 64, "copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": round(head["GB_per_s"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["GB_per_s"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT),
                     "algorithmic_bytes_per_launch": per_launch_bytes,
                     "us_per_launch": head["us_per_launch"],
                     "median_us_per_launch": head["median_us_per_launch"],
                     "median_over_replays": MEDIAN_REPLAYS},
        "cpu_baseline": cpu,
        "decode_tok_s": secondary.get("decode_llama_3_2_3b", {}).get("decode_tok_s"),
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
