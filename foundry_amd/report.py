"""Benchmark reports in the reference's report.json schema.

Restates the reference's bench (src/bench/mod.rs:50-360), its metrics
(src/bench/metrics.rs:20-260), statistics (src/bench/stats.rs:10-105) and the
CLI's record ({"metadata", ...report}, src/cli/command.rs:65-73, 403-500);
metric definitions as tools/reference/README.md:71-199 states them:

* inputs: one SplitMix64 stream (seed), depth rows of every sequence, then
  prompt rows, then (no prompt) one start id per sequence;
* a run: the depth rows untimed, then the prompt step and the decode steps,
  each timed on the host; generation scope includes greedy selection and the
  token readback, forward scope synchronises after the forward and selects
  outside the timer; N new tokens per sequence include the prefill's;
* summaries: count, mean, sample stdev/variance, min, max and p10..p99
  interpolated between ranks; throughputs are summarised across per-run
  rates.

The decode step is this build's captured step (one HIP graph replay reading
its token and position from device memory). With profile "kernels" the steps
run eagerly instead and every C-ABI call is bracketed with device events, so
decode_kernel_gpu_ns holds per-call GPU time, keyed by the call and its sizes.
"""
from __future__ import annotations

import argparse
import ctypes
import datetime
import json
import os
import subprocess
import sys
import time
from collections import OrderedDict
from dataclasses import asdict, dataclass

import numpy as np

from . import _lib, synth

NS_PER_S = 1e9


class BenchError(Exception):
    def __init__(self, kind: str, message: str = ""):
        super().__init__(f"{kind}: {message}" if message else kind)
        self.kind = kind


# ---------------- statistics (src/bench/stats.rs) ----------------

def percentile(sorted_samples, percent: int):
    """Linear interpolation between ranks, rank = percent * (n - 1) / 100 in
    integer arithmetic (stats.rs:80-97); None without samples."""
    if not sorted_samples:
        return None
    last = len(sorted_samples) - 1
    scaled = min(percent, 100) * last
    lo = scaled // 100
    frac = scaled % 100
    lower = sorted_samples[lo]
    upper = sorted_samples[lo + 1] if lo + 1 < len(sorted_samples) else lower
    return lower + (upper - lower) * frac / 100


def summary(samples) -> dict:
    samples = [float(s) for s in samples]
    if not samples:
        raise BenchError("NoSample")
    srt = sorted(samples)
    mean = sum(samples) / len(samples)
    variance = sum((s - mean) ** 2 for s in samples) / (len(samples) - 1) if len(samples) > 1 else 0.0
    out = OrderedDict(count=len(samples), mean=mean, stdev=variance ** 0.5, variance=variance, min=srt[0],
                      max=srt[-1])
    for p in (10, 25, 50, 75, 90, 99):
        out[f"p{p}"] = percentile(srt, p)
    return out


def _opt_summary(samples):
    samples = list(samples)
    return summary(samples) if samples else None


# ---------------- config, inputs ----------------

@dataclass
class BenchConfig:
    """BenchConfig (src/bench/mod.rs:48-60)."""

    prompt_token_count: int = 512
    new_token_count: int = 128
    timing_scope: str = "generation"  # or "forward"
    depth_token_count: int = 0
    warmup_run_count: int = 1
    warmup_ms: int = 0
    run_count: int = 10
    batch_size: int = 1
    seed: int = 0
    profile: str | None = None  # None, "steps" or "kernels"

    def decode_step_count(self) -> int:
        return max(self.new_token_count - (1 if self.prompt_token_count > 0 else 0), 0)


def draw_inputs(config: BenchConfig, vocab: int):
    """draw_inputs (src/bench/mod.rs:203-241): one SplitMix64 stream; every
    sequence's depth row, then every prompt row, then (without a prompt) one
    start id per sequence."""
    b = config.batch_size
    n = b * (config.depth_token_count + config.prompt_token_count) + (b if config.prompt_token_count == 0 else 0)
    ids = synth.token_ids(config.seed, n, vocab) if n else np.zeros(0, np.uint32)
    d, p = config.depth_token_count, config.prompt_token_count
    depth = ids[:b * d].reshape(b, d)
    prompt = ids[b * d:b * (d + p)].reshape(b, p)
    start = ids[b * (d + p):] if p == 0 else None
    return depth, prompt, start


# ---------------- metrics (src/bench/metrics.rs) ----------------

def _throughput(tokens: float, ns):
    return NS_PER_S * tokens / ns if tokens > 0 and ns and ns > 0 else None


def metrics_from_runs(runs: list, config: BenchConfig) -> dict:
    if not runs:
        raise BenchError("NoSample")
    prompt_tokens = float(config.batch_size * config.prompt_token_count)
    derived = []
    for run in runs:
        decode_tokens = float(config.batch_size * len(run["decode"]))
        output_tokens = float(sum(len(row) for row in run["token_ids"]))
        decode_ns = sum(s["step_ns"] for s in run["decode"])
        total_ns = (run.get("prompt_step_ns") or 0) + decode_ns
        gen = run.get("generation_ns")
        intervals = max(len(run["token_ids"][0]) - 1, 0) if run["token_ids"] else 0
        first = run.get("first_token_ns")
        derived.append({
            "prompt": _throughput(prompt_tokens, run.get("prompt_step_ns")) if run.get("prompt_step_ns") is not None else None,
            "decode": _throughput(decode_tokens, decode_ns),
            "output": _throughput(output_tokens, gen) if gen is not None else None,
            "total": _throughput(prompt_tokens + output_tokens, gen) if gen is not None else None,
            "processed": _throughput(prompt_tokens + decode_tokens, total_ns),
            "tpot": (gen - first) / intervals if first is not None and gen is not None and intervals > 0 else None,
        })

    def d(key):
        return _opt_summary(x[key] for x in derived if x[key] is not None)

    decode_samples = [s for run in runs for s in run["decode"]]

    def prof(select):
        return _opt_summary(v for s in decode_samples if s.get("profile") is not None
                            for v in [select(s, s["profile"])] if v is not None)

    by_pos = OrderedDict()
    for s in decode_samples:
        by_pos.setdefault((s["position"], s["context_tokens"]), []).append(s)
    kernels = {}
    for s in decode_samples:
        for k, t in (s.get("profile") or {}).get("kernels", {}).items():
            if t.get("gpu_ns") is not None:
                kernels.setdefault(k, []).append(t["gpu_ns"])
    return OrderedDict(
        prompt_step_ns=_opt_summary(r["prompt_step_ns"] for r in runs if r.get("prompt_step_ns") is not None),
        decode_step_ns=_opt_summary(s["step_ns"] for s in decode_samples),
        decode_by_position=[OrderedDict(position=p, context_tokens=c, step_ns=summary(x["step_ns"] for x in ss),
                                        inter_token_ns=_opt_summary(x["inter_token_ns"] for x in ss
                                                                    if x.get("inter_token_ns") is not None))
                            for (p, c), ss in sorted(by_pos.items())],
        inter_token_ns=_opt_summary(s["inter_token_ns"] for s in decode_samples if s.get("inter_token_ns") is not None),
        tpot_ns=d("tpot"),
        step_sum_ns=summary((r.get("prompt_step_ns") or 0) + sum(s["step_ns"] for s in r["decode"]) for r in runs),
        first_token_ns=_opt_summary(r["first_token_ns"] for r in runs if r.get("first_token_ns") is not None),
        generation_ns=_opt_summary(r["generation_ns"] for r in runs if r.get("generation_ns") is not None),
        prompt_tokens_per_s=d("prompt"),
        decode_tokens_per_s=d("decode"),
        output_tokens_per_s=d("output"),
        total_tokens_per_s=d("total"),
        processed_tokens_per_s=d("processed"),
        decode_dispatch_count=prof(lambda s, p: sum(k["dispatch_count"] for k in p["kernels"].values())),
        decode_allocation_count=prof(lambda s, p: p["allocation_count"]),
        decode_allocated_bytes=prof(lambda s, p: p["allocated_bytes"]),
        decode_gpu_busy_ns=prof(lambda s, p: p.get("gpu_busy_ns")),
        decode_gpu_idle_ns=prof(lambda s, p: None if p.get("gpu_busy_ns") is None else s["step_ns"] - p["gpu_busy_ns"]),
        decode_kernel_gpu_ns=OrderedDict((k, summary(v)) for k, v in sorted(kernels.items())),
    )


# ---------------- metadata (src/bench/metadata.rs, src/cli/command.rs:403-460) ----------------

def git_commit(stdout: bytes):
    """A full 40-digit lowercase hex commit, else None."""
    try:
        c = stdout.decode("utf-8").strip()
    except UnicodeDecodeError:
        return None
    return c if len(c) == 40 and all(ch in "0123456789abcdef" for ch in c) else None


def read_git_commit():
    try:
        out = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, timeout=10,
                             cwd=os.path.dirname(os.path.abspath(__file__)))
    except (OSError, subprocess.SubprocessError):
        return None
    return git_commit(out.stdout) if out.returncode == 0 else None


def test_time() -> str:
    return datetime.datetime.now(datetime.timezone.utc).replace(microsecond=0).isoformat().replace("+00:00", "Z")


# ---------------- per-call GPU timing (profile "kernels") ----------------

class _CallTimer:
    """Brackets every C-ABI compute call with device events while active."""

    SKIP = {"fh_upload", "fh_download", "fh_alloc", "fh_free", "fh_synchronize", "fh_timer_begin", "fh_timer_end",
            "fh_take_profile", "fh_device_stream"}

    def __init__(self, dev):
        self.dev = dev
        self.kernels = {}

    def __enter__(self):
        self._orig = _lib.call

        def timed(name, *args):
            if name in self.SKIP:
                return self._orig(name, *args)
            sizes = [str(a) for a in args if isinstance(a, int) and not isinstance(a, bool) and 0 <= a < 1 << 31]
            key = " ".join([name] + sizes[1:])  # the first int is the device handle
            self.dev.timer_begin()
            rc = self._orig(name, *args)
            ms = self.dev.timer_end()
            k = self.kernels.setdefault(key, {"dispatch_count": 0, "gpu_ns": 0.0})
            k["dispatch_count"] += 1
            k["gpu_ns"] += ms * 1e6
            return rc

        _lib.call = timed
        return self

    def __exit__(self, *exc):
        _lib.call = self._orig

    def take(self):
        k, self.kernels = self.kernels, {}
        busy = sum(v["gpu_ns"] for v in k.values())
        return OrderedDict(kernels=OrderedDict(sorted(k.items())), allocation_count=0, allocated_bytes=0,
                           gpu_busy_ns=busy)


# ---------------- the bench (src/bench/mod.rs:147-345) ----------------

def _run(model, dev, config: BenchConfig, depth, prompt, start):
    b = config.batch_size
    prompt_len = prompt.shape[1]
    new = config.new_token_count
    kernels = config.profile == "kernels"
    dev.synchronize()
    dev.reset_run_memory_peak()
    samples = {"prompt_step_ns": None, "decode": [], "first_token_ns": None, "generation_ns": None,
               "token_ids": [[] for _ in range(b)]}
    t_start = time.perf_counter_ns()
    past = 0
    if depth.shape[1]:
        for s0 in range(0, depth.shape[1], model.max_tokens):
            model.step(depth[:, s0:s0 + model.max_tokens], s0)
        past = depth.shape[1]
    if config.timing_scope == "forward":
        dev.synchronize()
    graph = None
    timer = _CallTimer(dev) if kernels else None
    steps = max(new, 1 if prompt_len > 0 else 0)
    tokens = None
    for position in range(steps):
        is_prompt = position == 0 and prompt_len > 0
        t0 = time.perf_counter_ns()
        ctx = past
        if timer:
            timer.__enter__()
        try:
            if is_prompt:
                model.step(prompt, past)
            elif position == 0:  # no prompt: the start ids, one per sequence
                model.step(start.reshape(b, 1), past)
            else:
                if kernels:
                    model.eager_step()
                else:
                    if graph is None:
                        graph = model.capture_step()
                    graph.launch()
        finally:
            if timer:
                timer.__exit__()
        if config.timing_scope == "forward" or new == 0:
            dev.synchronize()
            t_end = time.perf_counter_ns()
            tokens = model.next_tokens() if new > 0 else None
        else:
            tokens = model.next_tokens()
            t_end = time.perf_counter_ns()
        step_ns = t_end - t0
        profile = timer.take() if timer else None
        if new > 0 and config.timing_scope == "generation":
            elapsed = t_end - t_start
            inter = None if samples["generation_ns"] is None else elapsed - samples["generation_ns"]
            if samples["first_token_ns"] is None:
                samples["first_token_ns"] = elapsed
            samples["generation_ns"] = elapsed
        else:
            inter = None
        if is_prompt:
            samples["prompt_step_ns"] = step_ns
            if profile is not None:
                samples["prompt_profile"] = profile
        else:
            rec = OrderedDict(position=len(samples["decode"]), context_tokens=ctx, step_ns=step_ns,
                              inter_token_ns=inter)
            if profile is not None:
                rec["profile"] = profile
            samples["decode"].append(rec)
        if tokens is not None:
            for r in range(b):
                samples["token_ids"][r].append(int(tokens[r]))
        past += prompt_len if is_prompt else 1
    peak = dev.run_memory_peak()
    samples["peak_memory_bytes"] = peak["bytes"]
    return samples


def bench(model, dev, config: BenchConfig) -> dict:
    """The reference's bench(): warmup runs, measured runs, metrics, peaks."""
    if config.prompt_token_count == 0 and config.new_token_count == 0:
        raise BenchError("NoToken")
    if config.batch_size != model.batch:
        raise BenchError("BatchSize", f"model built for {model.batch} sequences")
    depth, prompt, start = draw_inputs(config, model.cfg.vocab)
    warm = 0
    t0 = time.perf_counter()
    while warm < config.warmup_run_count or (time.perf_counter() - t0) * 1e3 < config.warmup_ms:
        _run(model, dev, config, depth, prompt, start)
        warm += 1
    runs = [_run(model, dev, config, depth, prompt, start) for _ in range(config.run_count)]
    session = dev.max_memory_allocated()
    report = OrderedDict(
        config=asdict(config),
        depth_ids=depth.tolist(),
        prompt_ids=prompt.tolist(),
    )
    if start is not None:
        report["start_ids"] = start.tolist()
    report["warmup_run_count"] = warm
    report["runs"] = runs
    report["metrics"] = metrics_from_runs(runs, config)
    report["peak_memory_bytes"] = max(r["peak_memory_bytes"] for r in runs)
    report["session_peak_memory_bytes"] = session["bytes"]
    report["peak_memory_source"] = session["source"]
    return report


def write_report(out_dir, record: dict, file_name: str = "report.json") -> str:
    os.makedirs(out_dir, exist_ok=True)
    path = os.path.join(out_dir, file_name)
    with open(path, "w") as f:
        json.dump(record, f, indent=2)
        f.write("\n")
    return path


def main(argv=None) -> int:
    from .device import HipDevice
    from .llama import LlamaConfig, Q4Llama

    ap = argparse.ArgumentParser(description="Benchmark prefill and greedy decode on random token ids and "
                                             "write report.json (the reference's bench schema).")
    ap.add_argument("--model", default="3b", help="3b or 8b (random-init q4 of that shape), or a q4 checkpoint dir")
    ap.add_argument("--prompt-tokens", type=int, default=512)
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--depth-tokens", type=int, default=0)
    ap.add_argument("--batch-size", type=int, default=1)
    ap.add_argument("--runs", type=int, default=10)
    ap.add_argument("--warmup-runs", type=int, default=1)
    ap.add_argument("--warmup-ms", type=int, default=0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--timing-scope", choices=["generation", "forward"], default="generation")
    ap.add_argument("--profile", choices=["steps", "kernels"], default=None)
    ap.add_argument("--out", required=True, help="directory that receives report.json")
    a = ap.parse_args(argv)
    config = BenchConfig(a.prompt_tokens, a.new_tokens, a.timing_scope, a.depth_tokens, a.warmup_runs, a.warmup_ms,
                         a.runs, a.batch_size, a.seed, a.profile)
    dev = HipDevice(0)
    max_len = a.depth_tokens + a.prompt_tokens + max(a.new_tokens, 1)
    max_tokens = max(a.prompt_tokens, min(max(a.depth_tokens, 1), 4096), 1)
    if a.model in ("3b", "8b"):
        cfg = LlamaConfig.llama_3_2_3b() if a.model == "3b" else LlamaConfig.llama_3_1_8b()
        model = Q4Llama(dev, cfg, 0, max_len, max_tokens, batch=a.batch_size)
        model_id = f"random-init q4 Llama {'3.2-3B' if a.model == '3b' else '3.1-8B'} shape"
    else:
        model = Q4Llama.from_checkpoint(dev, a.model, max_len, max_tokens, batch=a.batch_size)
        model_id = os.path.abspath(a.model)
    report = bench(model, dev, config)
    record = OrderedDict(metadata=OrderedDict(
        git_commit=read_git_commit(), test_time=test_time(), device="hip", device_name=dev.device_name(),
        model_id=model_id, model_bytes=model.weight_bytes(), model_parameter_count=model.parameter_count()))
    record.update(report)
    path = write_report(a.out, record)
    m = report["metrics"]
    print(json.dumps({"report": path, "prompt_tokens_per_s": (m["prompt_tokens_per_s"] or {}).get("mean"),
                      "decode_tokens_per_s": (m["decode_tokens_per_s"] or {}).get("mean"),
                      "peak_memory_bytes": report["peak_memory_bytes"]}))
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
