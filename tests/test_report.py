"""report.json machinery (foundry_amd/report.py) on the CPU: the reference's
own known answers for Summary (src/bench/stats.rs:118-185), Metrics::from_runs
(src/bench/metrics.rs:262-420) and git_commit (src/bench/metadata.rs:24-60),
and draw_inputs against the golden prompt ids of the reference's report."""
import json
import os

import numpy as np
import pytest

from foundry_amd.report import BenchConfig, BenchError, draw_inputs, git_commit, metrics_from_runs, percentile, summary

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "prompt_ids_seed0_vocab128256.json")


def test_summary_of_five_samples_matches_hand_values():
    s = summary([30.0, 10.0, 50.0, 20.0, 40.0])
    assert dict(s) == {"count": 5, "mean": 30.0, "stdev": 250 ** 0.5, "variance": 250.0, "min": 10.0, "max": 50.0,
                       "p10": 14.0, "p25": 20.0, "p50": 30.0, "p75": 40.0, "p90": 46.0, "p99": 49.6}


def test_summary_of_one_sample_has_zero_spread():
    s = summary([7.0])
    assert (s["count"], s["stdev"], s["variance"], s["p10"], s["p99"]) == (1, 0.0, 0.0, 7.0, 7.0)


def test_summary_of_no_sample_is_rejected():
    with pytest.raises(BenchError) as e:
        summary([])
    assert e.value.kind == "NoSample"


def test_median_of_an_even_count_averages_the_middle_pair():
    assert summary([4.0, 1.0, 3.0, 2.0])["p50"] == 2.5
    assert percentile([], 50) is None


def config(prompt, batch):
    return BenchConfig(prompt_token_count=prompt, new_token_count=4, timing_scope="generation", depth_token_count=7,
                       warmup_run_count=0, warmup_ms=0, run_count=1, batch_size=batch, seed=0, profile=None)


def run(prompt_step_ns, decode_ns, tokens, batch):
    return {"prompt_step_ns": prompt_step_ns,
            "first_token_ns": prompt_step_ns if prompt_step_ns is not None else (decode_ns[0] if decode_ns else None),
            "generation_ns": (prompt_step_ns or 0) + sum(decode_ns),
            "decode": [{"position": i, "context_tokens": i + 11, "step_ns": ns,
                        "inter_token_ns": ns if (prompt_step_ns is not None or i > 0) else None}
                       for i, ns in enumerate(decode_ns)],
            "token_ids": [[1] * tokens for _ in range(batch)], "peak_memory_bytes": 2_000_000_000}


@pytest.mark.parametrize("batch", [1, 2])
def test_rates_use_all_steps_and_actual_output_counts(batch):
    m = metrics_from_runs([run(1_000_000_000, [250_000_000, 250_000_000, 500_000_000], 4, batch)], config(4, batch))
    f = float(batch)
    assert m["prompt_tokens_per_s"]["mean"] == 4.0 * f
    assert m["decode_tokens_per_s"]["mean"] == 3.0 * f
    assert m["output_tokens_per_s"]["mean"] == 2.0 * f
    assert m["total_tokens_per_s"]["mean"] == 4.0 * f
    assert m["processed_tokens_per_s"]["mean"] == 3.5 * f
    assert m["step_sum_ns"]["mean"] == 2e9
    assert (m["decode_step_ns"]["count"], m["decode_step_ns"]["p50"]) == (3, 250_000_000.0)


def test_prompt_only_and_decode_only_have_defined_metrics():
    prompt = metrics_from_runs([{"prompt_step_ns": 250_000_000, "decode": [], "token_ids": [[]],
                                 "first_token_ns": None, "generation_ns": None}], config(2, 1))
    assert prompt["prompt_tokens_per_s"]["mean"] == 8.0
    assert prompt["output_tokens_per_s"] is None
    assert (prompt["decode_step_ns"], prompt["decode_tokens_per_s"]) == (None, None)
    decode = metrics_from_runs([run(None, [500_000_000] * 2, 2, 1)], config(0, 1))
    assert decode["prompt_tokens_per_s"] is None and decode["decode_tokens_per_s"]["mean"] == 2.0


def test_summaries_average_per_run_rates_and_preserve_dispersion():
    m = metrics_from_runs([run(None, [500_000_000] * 2, 2, 1), run(None, [250_000_000] * 2, 2, 1)], config(0, 1))
    r = m["output_tokens_per_s"]
    assert (r["count"], r["mean"], r["p50"], r["variance"]) == (2, 3.0, 3.0, 2.0)


def test_zero_duration_retains_latency_without_infinite_throughput():
    m = metrics_from_runs([run(0, [], 1, 1)], config(2, 1))
    assert m["step_sum_ns"]["mean"] == 0.0 and m["output_tokens_per_s"] is None


def test_empty_measurements_are_rejected():
    with pytest.raises(BenchError) as e:
        metrics_from_runs([], config(0, 1))
    assert e.value.kind == "NoSample"


def test_decode_by_position_and_kernel_summaries():
    r1 = run(1_000, [10, 20], 3, 1)
    r2 = run(1_000, [30, 40], 3, 1)
    r1["decode"][0]["profile"] = {"kernels": {"k": {"dispatch_count": 2, "gpu_ns": 5.0}}, "allocation_count": 0,
                                  "allocated_bytes": 0, "gpu_busy_ns": 5.0}
    m = metrics_from_runs([r1, r2], config(1, 1))
    assert [(p["position"], p["step_ns"]["mean"]) for p in m["decode_by_position"]] == [(0, 20.0), (1, 30.0)]
    assert m["decode_kernel_gpu_ns"]["k"]["mean"] == 5.0 and m["decode_dispatch_count"]["mean"] == 2.0
    assert m["decode_gpu_idle_ns"]["mean"] == 5.0
    json.dumps(m)  # serialisable


@pytest.mark.parametrize("stdout,expected", [
    (b"1a507290862799c21d9795b56a2c5909de82b3ae\n", "1a507290862799c21d9795b56a2c5909de82b3ae"),
    (b"", None), (b"1a50729\n", None), (b"1A507290862799C21D9795B56A2C5909DE82B3AE\n", None),
    (b"HEAD\nfatal: not a git repository\n", None)])
def test_git_commit_accepts_only_a_full_hash(stdout, expected):
    assert git_commit(stdout) == expected


def test_draw_inputs_order_and_golden_prompt():
    with open(GOLDEN) as f:
        golden = json.load(f)
    golden = golden["prompt_ids"] if isinstance(golden, dict) else golden
    golden = np.asarray(golden).ravel()
    depth, prompt, start = draw_inputs(BenchConfig(prompt_token_count=512, new_token_count=1), 128256)
    assert depth.shape == (1, 0) and start is None and np.array_equal(prompt[0], golden[:512])
    # depth rows of every sequence come first, then prompt rows, from one stream
    d2, p2, _ = draw_inputs(BenchConfig(prompt_token_count=5, depth_token_count=3, batch_size=2), 128256)
    flat = np.concatenate([d2.ravel(), p2.ravel()])
    assert np.array_equal(flat, draw_inputs(BenchConfig(prompt_token_count=16, batch_size=1), 128256)[1][0])
    _, _, s3 = draw_inputs(BenchConfig(prompt_token_count=0, new_token_count=3, batch_size=2), 128256)
    assert s3.shape == (2,)
