"""Pins of the decoder restatement (oracle/llama_ref.py), the checker of the
HIP decoder. Each check is a reference test restated (file:line), a closed
form, or a planted mistake that must fail."""
import math

import numpy as np
import pytest

from oracle import llama_ref as R

LLAMA3 = (32.0, 1.0, 4.0, 8192)


def test_inv_freq_follow_the_llama3_formula_in_each_band():
    """src/models/llama/rotary_emb.rs:203-239: indices 0, 32 and 63 of head
    dim 128, theta 500000 (one per band) within 1e-5 of the float64 formula."""
    f = R.inv_freq(128, 500000.0, LLAMA3)
    assert len(f) == 64
    for j in (0, 32, 63):
        period = 500000.0 ** (j * 2.0 / 128.0)
        wavelen = 2 * math.pi * period
        period_scaled = 32.0 * period if wavelen > 8192.0 else period
        smooth = (8192.0 / wavelen - 1.0) / (4.0 - 1.0)
        period_expected = period_scaled / ((1.0 - smooth) / 32.0 + smooth) if 2048.0 < wavelen < 8192.0 \
            else period_scaled
        expected = 1.0 / period_expected
        assert abs(float(f[j]) - expected) <= 1e-5 * expected, j


def test_inv_freq_without_scaling_are_powers_of_theta():
    """src/models/llama/rotary_emb.rs:241-259."""
    f = R.inv_freq(64, 100000.0, None)
    assert len(f) == 32
    for j in (0, 16, 31):
        expected = 100000.0 ** (-(j * 2.0 / 64.0))
        assert abs(float(f[j]) - expected) <= 1e-5 * expected


def test_angles_repeat_the_frequencies_for_both_halves():
    """src/models/llama/rotary_emb.rs:276-285."""
    got = R.angles([1.0, 0.5], 3).ravel().tolist()
    assert got == [0.0, 0.0, 0.0, 0.0, 1.0, 0.5, 1.0, 0.5, 2.0, 1.0, 2.0, 1.0]


def test_rope_tables_are_rounded_cos_and_sin():
    cos, sin = R.rope_tables(8, 10000.0, None, 5)
    ang = R.angles(R.inv_freq(8, 10000.0, None), 5).astype(np.float64)
    assert np.all(np.abs(cos - np.cos(ang)) <= 2.0 ** -8 * np.maximum(np.abs(np.cos(ang)), 2.0 ** -126))
    assert np.all(np.abs(sin - np.sin(ang)) <= 2.0 ** -8 * np.maximum(np.abs(np.sin(ang)), 2.0 ** -126))
    assert np.array_equal(cos[0], np.ones(8, np.float32)) and not sin[0].any()


def test_rne_matches_the_c_oracle(oracle):
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x7F800001, 0xFFC12345, 0x3F808000, 0x3F818000, 0x7F7FFFFF], np.uint32)])
    vals = bits.view(np.float32)
    got = (R.rne(vals).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(got, oracle.bf16_from_f32(vals))


def test_rms_norm_closed_form_and_planted_mistakes():
    """x = c (all equal), eps = 0: scale = 1/|c|, x*scale = +-1 exactly, so
    y = RNE(w). A random row agrees with float64 to one bf16 ulp; a sum in
    place of the mean, a missing sqrt or a skipped rounding of h * scale do
    not, and on a row of tiny values (where eps dominates) neither does eps
    moved outside the sqrt."""
    w = R.rne(np.linspace(0.5, 1.5, 64, dtype=np.float32))
    assert np.array_equal(R.rms_norm(np.full((1, 64), -2.0, np.float32), w, 0.0), -w[None, :])
    rng = np.random.default_rng(1)
    h = R.rne(rng.standard_normal((3, 3072)).astype(np.float32))
    wn = R.rne((1 + 0.1 * rng.standard_normal(3072)).astype(np.float32))
    got = R.rms_norm(h, wn, 1e-5).astype(np.float64)
    h64 = h.astype(np.float64)

    def ref64(scale, hh=h64, round_mid=True):
        mid = (hh * scale).astype(np.float32)
        return R.rne((R.rne(mid) if round_mid else mid) * wn).astype(np.float64)

    def ulp(v):
        return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126))) - 7)

    ms = (h64 * h64).mean(axis=-1, keepdims=True)
    good = ref64(1.0 / np.sqrt(ms + 1e-5))
    assert np.all(np.abs(got - good) <= ulp(got)) and np.mean(got == good) >= 0.99
    for bad in (ref64(1.0 / np.sqrt((h64 * h64).sum(axis=-1, keepdims=True) + 1e-5)),
                ref64(1.0 / np.sqrt(ms + 1e-5), round_mid=False)):
        assert np.mean(got == bad) < 0.9
    # a missing sqrt, on a row whose mean square is far from 1
    h3 = R.rne(3 * h)
    got3 = R.rms_norm(h3, wn, 1e-5).astype(np.float64)
    ms3 = (h3.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    assert np.mean(got3 == ref64(1.0 / np.sqrt(ms3 + 1e-5), h3.astype(np.float64))) >= 0.99
    assert np.mean(got3 == ref64(1.0 / (ms3 + 1e-5), h3.astype(np.float64))) < 0.9
    # eps outside the sqrt, on a row of tiny values where eps dominates
    tiny = R.rne(1e-3 * rng.standard_normal((1, 3072)).astype(np.float32))
    got_t = R.rms_norm(tiny, wn, 1e-5).astype(np.float64)
    t64 = tiny.astype(np.float64)
    ms_t = (t64 * t64).mean(axis=-1, keepdims=True)
    assert np.mean(got_t == ref64(1.0 / np.sqrt(ms_t + 1e-5), t64)) >= 0.99
    assert np.mean(got_t == ref64(1.0 / np.sqrt(ms_t) + 1e-5, t64)) < 0.9


def test_silu_mul_known_values():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0], np.float32)
    u = np.ones_like(g)
    expected = g / (1.0 + np.exp(-g.astype(np.float64)))
    got = R.silu_mul(g, u)
    assert got[0] == 0.0 and got[3] == 20.0
    assert np.all(np.abs(got - expected) <= 2.0 ** -8 * np.maximum(np.abs(expected), 1e-30))


def test_sdpa_closed_forms():
    rng = np.random.default_rng(2)
    v = R.rne(rng.standard_normal((5, 16)).astype(np.float32))
    k = R.rne(rng.standard_normal((5, 16)).astype(np.float32))
    q = R.rne(rng.standard_normal((1, 16)).astype(np.float32))
    # one key: p = 1, out = v
    assert np.array_equal(R.sdpa(q, k[:1], v[:1], [0], 0.25), v[:1])
    # q = 0: every score 0, p = RNE(1/n), out = RNE(p * sum v)
    out = R.sdpa(np.zeros((1, 16), np.float32), k, v, [4], 0.25)
    want = R.rne((R.rne(np.float32(1 / 5)) * v.astype(np.float64).sum(axis=0)).astype(np.float32))
    assert np.max(np.abs(out - want)) <= 2.0 ** -7 * np.max(np.abs(want))
    # causal: keys past the position do not matter
    k2, v2 = k.copy(), v.copy()
    k2[3:], v2[3:] = 100.0, -100.0
    assert np.array_equal(R.sdpa(q, k, v, [2], 0.25), R.sdpa(q, k2, v2, [2], 0.25))


def test_argmax_and_top_ids_tie_rules():
    """src/metal/mod.rs:2038-2096 (first index on ties, also across threads)
    and src/eval/generation.rs:241-257 (top-k by value, then lowest id)."""
    assert R.argmax([3.0, 7.0, 7.0, 1.0]) == 1
    x = np.array([9.0 if i in (10, 300) else float(i % 7) for i in range(600)], np.float32)
    assert R.argmax(x) == 10
    assert R.top_ids([-1.0, -0.5, -0.5, -3.0], 3) == [1, 2, 0]


def test_compare_generation_reference_cases():
    """src/eval/generation.rs:259-431, with top-k entries as ids."""
    c = R.compare_generation
    r = c([7, 8], [[7], [8]], [7, 8], [[7], [8]])
    assert (r["compared_tokens"], r["matched_tokens"], r["first_divergence"], r["close"]) == (2, 2, None, True)
    r = c([16543, 1], [[16543, 220], [1]], [220, 83017], [[220, 16543], [83017]])
    assert (r["matched_tokens"], r["first_divergence"], r["close"]) == (0, 0, True)
    assert not c([9], [[9, 5]], [5], [[5, 6]])["close"]
    assert not c([6], [[6, 7]], [5], [[5, 6]])["close"]
    r = c([2], [[2]], [2, 4, 4], [[2], [4], [4]])
    assert (r["compared_tokens"], r["matched_tokens"], r["close"]) == (1, 1, True)
    r = c([4], [[4]], [], [])
    assert (r["compared_tokens"], r["close"]) == (0, False)
