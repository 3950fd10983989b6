"""Pins the CPU oracle before anything is checked against it.

How each oracle function is pinned:
- or_splitmix_next / below: the reference's known answers
  (src/bench/rng.rs:52-63, :66-75) and the 512 prompt ids recorded in
  benchmarks/20261018T165910Z-llama-3.2-3b-metal/report.json (golden vector).
- or_bf16_from_f32 / to_f32: the reference's RNE known answers
  (src/metal/mod.rs:1348-1434), NaN quieting (common.metal:39-41), and an
  exhaustive sweep against an independent integer formulation.
- q4 pack/unpack: a hand vector (0x76543210 -> 0..7) and round trips.
- q4 dequant: brute force over all 16 q and a sweep of bf16 s, b against
  float64 (where s*q + b is exact, so one rounding to f32 is the truth);
  special cases q=8,b=-8s -> 0; s=0 -> b; NaN/Inf propagate.
- q4 gather: the reference's index_select known answer (rows [2, 0] of a
  3 x 4 table -> [8..11, 0..3], src/metal/mod.rs:2745-2899) through a q4
  table that stores those integers, and zero rows for out-of-range ids.
- fp32 matmul: the reference's known answers (src/metal/mod.rs:2154-2236,
  :2239-2312, and the multi-tile 37x20x33 case at :2444-2540 within 1e-5).
- q4 linear (reference arithmetic): bit-equal to dequant_f32 composed with
  the pinned fp32 matmul, and the 2x3 . 3x2 known answer through q4 weights.
- linear_f64 (tolerance oracle): exact rational brute force on tiny shapes.
- generators: equal to foundry_amd.synth's vectorised form, and the stated
  distributions hold.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_splitmix_matches_reference_sequence(oracle):
    rng = oracle.SplitMix64(0)
    assert [rng.next_u64() for _ in range(3)] == [
        0xE220A8397B1DCDAF,
        0x6E789E6AA1B965F4,
        0x06C45D188009454F,
    ]


def test_splitmix_at_equals_sequential(oracle):
    rng = oracle.SplitMix64(12345)
    seq = [rng.next_u64() for _ in range(10)]
    assert seq == [oracle.splitmix_at(12345, i) for i in range(10)]


def test_below_one_is_zero(oracle):
    rng = oracle.SplitMix64(3)
    assert [rng.below(1) for _ in range(4)] == [0, 0, 0, 0]
    assert oracle.SplitMix64(3).below(0) is None


def test_prompt_ids_match_reference_report(oracle):
    with open(os.path.join(GOLDEN, "prompt_ids_seed0_vocab128256.json")) as f:
        gold = json.load(f)
    ids = oracle.gen_token_ids(gold["seed"], gold["prompt_token_count"], gold["vocab_size"])
    assert ids.tolist() == gold["prompt_ids"]
    assert ids[:3].tolist() == [100783, 9972, 106831]


def test_bf16_rne_known_answers(oracle):
    bits = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0xBF808000], dtype=np.uint32)
    assert oracle.bf16_from_f32(bits.view(np.float32)).tolist() == [0x3F80, 0x3F82, 0x3F81, 0xBF80]
    rt = oracle.bf16_to_f32(oracle.bf16_from_f32(np.array([1.0, -2.5, np.pi], dtype=np.float32)))
    assert rt.tolist() == [1.0, -2.5, 3.140625]
    ones_to_six = oracle.bf16_from_f32(np.array([1, 4, 2, 5, 3, 6], dtype=np.float32))
    assert ones_to_six.tolist() == [0x3F80, 0x4080, 0x4000, 0x40A0, 0x4040, 0x40C0]


def test_bf16_nan_is_quieted_and_inf_kept(oracle):
    snan = np.array([0x7F800001, 0xFF810000, 0x7FC00000], dtype=np.uint32).view(np.float32)
    out = oracle.bf16_from_f32(snan).tolist()
    assert out == [0x7FC0, 0xFFC1, 0x7FC0]
    inf = np.array([np.inf, -np.inf], dtype=np.float32)
    assert oracle.bf16_from_f32(inf).tolist() == [0x7F80, 0xFF80]
    # the largest finite f32 rounds up to infinity
    assert oracle.bf16_from_f32(np.array([3.4028235e38], dtype=np.float32)).tolist() == [0x7F80]


def test_bf16_rne_sweep_matches_integer_rounding(oracle):
    # independent formulation: nearest representable, ties to even mantissa
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=4000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite only
    f = bits.view(np.float32)
    got = oracle.bf16_from_f32(f)
    hi = (bits >> 16).astype(np.int64)
    rem = (bits & 0xFFFF).astype(np.int64)
    up = (rem > 0x8000) | ((rem == 0x8000) & ((hi & 1) == 1))
    want = (hi + up).astype(np.uint16)
    assert np.array_equal(got, want)


def test_q4_nibble_order_is_little_endian(oracle):
    wq = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert oracle.q4_unpack(wq, 16).tolist() == [list(range(16))]
    assert oracle.lib().or_q4_get(wq.ctypes.data_as(oracle.oracle._u32p), 16, 0, 9) == 9


def test_q4_pack_unpack_round_trip(oracle):
    rng = np.random.default_rng(1)
    wq = rng.integers(0, 2**32, size=(5, 24), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(oracle.q4_pack(oracle.q4_unpack(wq, 192)), wq)
    q = rng.integers(0, 16, size=(3, 64), dtype=np.uint8)
    assert np.array_equal(oracle.q4_unpack(oracle.q4_pack(q), 64), q)


def test_q4_dequant_brute_force(oracle):
    # bf16 scales/biases spanning small and large magnitudes, both signs
    vals = [0.0, 0.004, 0.0123, 0.02, 0.5, 1.0, 3.0, 117.0, -0.07, -1.5, 1e-30, 6e4]
    bf = oracle.bf16_from_f32(np.array(vals, dtype=np.float32))
    for s in bf:
        for b in bf:
            sf = float(oracle.bf16_to_f32(np.array([s]))[0])
            bf_ = float(oracle.bf16_to_f32(np.array([b]))[0])
            for q in range(16):
                want = np.float32(sf * q + bf_)  # float64 is exact here; one rounding
                got = oracle.q4_dequant_one(int(s), q, int(b))
                assert np.float32(got) == want, (sf, q, bf_)


def test_q4_dequant_special_cases(oracle):
    s = int(oracle.bf16_from_f32(np.array([0.015625], dtype=np.float32))[0])
    b = int(oracle.bf16_from_f32(np.array([-0.125], dtype=np.float32))[0])
    assert oracle.q4_dequant_one(s, 8, b) == 0.0  # q=8 with b=-8s
    assert oracle.q4_dequant_one(0, 13, b) == -0.125  # s=0 gives b
    nan = 0x7FC0
    assert np.isnan(oracle.q4_dequant_one(nan, 3, b))
    assert np.isnan(oracle.q4_dequant_one(s, 3, nan))
    assert oracle.q4_dequant_one(s, 3, 0x7F80) == np.inf


def test_q4_dequant_bf16_is_rne_of_f32(oracle):
    wq, s, b = oracle.gen_q4(5, 8, 128)
    f = oracle.q4_dequant_f32(wq, s, b)
    assert np.array_equal(oracle.q4_dequant_bf16(wq, s, b), oracle.bf16_from_f32(f).reshape(f.shape))
    # group mapping: element j uses scale/bias j // 64
    q = oracle.q4_unpack(wq, 128).astype(np.float64)
    sf = oracle.bf16_to_f32(s).astype(np.float64)
    bf = oracle.bf16_to_f32(b).astype(np.float64)
    want = (q * np.repeat(sf, 64, axis=1) + np.repeat(bf, 64, axis=1)).astype(np.float32)
    assert np.array_equal(f, want)


def _integer_table(oracle, values: np.ndarray, k: int):
    """q4 table whose first columns hold small integers exactly (s=1, b=0)."""
    rows = values.shape[0]
    q = np.zeros((rows, k), dtype=np.uint8)
    q[:, : values.shape[1]] = values
    one = int(oracle.bf16_from_f32(np.array([1.0], dtype=np.float32))[0])
    s = np.full((rows, k // 64), one, dtype=np.uint16)
    b = np.zeros((rows, k // 64), dtype=np.uint16)
    return oracle.q4_pack(q), s, b


def test_q4_embed_known_answer_and_zero_rows(oracle):
    wq, s, b = _integer_table(oracle, np.arange(12, dtype=np.uint8).reshape(3, 4), 64)
    rows = oracle.q4_embed(wq, s, b, np.array([2, 0], dtype=np.uint32))
    assert oracle.bf16_to_f32(rows[:, :4]).tolist() == [[8, 9, 10, 11], [0, 1, 2, 3]]
    assert not rows[:, 4:].any()
    oor = oracle.q4_embed(wq, s, b, np.array([3, 2**32 - 1], dtype=np.uint32))
    assert not oor.any()


def test_matmul_f32_known_answers(oracle):
    lhs = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    rhs = np.array([[7, 8], [9, 10], [11, 12]], dtype=np.float32)
    assert oracle.matmul_f32(lhs, rhs.T).ravel().tolist() == [58, 64, 139, 154]
    x = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    w = np.array([[1, 0, -1], [2, 1, 0]], dtype=np.float32)
    assert oracle.matmul_f32(x, w).ravel().tolist() == [-2, 4, -2, 13]


def test_matmul_f32_multi_tile(oracle):
    def pattern(count, seed):
        idx = np.arange(count, dtype=np.uint32)
        step = ((idx * seed) & 0xFFFF) + 3
        return (((step & 0xFFFF) % 17).astype(np.float32) - 8.0) / 8.0

    lhs = pattern(37 * 20, 3).reshape(37, 20)
    rhs = pattern(20 * 33, 11).reshape(20, 33)
    want = lhs.astype(np.float64) @ rhs.astype(np.float64)
    got = oracle.matmul_f32(lhs, np.ascontiguousarray(rhs.T))
    assert np.all(np.abs(got - want) <= 1e-5 * np.maximum(np.abs(want), np.finfo(np.float32).tiny))


def test_q4_linear_is_dequant_then_sequential_matmul(oracle):
    wq, s, b = oracle.gen_q4(9, 24, 192)
    x = oracle.gen_bf16_normal(10, (3, 192))
    y32, y16 = oracle.q4_linear(x, wq, s, b)
    want = oracle.matmul_f32(oracle.bf16_to_f32(x).reshape(3, 192), oracle.q4_dequant_f32(wq, s, b))
    assert np.array_equal(y32, want)
    assert np.array_equal(y16, oracle.bf16_from_f32(y32).reshape(y32.shape))
    # threads split weight rows only; results are identical
    y32t, _ = oracle.q4_linear(x, wq, s, b, threads=5)
    assert np.array_equal(y32, y32t)


def test_q4_linear_known_answer(oracle):
    # [[1,2,3],[4,5,6]] . [[7,8],[9,10],[11,12]] with K padded to 64
    w = np.array([[7, 9, 11], [8, 10, 12]], dtype=np.uint8)  # W = rhs^T, q = value
    wq, s, b = _integer_table(oracle, w, 64)
    x = np.zeros((2, 64), dtype=np.float32)
    x[:, :3] = [[1, 2, 3], [4, 5, 6]]
    y32, y16 = oracle.q4_linear(oracle.bf16_from_f32(x).reshape(2, 64), wq, s, b)
    assert y32.ravel().tolist() == [58, 64, 139, 154]
    assert oracle.bf16_to_f32(y16).ravel().tolist() == [58, 64, 139, 154]


def test_linear_f64_brute_force(oracle):
    wq, s, b = oracle.gen_q4(13, 5, 128)
    x = oracle.gen_bf16_normal(14, (2, 128))
    got = oracle.linear_f64(x, wq, s, b)
    q = oracle.q4_unpack(wq, 128)
    xf = oracle.bf16_to_f32(x).reshape(2, 128)
    sf, bf = oracle.bf16_to_f32(s), oracle.bf16_to_f32(b)
    for i in range(2):
        for r in range(5):
            exact = sum(
                Fraction(float(xf[i, j])) * (Fraction(float(sf[r, j // 64])) * int(q[r, j]) + Fraction(float(bf[r, j // 64])))
                for j in range(128)
            )
            assert abs(got[i, r] - float(exact)) <= 1e-12 * max(1.0, abs(float(exact)))
    # rows= selects weight rows (output columns)
    assert np.allclose(oracle.linear_f64(x, wq, s, b, rows=[3, 1]), got[:, [3, 1]], rtol=0, atol=0)


def test_reference_arithmetic_meets_the_tolerance(oracle):
    wq, s, b = oracle.gen_q4(15, 64, 3072)
    x = oracle.gen_bf16_normal(16, (2, 3072))
    y32, _ = oracle.q4_linear(x, wq, s, b)
    y64 = oracle.linear_f64(x, wq, s, b)
    assert np.max(np.abs(y32 - y64)) / np.max(np.abs(y64)) <= 2e-3


def test_generators_match_product_generator(oracle):
    from foundry_amd import synth

    for seed, rows, k in [(0, 3, 64), (7, 33, 3072), (2**63 + 5, 2, 128)]:
        a = oracle.gen_q4(seed, rows, k)
        bb = synth.q4_weights(seed, rows, k)
        for u, v in zip(a, bb):
            assert np.array_equal(u, v)
    assert np.array_equal(oracle.gen_bf16_normal(4, (7, 64)), synth.bf16_normal(4, (7, 64)))
    assert synth.token_ids(0, 16, 128256).tolist() == oracle.gen_token_ids(0, 16, 128256).tolist()


def test_generator_distributions(oracle):
    wq, s, b = oracle.gen_q4(3, 256, 3072)
    sf = oracle.bf16_to_f32(s)
    bf = oracle.bf16_to_f32(b)
    assert sf.min() >= 0.0039 and sf.max() <= 0.0201
    resid = bf.astype(np.float64) + 8 * sf.astype(np.float64)
    assert abs(resid.mean()) < 1e-4 and 0.8e-3 < resid.std() < 1.3e-3
    q = oracle.q4_unpack(wq, 3072)
    counts = np.bincount(q.ravel(), minlength=16) / q.size
    assert np.all(np.abs(counts - 1 / 16) < 2e-3)
    x = oracle.bf16_to_f32(oracle.gen_bf16_normal(5, (200000,)))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_golden_fixture_is_reproduced(oracle):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.build()
    with np.load(os.path.join(GOLDEN, "q4_small.npz")) as g:
        assert sorted(g.files) == sorted(fresh)
        for name in g.files:
            assert np.array_equal(g[name], fresh[name]), name


@pytest.mark.parametrize("mistake", ["transpose", "drop_bias", "wrong_group"])
def test_planted_mistakes_are_caught(oracle, mistake):
    """A plausible oracle bug, planted on the CPU, fails the fp64 comparison."""
    wq, s, b = oracle.gen_q4(17, 64, 256)
    x = oracle.gen_bf16_normal(18, (64, 256))
    good = oracle.linear_f64(x, wq, s, b)
    w = oracle.q4_dequant_f32(wq, s, b).astype(np.float64)
    xf = oracle.bf16_to_f32(x).reshape(64, 256).astype(np.float64)
    if mistake == "transpose":
        bad = (xf @ w.T).T
    elif mistake == "drop_bias":
        q = oracle.q4_unpack(wq, 256).astype(np.float64)
        bad = xf @ (q * np.repeat(oracle.bf16_to_f32(s), 64, axis=1)).T
    else:
        # group index taken in the wrong order along K
        q = oracle.q4_unpack(wq, 256).astype(np.float64)
        sf = np.repeat(oracle.bf16_to_f32(s)[:, ::-1], 64, axis=1)
        bf = np.repeat(oracle.bf16_to_f32(b)[:, ::-1], 64, axis=1)
        bad = xf @ (q * sf + bf).T
    assert np.max(np.abs(bad - good)) / np.max(np.abs(good)) > 2e-3
