"""GPU parity of the q4 path against the CPU oracle, through the C-ABI.

Bars (written into each check):
- fh_q4_dequant and fh_q4_embed: bit-exact against the oracle.
- fh_q4_matmul, fp32 output: max|y - y64| / max|y64| <= 2e-3 against the fp64
  dequant-then-matmul oracle. (The decode GEMV keeps every weight exact in
  fp32 and lands near 1e-6; the GEMM feeds the matrix cores the bf16 weight
  RNE(s*q + b) and lands near 1e-3.)
- bf16 output: bit-identical to RNE of the same kernel's fp32 output, and
  within 1 bf16 ulp of the fp64 value plus the fp32 bound above.
Full-size configs that the fp64 oracle cannot hold whole are compared on a
seeded sample of output rows/columns.
"""
import ctypes
import os

import numpy as np
import pytest

from foundry_amd import _lib, synth
from foundry_amd.device import HipDevice
from foundry_amd.nn import Q4Embedding, Q4Linear, Q4Weight
from foundry_amd.primitive import DType
from foundry_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

FP32_BOUND = 2e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4_small.npz")


def assert_bf16_identical(got, want):
    """Bit-exact for every non-NaN value; NaN in the same places and quiet.
    Which NaN an invalid operation or two NaN operands produce (payload, sign)
    is left open by IEEE 754 and differs between x86 and CDNA, so NaN bits
    are not compared."""
    got_nan = ((got & 0x7F80) == 0x7F80) & ((got & 0x7F) != 0)
    want_nan = ((want & 0x7F80) == 0x7F80) & ((want & 0x7F) != 0)
    assert np.array_equal(got_nan, want_nan), "NaN positions differ"
    assert np.all(got[got_nan] & 0x40), "a NaN output is not quiet"
    assert np.array_equal(got[~got_nan], want[~want_nan]), "non-NaN values differ"


def up(dev, arr, dtype):
    return Tensor.from_numpy(dev, arr, dtype)


def weight(dev, wq, s, b):
    return Q4Weight(up(dev, wq, DType.U32), up(dev, s, DType.BF16), up(dev, b, DType.BF16))


def matmul_raw(dev, x_t, w: Q4Weight, m, k, x_ld, y_dtype):
    n = w.out_features
    item = 4 if y_dtype == _lib.F32 else 2
    out = dev.empty(max(m * n * item, 1))
    _lib.call("fh_q4_matmul", dev.handle, ctypes.c_void_p(x_t.storage.ptr), m, k, x_ld,
              ctypes.c_void_p(w.wq.storage.ptr), ctypes.c_void_p(w.scales.storage.ptr),
              ctypes.c_void_p(w.biases.storage.ptr), n, 64, ctypes.c_void_p(out.ptr), y_dtype)
    raw = np.empty(m * n * item, dtype=np.uint8)
    if raw.size:
        _lib.call("fh_download", dev.handle, raw.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(out.ptr), raw.size)
    return raw.view(np.float32 if y_dtype == _lib.F32 else np.uint16).reshape(m, n)


def bf16_ulp(v):
    a = np.abs(v).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 2.0**-126)))
    return 2.0 ** (e - 7)


def check_matmul(y32, y16, y64, bound=FP32_BOUND):
    scale = float(np.max(np.abs(y64))) or 1.0
    err32 = float(np.max(np.abs(y32.astype(np.float64) - y64))) / scale
    assert err32 <= bound, f"fp32 rel err {err32:.3e} > {bound}"
    assert np.array_equal(y16, synth.bf16_rne(y32)), "bf16 output is not RNE of the fp32 result"
    err16 = np.abs(synth.bf16_to_f32(y16).astype(np.float64) - y64)
    assert np.all(err16 <= bf16_ulp(y64) + bound * scale), "bf16 output beyond 1 ulp + bound"
    return err32


def run_linear(dev, oracle, m, n, k, seed, x_ld=None, sample=None):
    wq, s, b = synth.q4_weights(seed, n, k)
    x_ld = x_ld or k
    x = synth.bf16_normal(seed + 1, (m, x_ld))
    w = weight(dev, wq, s, b)
    xt = up(dev, x, DType.BF16)
    y32 = matmul_raw(dev, xt, w, m, k, x_ld, _lib.F32)
    y16 = matmul_raw(dev, xt, w, m, k, x_ld, _lib.BF16)
    xs = x[:, :k]
    if sample is None:
        y64 = oracle.linear_f64(xs, wq, s, b)
        return check_matmul(y32, y16, y64)
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(m, size=min(m, sample[0]), replace=False))
    cols = np.sort(rng.choice(n, size=min(n, sample[1]), replace=False))
    y64 = oracle.linear_f64(np.ascontiguousarray(xs[rows]), wq, s, b, rows=cols)
    return check_matmul(y32[np.ix_(rows, cols)], y16[np.ix_(rows, cols)], y64)


# ---------------- dequant and gather: bit-exact ----------------

def test_dequant_golden_and_config_shape(device, oracle):
    with np.load(GOLDEN) as g:
        for case in ("gemv", "gemm"):
            wq, s, b = g[f"{case}_wq"], g[f"{case}_s"], g[f"{case}_b"]
            out = dev_dequant(device, wq, s, b)
            assert np.array_equal(out, g[f"{case}_deq"])
    wq, s, b = synth.q4_weights(101, 8192, 3072)
    assert np.array_equal(dev_dequant(device, wq, s, b), oracle.q4_dequant_bf16(wq, s, b))


def dev_dequant(dev, wq, s, b):
    rows, k = wq.shape[0], wq.shape[1] * 8
    w = weight(dev, wq, s, b)
    out = dev.empty(rows * k * 2)
    _lib.call("fh_q4_dequant", dev.handle, ctypes.c_void_p(w.wq.storage.ptr),
              ctypes.c_void_p(w.scales.storage.ptr), ctypes.c_void_p(w.biases.storage.ptr),
              rows, k, 64, ctypes.c_void_p(out.ptr))
    raw = np.empty(rows * k, dtype=np.uint16)
    _lib.call("fh_download", dev.handle, raw.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(out.ptr), raw.nbytes)
    return raw.reshape(rows, k)


def test_dequant_special_values(device, oracle):
    specials = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0x0001, 0x7F7F, 0x3C80, 0xBC80,
                         0x4700, 0xC2F0, 0x3B83, 0x0080, 0x8001, 0x3F80], dtype=np.uint16)
    rows = 16
    r = np.arange(rows)
    s = np.stack([specials[r], specials[(r + 7) % 16]], axis=1).astype(np.uint16)
    b = np.stack([specials[(r + 3) % 16], specials[(r * 5 + 1) % 16]], axis=1).astype(np.uint16)
    wq = synth.q4_weights(5, rows, 128)[0]
    got = dev_dequant(device, wq, s, b)
    want = oracle.q4_dequant_bf16(wq, s, b)
    assert_bf16_identical(got, want)
    # every (s, b) pair of the specials with all 16 q values, one group per row
    s2 = np.repeat(specials, 16).reshape(256, 1).copy()
    b2 = np.tile(specials, 16).reshape(256, 1).copy()
    wq2 = oracle.q4_pack(np.tile(np.arange(64) % 16, (256, 1)).astype(np.uint8))
    assert_bf16_identical(dev_dequant(device, wq2, s2, b2), oracle.q4_dequant_bf16(wq2, s2, b2))


def test_embed_golden(device):
    with np.load(GOLDEN) as g:
        emb = Q4Embedding(weight(device, g["gemv_wq"], g["gemv_s"], g["gemv_b"]))
        ids = up(device, g["embed_ids"], DType.U32)
        rows = emb.forward(device, ids).to_numpy(device)
        assert rows.shape == (g["embed_ids"].size, 128)
        assert np.array_equal(rows, g["embed_rows"])


def test_embed_known_answer(device, oracle):
    q = np.zeros((3, 64), dtype=np.uint8)
    q[:, :4] = np.arange(12).reshape(3, 4)
    wq = oracle.q4_pack(q)
    s = np.full((3, 1), 0x3F80, dtype=np.uint16)
    b = np.zeros((3, 1), dtype=np.uint16)
    emb = Q4Embedding(weight(device, wq, s, b))
    rows = emb.forward(device, up(device, np.array([2, 0, 3], dtype=np.uint32), DType.U32)).to_numpy(device)
    assert synth.bf16_to_f32(rows[:, :4]).tolist() == [[8, 9, 10, 11], [0, 1, 2, 3], [0, 0, 0, 0]]
    assert not rows[:, 4:].any()


@pytest.mark.parametrize("batch", [1, 64, 4096])
def test_embed_config2_full_table(device, oracle, batch, _config2_table):
    wq, s, b, w = _config2_table
    ids = synth.token_ids(batch, batch, 128256)
    if batch >= 64:  # edge ids: first, last, just past the end, max u32
        ids[:4] = [0, 128255, 128256, 2**32 - 1]
    out = Q4Embedding(w).forward(device, up(device, ids.reshape(1, -1), DType.U32)).to_numpy(device)
    assert out.shape == (1, batch, 3072)
    assert np.array_equal(out[0], oracle.q4_embed(wq, s, b, ids))


@pytest.mark.parametrize("k", [3072, 4096])
def test_gather_wave_rows_specials_and_tails(device, oracle, k):
    """The row-per-wavefront gather (k = 3072, 4096; at least 4 rows per CU):
    special scale and bias values (zeros, infinities, NaNs, denormals) bit for
    bit, 1029 ids (a partial last block) with ids past the table, and the
    materialised dequant of the same 1100-row table; then 13 ids of the same
    table (the per-word kernel of small batches)."""
    specials = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0x0001, 0x7F7F, 0x3C80, 0xBC80,
                         0x4700, 0xC2F0, 0x3B83, 0x0080, 0x8001, 0x3F80], dtype=np.uint16)
    rows, g = 1100, k // 64
    wq, s, b = synth.q4_weights(17 + k, rows, k)
    s[::3] = specials[np.arange(rows * g).reshape(rows, g)[::3] % 16]
    b[1::4] = specials[(np.arange(rows * g).reshape(rows, g)[1::4] * 7 + 3) % 16]
    assert_bf16_identical(dev_dequant(device, wq, s, b), oracle.q4_dequant_bf16(wq, s, b))
    ids = (synth.token_ids(k, 1029, 1200) % 1200).astype(np.uint32)
    ids[:5] = [0, rows - 1, rows, 2**32 - 1, 7]
    w = weight(device, wq, s, b)
    for sel in (ids, ids[:13]):
        out = Q4Embedding(w).forward(device, up(device, sel.reshape(1, -1), DType.U32))
        assert_bf16_identical(out.to_numpy(device)[0], oracle.q4_embed(wq, s, b, sel))


@pytest.fixture(scope="module")
def _config2_table(device):
    wq, s, b = synth.q4_weights(2, 128256, 3072)
    return wq, s, b, weight(device, wq, s, b)


def test_embed_empty(device):
    wq, s, b = synth.q4_weights(3, 8, 64)
    emb = Q4Embedding(weight(device, wq, s, b))
    out = emb.forward(device, up(device, np.zeros((0,), dtype=np.uint32), DType.U32))
    assert out.shape == (0, 64)


@pytest.mark.parametrize("k", [3072, 4096])
def test_embed_empty_table_writes_zero_rows(device, k):
    """A table of 0 rows makes every id out of range: each output row is zero
    (index_select_rows, src/metal/kernels/index_select.metal:11-29), and no
    table byte is read. 1024 ids is past the row count at which the gather
    takes its one-wavefront-per-row kernel for k = 3072 and 4096."""
    n_ids = 1024
    ids = np.arange(n_ids, dtype=np.uint32)
    ids_t = up(device, ids, DType.U32)
    table = device.empty(256)  # a live allocation that the call must not read
    out = device.empty(n_ids * k * 2)
    sentinel = np.full(n_ids * k, 0x7FC1, dtype=np.uint16)
    _lib.call("fh_upload", device.handle, ctypes.c_void_p(out.ptr), sentinel.ctypes.data_as(ctypes.c_void_p),
              sentinel.nbytes)
    _lib.call("fh_q4_embed", device.handle, ctypes.c_void_p(table.ptr), ctypes.c_void_p(table.ptr),
              ctypes.c_void_p(table.ptr), 0, k, 64, ctypes.c_void_p(ids_t.storage.ptr), n_ids,
              ctypes.c_void_p(out.ptr))
    got = np.empty(n_ids * k, dtype=np.uint16)
    _lib.call("fh_download", device.handle, got.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(out.ptr), got.nbytes)
    assert not got.any(), "an empty table must give all-zero rows"


# ---------------- GEMV (m <= 8) ----------------

@pytest.mark.parametrize(
    "m,n,k",
    [(1, 8192, 3072), (1, 3072, 8192), (1, 1000, 64), (1, 1024, 3072), (3, 40, 128),
     (2, 4096, 4096), (4, 333, 192), (8, 14336, 4096), (8, 4096, 14336), (5, 3072, 8192),
     (7, 129, 1024), (1, 17, 30720), (6, 256, 10240), (8, 512, 24576), (5, 128, 14336), (3, 64, 24576)],
)
def test_gemv_parity(device, oracle, m, n, k):
    err = run_linear(device, oracle, m, n, k, seed=1000 + m * 7 + n + k)
    assert err < 1e-4, f"GEMV keeps exact weights; rel err {err:.2e} suggests a wrong term"


def test_gemv_config1_and_lm_head_sampled(device, oracle):
    run_linear(device, oracle, 1, 8192, 3072, seed=1)
    run_linear(device, oracle, 1, 128256, 3072, seed=2, sample=(1, 4096))


def test_gemv_golden(device):
    with np.load(GOLDEN) as g:
        w = weight(device, g["gemv_wq"], g["gemv_s"], g["gemv_b"])
        x = up(device, g["gemv_x"], DType.BF16)
        m, k = g["gemv_x"].shape
        y32 = matmul_raw(device, x, w, m, k, k, _lib.F32)
        y16 = matmul_raw(device, x, w, m, k, k, _lib.BF16)
        check_matmul(y32, y16, g["gemv_y64"])


@pytest.mark.parametrize("m,n,k,x_ld", [(3, 512, 1024, 1024 + 64), (8, 256, 14336, 14336 + 128)])
def test_gemv_strided_x(device, oracle, m, n, k, x_ld):
    run_linear(device, oracle, m, n, k, seed=77, x_ld=x_ld)


# ---------------- GEMM (m > 8) ----------------

@pytest.mark.parametrize(
    "m,n,k", [(9, 128, 64), (20, 72, 256), (130, 200, 320), (256, 256, 3072), (512, 1000, 1024), (64, 64, 8192)]
)
def test_gemm_parity(device, oracle, m, n, k):
    run_linear(device, oracle, m, n, k, seed=2000 + m + n + k)


def test_gemm_config3_shapes_sampled(device, oracle):
    run_linear(device, oracle, 2048, 8192, 3072, seed=3, sample=(96, 8192))
    run_linear(device, oracle, 2048, 3072, 8192, seed=4, sample=(96, 3072))


# Shapes with at least one 256 x 256 tile per CU take the direct-weight
# kernel (q4_gemm_direct.hip) when k is a multiple of 512, else the LDS-staged
# one (q4_gemm.hip, k = 1920): ragged last tile rows and columns (rows past m
# and weight rows past n are read clamped and never stored), a row stride
# above k, and the 8B-shape prefill's gate/up and down widths. Rows compared:
# the first 16 and the last 48 (the ragged tile), every column.
@pytest.mark.parametrize("m,n,k,x_ld", [(2085, 8288, 1024, 1024), (2048, 8192, 1024, 1096),
                                        (4096, 14336, 512, 512), (4096, 4096, 1920, 1920)])
def test_gemm_full_chip_ragged_and_strided(device, oracle, m, n, k, x_ld):
    seed = 7000 + m + n + k
    wq, s, b = synth.q4_weights(seed, n, k)
    x = synth.bf16_normal(seed + 1, (m, x_ld))
    w = weight(device, wq, s, b)
    xt = up(device, x, DType.BF16)
    y32 = matmul_raw(device, xt, w, m, k, x_ld, _lib.F32)
    y16 = matmul_raw(device, xt, w, m, k, x_ld, _lib.BF16)
    rows = np.concatenate([np.arange(16), np.arange(m - 48, m)])
    y64 = oracle.linear_f64(np.ascontiguousarray(x[rows, :k]), wq, s, b)
    check_matmul(y32[rows], y16[rows], y64)


# Prompt-length GEMMs with fewer 256 x 256 tiles than CUs: the direct-weight
# kernel over two K ranges (2048 x 3072 x 8192, ragged 2000 x 3000 x 8192,
# 512 x 16384 x 3072) or the LDS-staged kernel split over K (1024 x 4096 x
# 8192), the ranges' f32 partials added in order by the reduce kernel. Rows
# compared: the first 16, 32 sampled, the last 48; every column. A second
# run is bit-identical.
@pytest.mark.parametrize("m,n,k", [(2048, 3072, 8192), (2000, 3000, 8192), (512, 16384, 3072), (1024, 4096, 8192)])
def test_gemm_split_ranges_sampled_and_repeatable(device, oracle, m, n, k):
    seed = 9000 + m + n + k
    wq, s, b = synth.q4_weights(seed, n, k)
    x = synth.bf16_normal(seed + 1, (m, k))
    w = weight(device, wq, s, b)
    xt = up(device, x, DType.BF16)
    y32 = matmul_raw(device, xt, w, m, k, k, _lib.F32)
    y16 = matmul_raw(device, xt, w, m, k, k, _lib.BF16)
    again = matmul_raw(device, xt, w, m, k, k, _lib.F32)
    assert np.array_equal(y32.view(np.uint32), again.view(np.uint32)), "split-K sums differ between runs"
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([np.arange(16), rng.integers(16, m - 48, 32), np.arange(m - 48, m)]))
    y64 = oracle.linear_f64(np.ascontiguousarray(x[rows]), wq, s, b)
    check_matmul(y32[rows], y16[rows], y64)


# Prompt-length rows whose tiles leave CUs idle split K (up to 8 ranges of
# at least 4 steps, f32 partials added in order): the config-4 prefill's
# down (5 splits) and q/k/v (3 splits) shapes, and m * n not a multiple of 4
# (the reduce's scalar tail).
@pytest.mark.parametrize("m,n,k", [(512, 3072, 8192), (512, 5120, 3072), (35, 198, 2048)])
def test_gemm_split_k(device, oracle, m, n, k):
    run_linear(device, oracle, m, n, k, seed=5000 + m + n, sample=(64, n) if m > 64 else None)


def test_gemm_golden(device):
    with np.load(GOLDEN) as g:
        w = weight(device, g["gemm_wq"], g["gemm_s"], g["gemm_b"])
        x = up(device, g["gemm_x"], DType.BF16)
        m, k = g["gemm_x"].shape
        y32 = matmul_raw(device, x, w, m, k, k, _lib.F32)
        y16 = matmul_raw(device, x, w, m, k, k, _lib.BF16)
        check_matmul(y32, y16, g["gemm_y64"])


def test_gemm_strided_x(device, oracle):
    run_linear(device, oracle, 40, 256, 512, seed=78, x_ld=512 + 8)


def test_zero_k_and_zero_m(device):
    w = weight(device, np.zeros((16, 0), dtype=np.uint32), np.zeros((16, 0), dtype=np.uint16),
               np.zeros((16, 0), dtype=np.uint16))
    for m in (1, 20):
        x = up(device, np.zeros((m, 8), dtype=np.uint16), DType.BF16)
        y = matmul_raw(device, x, w, m, 0, 8, _lib.F32)
        assert y.shape == (m, 16) and not y.any()
    wq, s, b = synth.q4_weights(9, 16, 64)
    x = up(device, np.zeros((1, 64), dtype=np.uint16), DType.BF16)
    assert matmul_raw(device, x, weight(device, wq, s, b), 0, 64, 64, _lib.BF16).shape == (0, 16)


# ---------------- modules, errors, batching, profiling ----------------

def test_q4_linear_module_shapes(device, oracle):
    wq, s, b = synth.q4_weights(31, 96, 256)
    x = synth.bf16_normal(32, (2, 3, 256))
    lin = Q4Linear(weight(device, wq, s, b))
    y = lin.forward(device, up(device, x, DType.BF16)).to_numpy(device)
    assert y.shape == (2, 3, 96)
    y64 = oracle.linear_f64(x.reshape(6, 256), wq, s, b).reshape(2, 3, 96)
    err = np.abs(synth.bf16_to_f32(y).astype(np.float64) - y64)
    assert np.all(err <= bf16_ulp(y64) + 1e-5 * np.max(np.abs(y64)))


@pytest.mark.parametrize("rows", [3, 12])  # the GEMV and the GEMM route
def test_q4_matmul_op_stages_views_it_cannot_read_in_place(device, rows):
    """A transposed x (column stride != 1) and a broadcast x (row stride 0)
    are copied to contiguous rows first (the reference's matmul operand rule),
    so they give exactly what the same rows give when stored contiguously."""
    from foundry_amd.primitive import QuantizedMatmul

    wq, s, b = synth.q4_weights(33, 96, 256)
    w = weight(device, wq, s, b)
    op = QuantizedMatmul(bits=4, group=64)
    x = synth.bf16_normal(34, (rows, 256))
    want = up(device, x, DType.BF16).apply(device, op, [w.wq, w.scales, w.biases]).to_numpy(device)
    xt = up(device, np.ascontiguousarray(x.T), DType.BF16).permute((1, 0))
    assert xt.layout.strides == (1, rows)
    got = xt.apply(device, op, [w.wq, w.scales, w.biases]).to_numpy(device)
    assert np.array_equal(got, want)
    row = up(device, x[:1], DType.BF16).expand((rows, 256))
    assert row.layout.strides == (0, 1)
    got = row.apply(device, op, [w.wq, w.scales, w.biases]).to_numpy(device)
    one = up(device, np.repeat(x[:1], rows, axis=0), DType.BF16)
    assert np.array_equal(got, one.apply(device, op, [w.wq, w.scales, w.biases]).to_numpy(device))


def test_foreign_and_out_of_bounds_storage_are_rejected(device):
    wq, s, b = synth.q4_weights(41, 64, 128)
    w = weight(device, wq, s, b)
    x = up(device, synth.bf16_normal(42, (1, 128)), DType.BF16)
    other = HipDevice(0)
    try:
        xo = up(other, synth.bf16_normal(42, (1, 128)), DType.BF16)
        with pytest.raises(_lib.HipError) as e:
            matmul_raw(device, xo, w, 1, 128, 128, _lib.BF16)
        assert e.value.status == _lib.ERR_FOREIGN_STORAGE
    finally:
        del xo
        other.close()
    out = device.empty(65 * 2)
    with pytest.raises(_lib.HipError) as e:  # n=65 rows do not fit a 64-row weight
        _lib.call("fh_q4_matmul", device.handle, ctypes.c_void_p(x.storage.ptr), 1, 128, 128,
                  ctypes.c_void_p(w.wq.storage.ptr), ctypes.c_void_p(w.scales.storage.ptr),
                  ctypes.c_void_p(w.biases.storage.ptr), 65, 64, ctypes.c_void_p(out.ptr), _lib.BF16)
    assert e.value.status == _lib.ERR_OUT_OF_BOUNDS
    with pytest.raises(_lib.HipError) as e:
        _lib.call("fh_q4_matmul", device.handle, ctypes.c_void_p(x.storage.ptr), 1, 128, 128,
                  ctypes.c_void_p(w.wq.storage.ptr), ctypes.c_void_p(w.scales.storage.ptr),
                  ctypes.c_void_p(w.biases.storage.ptr), 64, 32, ctypes.c_void_p(out.ptr), _lib.BF16)
    assert e.value.status == _lib.ERR_UNSUPPORTED
    # validation errors launch nothing and are not sticky
    y = matmul_raw(device, x, w, 1, 128, 128, _lib.BF16)
    assert y.shape == (1, 64)


def test_graph_replay_matches_eager(device):
    wq, s, b = synth.q4_weights(51, 512, 1024)
    w = weight(device, wq, s, b)
    xs = {m: up(device, synth.bf16_normal(52 + m, (m, 1024)), DType.BF16) for m in (1, 4, 64)}
    ids = up(device, np.array([5, 511, 512, 0], dtype=np.uint32), DType.U32)
    outs = {m: device.empty(m * 512 * 2) for m in xs}
    emb_out = device.empty(4 * 1024 * 2)

    def enqueue():
        for m, xt in xs.items():
            _lib.call("fh_q4_matmul", device.handle, ctypes.c_void_p(xt.storage.ptr), m, 1024, 1024,
                      ctypes.c_void_p(w.wq.storage.ptr), ctypes.c_void_p(w.scales.storage.ptr),
                      ctypes.c_void_p(w.biases.storage.ptr), 512, 64, ctypes.c_void_p(outs[m].ptr), _lib.BF16)
        _lib.call("fh_q4_embed", device.handle, ctypes.c_void_p(w.wq.storage.ptr),
                  ctypes.c_void_p(w.scales.storage.ptr), ctypes.c_void_p(w.biases.storage.ptr),
                  512, 1024, 64, ctypes.c_void_p(ids.storage.ptr), 4, ctypes.c_void_p(emb_out.ptr))

    def read():
        res = {}
        for m, st in list(outs.items()) + [("emb", emb_out)]:
            raw = np.empty(st.nbytes, dtype=np.uint8)
            _lib.call("fh_download", device.handle, raw.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(st.ptr), raw.size)
            res[m] = raw
        return res

    enqueue()
    eager = read()
    device.capture_begin()
    enqueue()
    graph = device.capture_end()
    for _ in range(3):
        for st in list(outs.values()) + [emb_out]:  # clobber between replays
            junk = np.full(st.nbytes, 0xAB, dtype=np.uint8)
            _lib.call("fh_upload", device.handle, ctypes.c_void_p(st.ptr), junk.ctypes.data_as(ctypes.c_void_p), junk.size)
        graph.launch()
        device.synchronize()
        got = read()
        for key in eager:
            assert np.array_equal(got[key], eager[key]), key


def _live_bytes(dev) -> int:
    """Bytes the device holds now: the run peak right after a reset."""
    dev.reset_run_memory_peak()
    return dev.run_memory_peak()["bytes"]


def _alloc(dev, nbytes):
    p = ctypes.c_void_p()
    _lib.call("fh_alloc", dev.handle, nbytes, 0, ctypes.byref(p))
    return p.value


def test_graph_retains_allocations_freed_before_or_during_capture_end():
    """A graph keeps every allocation its ops touched: freeing one after
    capture (or during it) retires it until the graph is destroyed, so a
    replay never reads freed memory. A free during capture of memory the graph
    does not use happens at capture end."""
    dev = HipDevice(0)
    try:
        wq, s, b = synth.q4_weights(71, 512, 1024)
        x = synth.bf16_normal(72, (1, 1024))
        ptrs = {}
        for name, arr in (("wq", wq), ("s", s), ("b", b), ("x", x)):
            ptrs[name] = _alloc(dev, arr.nbytes)
            _lib.call("fh_upload", dev.handle, ctypes.c_void_p(ptrs[name]), arr.ctypes.data_as(ctypes.c_void_p),
                      arr.nbytes)
        y = _alloc(dev, 512 * 4)
        unused = _alloc(dev, 1 << 20)

        def gemv():
            _lib.call("fh_q4_matmul", dev.handle, ctypes.c_void_p(ptrs["x"]), 1, 1024, 1024,
                      ctypes.c_void_p(ptrs["wq"]), ctypes.c_void_p(ptrs["s"]), ctypes.c_void_p(ptrs["b"]), 512, 64,
                      ctypes.c_void_p(y), _lib.F32)

        def read_y():
            out = np.empty(512, np.float32)
            _lib.call("fh_download", dev.handle, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(y), out.nbytes)
            return out

        gemv()
        eager = read_y()
        before = _live_bytes(dev)
        dev.capture_begin()
        gemv()
        _lib.call("fh_free", dev.handle, ctypes.c_void_p(ptrs["wq"]))  # used by the capture: kept
        _lib.call("fh_free", dev.handle, ctypes.c_void_p(unused))  # not used: freed at capture end
        graph = dev.capture_end()
        assert _live_bytes(dev) == before - (1 << 20)
        _lib.call("fh_free", dev.handle, ctypes.c_void_p(ptrs["x"]))  # after capture: retired
        assert _live_bytes(dev) == before - (1 << 20)
        # retired allocations are no longer valid operands
        with pytest.raises(_lib.HipError) as e:
            gemv()
        assert e.value.kind == "ForeignStorage"
        for _ in range(3):
            zero = np.zeros(512, np.float32)
            _lib.call("fh_upload", dev.handle, ctypes.c_void_p(y), zero.ctypes.data_as(ctypes.c_void_p), zero.nbytes)
            graph.launch()
            assert np.array_equal(read_y(), eager)
        del graph  # fh_graph_destroy: waits, then frees what the caller released
        assert _live_bytes(dev) == before - (1 << 20) - wq.nbytes - x.nbytes
        # a graph may outlive its device; it can then only be destroyed
        dev.capture_begin()
        _lib.call("fh_advance_positions", dev.handle, ctypes.c_void_p(y), 4, 1)
        orphan = dev.capture_end()
    finally:
        dev.close()
    assert _lib.load().fh_graph_destroy(ctypes.c_void_p(orphan._handle)) == _lib.OK
    orphan._handle = None


def test_profiled_device_counts_dispatches(device):
    prof = HipDevice.profiled(_lib.PROFILE_KERNELS)
    try:
        wq, s, b = synth.q4_weights(61, 256, 512)
        w = weight(prof, wq, s, b)
        x = up(prof, synth.bf16_normal(62, (1, 512)), DType.BF16)
        assert prof.take_profile()["allocations"] == 4
        for _ in range(3):
            Q4Linear(w).forward(prof, x)
        p = prof.take_profile()
        assert p["dispatches"] == 3 and p["gpu_busy_ns"] > 0 and p["allocations"] == 3
        assert prof.take_profile()["dispatches"] == 0
        assert prof.max_memory_allocated()["bytes"] > 0
    finally:
        prof.close()
    assert device.take_profile() is None
