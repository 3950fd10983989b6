"""GPU parity of the decode-step fusions of the q4 Linear (fh_q4_matmul_rmsnorm,
fh_q4_gate_up_silu), through the C-ABI.

Bars:
- residual_out, h = RNE(x + residual): bit-exact against the restatement.
- fh_q4_gate_up_silu: bit-identical to fh_q4_matmul on [gate; up] followed
  by fh_silu_mul (the epilogue rounds g and u to bf16 exactly as the stored
  linear output is rounded, then applies the same SiLU arithmetic) whenever
  both launch the same GEMV shape. The epilogue needs at most 32 lanes per
  weight row; where the plain GEMV picks 64 (k = 4096 here) the fp32 lane
  partials are added in another order, so g or u can differ by one bf16 ulp;
  the bar is then 99% identical and every output within 2^-7 of its row's
  largest magnitude (one ulp of g or u moves silu(g) * u by about that much;
  near zero that is many ulps of the output itself). From 2 rows both run
  the matrix-core GEMV with the same K split: a task there is 16 weight rows,
  or 8 gate rows and their 8 up rows, so f need only be a multiple of 8
  (f = 1000 below).
- fh_q4_gate_up_silu above 8 rows (no norm): the direct GEMM with the
  activation in its epilogue, bit-identical to fh_q4_matmul (the same kernel
  and K order) followed by fh_silu_mul.
- fh_q4_matmul_rmsnorm: the prologue sums h^2 in another order than
  fh_rms_norm, and sums each staged chunk of x in pairs, so a normalised value
  or a chunk sum can differ in its last bit. Bars: the fp32 output within 2e-3
  of the fp64 oracle applied to the restated RMSNorm row (src/nn/norm.rs:
  32-50), bf16 output = RNE of the fp32 output, and at least 99% of the bf16
  outputs identical to fh_rms_norm followed by fh_q4_matmul.
"""
import ctypes

import numpy as np
import pytest

from foundry_amd import _lib, synth
from oracle import llama_ref as R

pytestmark = pytest.mark.gpu

BOUND = 2e-3
EPS = 1e-5


def up(dev, arr):
    return dev.storage_from_bytes(np.ascontiguousarray(arr).tobytes())


def down(dev, st, dtype, count):
    out = np.empty(count, dtype=dtype)
    _lib.call("fh_download", dev.handle, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(st.ptr), out.nbytes)
    return out


def P(s):
    return None if s is None else ctypes.c_void_p(s.ptr)


def q4(dev, seed, n, k):
    wq, s, b = synth.q4_weights(seed, n, k)
    return (wq, s, b), [up(dev, a) for a in (wq, s, b)]


def matmul(dev, x, m, k, w, n, dtype):
    item = 4 if dtype == _lib.F32 else 2
    y = dev.empty(m * n * item)
    _lib.call("fh_q4_matmul", dev.handle, P(x), m, k, k, P(w[0]), P(w[1]), P(w[2]), n, 64, P(y), dtype)
    return down(dev, y, np.float32 if dtype == _lib.F32 else np.uint16, m * n).reshape(m, n)


def rel_err(y32, y64):
    return float(np.max(np.abs(y32.astype(np.float64) - y64))) / (float(np.max(np.abs(y64))) or 1.0)


def bits(a):
    return (np.ascontiguousarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("m,k,with_res", [(1, 3072, False), (1, 3072, True), (3, 3072, True), (8, 3072, True),
                                          (8, 4096, False), (2, 8192, True), (8, 8192, True), (5, 6144, False)])
def test_matmul_rmsnorm(device, oracle, m, k, with_res):
    n = 1024
    x = synth.bf16_normal(30 + m, (m, k))
    res = synth.bf16_normal(40 + m, (m, k)) if with_res else None
    w_norm = synth.bf16_rne((1 + 0.1 * synth.bf16_to_f32(synth.bf16_normal(50, (k,)))).astype(np.float32))
    (wq, s, b), w = q4(device, 60 + m, n, k)
    sx, sw = up(device, x), up(device, w_norm)
    sres = up(device, res) if with_res else None
    hout = device.empty(m * k * 2) if with_res else None
    outs = {}
    for dt in (_lib.F32, _lib.BF16):
        item = 4 if dt == _lib.F32 else 2
        y = device.empty(m * n * item)
        _lib.call("fh_q4_matmul_rmsnorm", device.handle, P(sx), P(sres), P(hout), P(sw), ctypes.c_float(EPS), m, k,
                  P(w[0]), P(w[1]), P(w[2]), n, 64, P(y), dt)
        outs[dt] = down(device, y, np.float32 if dt == _lib.F32 else np.uint16, m * n).reshape(m, n)
    h_ref = R.rne(R.from_bf16(x) + R.from_bf16(res)) if with_res else R.from_bf16(x)
    if with_res:
        assert np.array_equal(down(device, hout, np.uint16, m * k).reshape(m, k), bits(h_ref))
    cfg = type("C", (), {"rms_norm_eps": EPS})()
    x_norm = R.RefLlama.rms_norm(type("M", (), {"cfg": cfg})(), h_ref, R.from_bf16(w_norm))
    y64 = oracle.linear_f64(bits(x_norm), wq, s, b)
    assert rel_err(outs[_lib.F32], y64) <= BOUND
    assert np.array_equal(outs[_lib.BF16], synth.bf16_rne(outs[_lib.F32]))
    xn = device.empty(m * k * 2)
    h2 = device.empty(m * k * 2) if with_res else None
    _lib.call("fh_rms_norm", device.handle, P(sx), P(sres), P(h2), P(sw), m, k, ctypes.c_float(EPS), P(xn))
    unfused = matmul(device, xn, m, k, w, n, _lib.BF16)
    assert np.mean(unfused == outs[_lib.BF16]) >= 0.99


@pytest.mark.parametrize("m,k,f,same_shape", [(1, 3072, 8192, True), (4, 3072, 8192, True), (8, 4096, 1000, True),
                                              (1, 4096, 8192, False), (2, 256, 64, True)])
def test_gate_up_silu(device, m, k, f, same_shape):
    x = synth.bf16_normal(70 + m, (m, k))
    _, w = q4(device, 80 + m, 2 * f, k)
    sx = up(device, x)
    act = device.empty(m * f * 2)
    _lib.call("fh_q4_gate_up_silu", device.handle, P(sx), None, None, None, ctypes.c_float(EPS), m, k, P(w[0]),
              P(w[1]), P(w[2]), 2 * f, 64, P(act))
    got = down(device, act, np.uint16, m * f).reshape(m, f)
    gu = device.empty(m * 2 * f * 2)
    _lib.call("fh_q4_matmul", device.handle, P(sx), m, k, k, P(w[0]), P(w[1]), P(w[2]), 2 * f, 64, P(gu), _lib.BF16)
    want = device.empty(m * f * 2)
    _lib.call("fh_silu_mul", device.handle, P(gu), m, f, P(want))
    want = down(device, want, np.uint16, m * f).reshape(m, f)
    if same_shape:
        assert np.array_equal(got, want)
    else:
        gf, wf = R.from_bf16(got), R.from_bf16(want)
        row_max = np.abs(wf).max(axis=1, keepdims=True)
        assert np.mean(got == want) >= 0.99 and (np.abs(gf - wf) <= row_max * 2.0**-7).all()


@pytest.mark.parametrize("m,k,f", [(2048, 3072, 4096), (1000, 2048, 8192), (4096, 4096, 14336)])
def test_gate_up_silu_prompt_rows(device, m, k, f):
    """Above 8 rows the activation is formed in the prompt GEMM's epilogue
    (tiles of 256 rows x 128 gate/up column pairs that fill the chip), with
    no gate/up tensor in memory: bit-identical to fh_q4_matmul on [gate; up]
    followed by fh_silu_mul. m = 1000 leaves a ragged last row tile; f = 14336
    is the 8B shape's FFN."""
    x = synth.bf16_normal(75 + m, (m, k))
    _, w = q4(device, 85 + m, 2 * f, k)
    sx = up(device, x)
    act = device.empty(m * f * 2)
    _lib.call("fh_q4_gate_up_silu", device.handle, P(sx), None, None, None, ctypes.c_float(EPS), m, k, P(w[0]),
              P(w[1]), P(w[2]), 2 * f, 64, P(act))
    gu = device.empty(m * 2 * f * 2)
    _lib.call("fh_q4_matmul", device.handle, P(sx), m, k, k, P(w[0]), P(w[1]), P(w[2]), 2 * f, 64, P(gu), _lib.BF16)
    want = device.empty(m * f * 2)
    _lib.call("fh_silu_mul", device.handle, P(gu), m, f, P(want))
    got, want = down(device, act, np.uint16, m * f), down(device, want, np.uint16, m * f)
    assert np.array_equal(got, want)
    assert np.count_nonzero(got) > got.size // 2  # a real activation, not a cleared buffer


@pytest.mark.parametrize("m", [1, 3])
def test_gate_up_silu_with_rmsnorm(device, m):
    """Norm prologue and SiLU epilogue together equal fh_q4_matmul_rmsnorm's
    gate/up output (the same kernel prologue) followed by fh_silu_mul; h is
    bit-exact."""
    k, f = 3072, 8192
    x = synth.bf16_normal(90 + m, (m, k))
    res = synth.bf16_normal(91 + m, (m, k))
    wn = synth.bf16_rne((1 + 0.1 * synth.bf16_to_f32(synth.bf16_normal(92, (k,)))).astype(np.float32))
    _, w = q4(device, 93 + m, 2 * f, k)
    sx, sres, swn = up(device, x), up(device, res), up(device, wn)
    h1, h2 = device.empty(m * k * 2), device.empty(m * k * 2)
    act = device.empty(m * f * 2)
    _lib.call("fh_q4_gate_up_silu", device.handle, P(sx), P(sres), P(h1), P(swn), ctypes.c_float(EPS), m, k, P(w[0]),
              P(w[1]), P(w[2]), 2 * f, 64, P(act))
    gu = device.empty(m * 2 * f * 2)
    _lib.call("fh_q4_matmul_rmsnorm", device.handle, P(sx), P(sres), P(h2), P(swn), ctypes.c_float(EPS), m, k,
              P(w[0]), P(w[1]), P(w[2]), 2 * f, 64, P(gu), _lib.BF16)
    want = device.empty(m * f * 2)
    _lib.call("fh_silu_mul", device.handle, P(gu), m, f, P(want))
    assert np.array_equal(down(device, act, np.uint16, m * f), down(device, want, np.uint16, m * f))
    h_ref = bits(R.rne(R.from_bf16(x) + R.from_bf16(res))).ravel()
    assert np.array_equal(down(device, h1, np.uint16, m * k), h_ref)


def test_fused_matmul_argument_errors(device):
    k, n = 256, 64
    _, w = q4(device, 90, n, k)
    x = device.zeros(16 * k * 2)
    wn = device.zeros(k * 2)
    y = device.empty(16 * n * 4)

    def call(m, x_, res, res_out):
        _lib.call("fh_q4_matmul_rmsnorm", device.handle, P(x_), P(res), P(res_out), P(wn), ctypes.c_float(EPS), m, k,
                  P(w[0]), P(w[1]), P(w[2]), n, 64, P(y), _lib.F32)

    with pytest.raises(_lib.HipError, match="Unsupported"):
        call(9, x, None, None)
    with pytest.raises(_lib.HipError, match="overlaps"):
        call(2, x, x, x)
    with pytest.raises(_lib.HipError, match="without residual"):
        call(1, x, None, x)

    def gus(m, n_, res=None, wn_=None):
        _lib.call("fh_q4_gate_up_silu", device.handle, P(x), P(res), None, P(wn_), ctypes.c_float(EPS), m, k, P(w[0]),
                  P(w[1]), P(w[2]), n_, 64, P(y))

    with pytest.raises(_lib.HipError, match="Unsupported"):
        gus(9, n)
    with pytest.raises(_lib.HipError, match="gate; up"):
        gus(1, n - 1)
    with pytest.raises(_lib.HipError, match="without a norm weight"):
        gus(1, n, res=x)
