"""GPU tests of the strided entry points (the reference's non-quantized Ops)
through Tensor -> HipDevice.run / run_in_place -> the C-ABI.

The first group restates the reference's Metal known answers
(src/metal/mod.rs:1437-3200) with their tolerances (1e-5 for F32, 1e-2 for
BF16, relative). The second group compares strided, broadcast and permuted
inputs with numpy restatements of the Metal kernels' arithmetic:
- copy, to_dtype, index_select, cat, slice_scatter: bit-exact;
- neg, add, sub, mul, div (one correctly rounded fp32 op, then one rounding):
  bit-exact;
- exp, sqrt, reciprocal: within one fp32 ulp of float64 before the output
  rounding (bf16 outputs within one bf16 ulp);
- sum and amax: bit-exact against the restated 256-thread fold and halving
  tree (reduce.metal:17-40); argmax exact, first index on ties;
- matmul: within 1e-5 (F32) or one bf16 ulp plus 1e-5 (BF16) of float64,
  relative to max|out|.
"""
import math

import numpy as np
import pytest

from foundry_amd import _lib
from foundry_amd.primitive import DType, TensorError
from foundry_amd.tensor import Tensor
from oracle import llama_ref as R

pytestmark = pytest.mark.gpu

E = math.e


def f32(device, values, shape):
    return Tensor.from_numpy(device, np.asarray(values, np.float32).reshape(shape), DType.F32)


def u32(device, values):
    return Tensor.from_numpy(device, np.asarray(values, np.uint32), DType.U32)


def values(device, t):
    """A tensor's values as float32 (bf16 decoded exactly)."""
    if t.dtype is DType.BF16:
        return R.from_bf16(t.to_numpy(device))
    return t.to_numpy(device)


def close(actual, expected, tol):
    actual, expected = np.asarray(actual, np.float64).ravel(), np.asarray(expected, np.float64).ravel()
    assert actual.shape == expected.shape
    assert np.all(np.abs(actual - expected) <= tol * np.maximum(np.abs(expected), np.finfo(np.float32).tiny)), \
        (actual, expected)


TOL = {DType.F32: 1e-5, DType.BF16: 1e-2}


# ---------------- the reference's known answers ----------------

@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_unary_known_answers(device, dtype):
    """src/metal/mod.rs:1437-1530."""
    cases = {"neg": ([1.0, -2.5, 0.0], [-1.0, 2.5, 0.0]), "exp": ([0.0, 1.0, -1.0], [1.0, E, 1 / E]),
             "sqrt": ([4.0, 2.25, 0.0], [2.0, 1.5, 0.0]), "reciprocal": ([2.0, -4.0, 0.5], [0.5, -0.25, 2.0])}
    for name, (x, want) in cases.items():
        t = f32(device, x, (3,)).to_dtype(device, dtype)
        out = getattr(t, name)(device)
        assert out.dtype is dtype
        close(values(device, out.to_dtype(device, DType.F32)), want, TOL[dtype])


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_binary_known_answers(device, dtype):
    """src/metal/mod.rs:1533-1630."""
    a = f32(device, [1, 2, 3, 4], (4,)).to_dtype(device, dtype)
    b = f32(device, [2, 4, 0.5, -1], (4,)).to_dtype(device, dtype)
    for name, want in (("add", [3, 6, 3.5, 3]), ("sub", [-1, -2, 2.5, 5]), ("mul", [2, 8, 1.5, -4]),
                       ("div", [0.5, 0.5, 6, -4])):
        close(values(device, getattr(a, name)(device, b)), want, TOL[dtype])


def test_add_broadcasts_and_strided_reads(device):
    """src/metal/mod.rs:1633-1780: a row over a matrix; neg and mul of
    permuted operands."""
    m = f32(device, [0, 1, 2, 3, 4, 5], (2, 3))
    s = m.add(device, f32(device, [10, 20, 30], (3,)))
    assert s.shape == (2, 3) and values(device, s).tolist() == [[10, 21, 32], [13, 24, 35]]
    n = m.permute((1, 0)).neg(device)
    assert n.shape == (3, 2) and values(device, n).ravel().tolist() == [-0.0, -3.0, -1.0, -4.0, -2.0, -5.0]
    p = f32(device, [0, 1, 2, 3, 4, 5], (3, 2)).permute((1, 0)).mul(device, f32(device, [1, 2, 3, 4, 5, 6], (2, 3)))
    assert values(device, p).ravel().tolist() == [0, 4, 12, 4, 15, 30]


def test_long_chains_keep_submission_order(device):
    """src/metal/mod.rs:1783-1856: 300 adds of one; zeros interleaved."""
    ones = f32(device, [1] * 4, (4,))
    acc = Tensor.zeros(device, DType.F32, (4,))
    for _ in range(300):
        acc = acc.add(device, ones)
    assert values(device, acc).tolist() == [300.0] * 4
    acc = f32(device, [1] * 3, (3,))
    ones = f32(device, [1] * 3, (3,))
    for _ in range(100):
        acc = acc.add(device, Tensor.zeros(device, DType.F32, (3,))).add(device, ones)
    assert values(device, acc).tolist() == [101.0] * 3


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_reduce_known_answers(device, dtype):
    """src/metal/mod.rs:1859-2007: sum, amax and argmax over each dim."""
    x = f32(device, [1, 5, 3, 4, 2, 6], (2, 3)).to_dtype(device, dtype)
    for name, dim, dims, want in (("sum_keepdim", 0, (1, 3), [5, 7, 9]), ("sum_keepdim", 1, (2, 1), [9, 12]),
                                  ("amax_keepdim", 0, (1, 3), [4, 5, 6]), ("amax_keepdim", 1, (2, 1), [5, 6])):
        r = getattr(x, name)(device, dim)
        assert r.dtype is dtype and r.shape == dims
        close(values(device, r), want, TOL[dtype])
    for dim, dims, want in ((0, (1, 3), [1, 0, 1]), (1, (2, 1), [1, 2])):
        r = x.argmax_keepdim(device, dim)
        assert r.dtype is DType.U32 and r.shape == dims and r.to_numpy(device).ravel().tolist() == want


def test_reduce_edge_cases(device):
    """src/metal/mod.rs:2009-2150: 4096 bf16 ones sum to 4096; argmax ties
    (also across threads); a permuted input; an empty sum is 0."""
    s = f32(device, [1.0] * 4096, (4096,)).to_dtype(device, DType.BF16).sum_keepdim(device, 0)
    assert values(device, s).tolist() == [4096.0]
    assert f32(device, [3, 7, 7, 1], (4,)).argmax_keepdim(device, 0).to_numpy(device).tolist() == [1]
    v = [9.0 if i in (10, 300) else float(i % 7) for i in range(600)]
    assert f32(device, v, (600,)).argmax_keepdim(device, 0).to_numpy(device).tolist() == [10]
    t = f32(device, [0, 1, 2, 3, 4, 5], (2, 3)).permute((1, 0)).sum_keepdim(device, 1)
    assert t.shape == (3, 1) and values(device, t).ravel().tolist() == [3, 5, 7]
    e = Tensor.from_bytes(device, b"", DType.F32, (2, 0)).sum_keepdim(device, 1)
    assert e.shape == (2, 1) and values(device, e).ravel().tolist() == [0.0, 0.0]
    with pytest.raises(TensorError) as err:
        Tensor.from_bytes(device, b"", DType.F32, (2, 0)).amax_keepdim(device, 1)
    assert err.value.kind == "EmptyReduction"


def _pattern(count, seed):
    """src/metal/mod.rs:2339-2346: ((i * seed + 3) % 17 - 8) / 8, u16 wrap."""
    return np.array([(((i * seed) & 0xFFFF) + 3) % 17 for i in range(count)], np.float32) / 8 - 1


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_matmul_known_answers(device, dtype):
    """src/metal/mod.rs:2154-2440: [2,3]x[3,2]; x.W^T and L^T x R read in
    place; batched [2,3,40]x[2,40,5]."""
    a = f32(device, [1, 2, 3, 4, 5, 6], (2, 3)).to_dtype(device, dtype)
    b = f32(device, [7, 8, 9, 10, 11, 12], (3, 2)).to_dtype(device, dtype)
    close(values(device, a.matmul(device, b)), [58, 64, 139, 154], TOL[dtype])
    x = f32(device, [1, 2, 3, 4, 5, 6], (2, 3))
    w = f32(device, [1, 0, -1, 2, 1, 0], (2, 3))
    lt = f32(device, [1, 4, 2, 5, 3, 6], (3, 2))
    r = f32(device, [7, 8, 9, 10, 11, 12], (3, 2))
    assert values(device, x.matmul(device, w.permute((1, 0)))).ravel().tolist() == [-2, 4, -2, 13]
    assert values(device, lt.permute((1, 0)).matmul(device, r)).ravel().tolist() == [58, 64, 139, 154]
    lv, rv = _pattern(2 * 3 * 40, 7), _pattern(2 * 40 * 5, 5)
    want = np.einsum("bij,bjk->bik", lv.reshape(2, 3, 40).astype(np.float64), rv.reshape(2, 40, 5).astype(np.float64))
    got = f32(device, lv, (2, 3, 40)).to_dtype(device, dtype).matmul(device, f32(device, rv, (2, 40, 5))
                                                                     .to_dtype(device, dtype))
    close(values(device, got), want, TOL[dtype])


def test_matmul_tiles_strides_and_empty(device):
    """src/metal/mod.rs:2443-2740: 37x20x33 over several tiles within 1e-5;
    a rhs permuted to strides (12, 4) on its last dims; permuted batch dims
    equal to the contiguous copy; an empty output."""
    lv, rv = _pattern(37 * 20, 3), _pattern(20 * 33, 11)
    want = lv.reshape(37, 20).astype(np.float64) @ rv.reshape(20, 33).astype(np.float64)
    close(values(device, f32(device, lv, (37, 20)).matmul(device, f32(device, rv, (20, 33)))), want, 1e-5)
    for dtype in (DType.F32, DType.BF16):
        rhs = f32(device, np.arange(24), (2, 3, 4)).to_dtype(device, dtype).permute((2, 0, 1))
        lhs = f32(device, np.arange(16), (4, 2, 2)).to_dtype(device, dtype)
        r64 = np.arange(24, dtype=np.float64).reshape(2, 3, 4).transpose(2, 0, 1)
        want = np.einsum("bij,bjk->bik", np.arange(16, dtype=np.float64).reshape(4, 2, 2), r64)
        close(values(device, lhs.matmul(device, rhs)), want, TOL[dtype])
    lhs = f32(device, np.arange(48), (2, 3, 2, 4)).permute((1, 0, 2, 3))
    rhs = f32(device, np.arange(24), (3, 2, 4, 1))
    assert lhs.matmul(device, rhs).to_bytes(device) == lhs.contiguous(device).matmul(device, rhs).to_bytes(device)
    e = Tensor.from_bytes(device, b"", DType.F32, (0, 3)).matmul(device, f32(device, np.arange(6), (3, 2)))
    assert e.shape == (0, 2) and e.to_bytes(device) == b""


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_index_select_known_answers(device, dtype):
    """src/metal/mod.rs:2745-2900: rows [2, 0]; an id past the table gives
    zeros; a permuted table."""
    t = f32(device, np.arange(12), (3, 4)).to_dtype(device, dtype)
    rows = t.index_select(device, 0, u32(device, [2, 0]))
    assert rows.shape == (2, 4)
    close(values(device, rows), [8, 9, 10, 11, 0, 1, 2, 3], TOL[dtype])
    z = f32(device, np.arange(6), (3, 2)).index_select(device, 0, u32(device, [1, 3]))
    assert values(device, z).ravel().tolist() == [2, 3, 0, 0]
    p = f32(device, np.arange(6), (2, 3)).permute((1, 0)).index_select(device, 0, u32(device, [2, 0]))
    assert values(device, p).ravel().tolist() == [2, 5, 0, 3]


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_cat_and_slice_scatter_known_answers(device, dtype):
    """src/metal/mod.rs:2902-3200: cat on the first and last dim, of a
    permuted input, with an empty input; slice_scatter of one cache
    position."""
    top, bottom = f32(device, [0, 1, 2], (1, 3)), f32(device, np.arange(3, 9), (2, 3))
    left, right = f32(device, [10, 20], (2, 1)), f32(device, np.arange(6), (2, 3))
    c0 = Tensor.cat(device, [top.to_dtype(device, dtype), bottom.to_dtype(device, dtype)], 0)
    c1 = Tensor.cat(device, [left.to_dtype(device, dtype), right.to_dtype(device, dtype)], 1)
    assert c0.shape == (3, 3) and c1.shape == (2, 4)
    close(values(device, c0), np.arange(9), TOL[dtype])
    close(values(device, c1), [10, 0, 1, 2, 20, 3, 4, 5], TOL[dtype])
    pc = Tensor.cat(device, [f32(device, np.arange(6), (2, 3)).permute((1, 0)), f32(device, [10, 11], (1, 2))], 0)
    assert values(device, pc).ravel().tolist() == [0, 3, 1, 4, 2, 5, 10, 11]
    ec = Tensor.cat(device, [Tensor.from_bytes(device, b"", DType.F32, (0, 3)), f32(device, np.arange(6), (2, 3))], 0)
    assert ec.shape == (2, 3) and values(device, ec).ravel().tolist() == list(range(6))
    heads, positions, head_dim, position = 2, 4, 3, 2
    cache = Tensor.zeros(device, dtype, (heads, positions, head_dim))
    update = f32(device, np.arange(1, 7), (heads, 1, head_dim)).to_dtype(device, dtype)
    cache.slice_scatter(device, update, 1, position)
    want = np.zeros((heads, positions, head_dim))
    want[:, position, :] = np.arange(1, 7).reshape(heads, head_dim)
    close(values(device, cache), want, TOL[dtype])


def test_slice_scatter_rejections(device):
    cache = Tensor.zeros(device, DType.F32, (2, 4, 3))
    upd = f32(device, np.arange(6), (2, 1, 3))
    with pytest.raises(TensorError) as e:
        cache.slice_scatter(device, upd, 1, 4)
    assert e.value.kind == "SliceScatterOutOfBounds"
    view = cache.permute((1, 0, 2))
    with pytest.raises(TensorError) as e:
        view.slice_scatter(device, upd.permute((1, 0, 2)), 0, 0)
    assert e.value.kind in ("SliceScatterNonContiguous", "SharedStorage")
    del view
    alias = cache.reshape((2, 4, 3))
    with pytest.raises(TensorError) as e:
        cache.slice_scatter(device, upd, 1, 0)
    assert e.value.kind == "SharedStorage"
    del alias
    cache.slice_scatter(device, upd, 1, 0)


# ---------------- strided inputs against numpy restatements ----------------

def _rne32(x64):
    return np.asarray(x64, np.float64).astype(np.float32)


def _as_dtype(x32, dtype):
    return R.rne(x32) if dtype is DType.BF16 else np.asarray(x32, np.float32)


def _ulp32(v):
    return np.spacing(np.abs(np.asarray(v, np.float32))).astype(np.float64)


def _permuted(device, rng, shape, perm, dtype):
    """A tensor whose view `perm` of a contiguous base has `shape`, plus the
    same values as a numpy array."""
    base_shape = tuple(shape[perm.index(d)] for d in range(len(shape)))
    base = _as_dtype(rng.standard_normal(base_shape).astype(np.float32) * 3, dtype)
    t = Tensor.from_numpy(device, base if dtype is DType.F32 else (base.view(np.uint32) >> 16).astype(np.uint16),
                          dtype)
    return t.permute(perm), base.transpose(perm)


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_elementwise_on_strided_and_broadcast_views(device, dtype):
    rng = np.random.default_rng(7)
    a, an = _permuted(device, rng, (3, 5, 7, 2), (2, 0, 3, 1), dtype)
    b, bn = _permuted(device, rng, (5, 1, 2), (2, 0, 1), dtype)  # broadcast over dims 0 and 2
    a2, an2 = _permuted(device, rng, (3, 5, 7, 2), (0, 1, 2, 3), dtype)
    for name, fn in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)):
        got = values(device, getattr(a, name)(device, b))
        want = _as_dtype(fn(an, bn).astype(np.float32), dtype)  # one fp32 rounding, then the output's
        assert np.array_equal(got, want), name
    assert np.array_equal(values(device, a.neg(device)), -an)
    for name, fn, src in (("exp", np.exp, an2), ("sqrt", np.sqrt, np.abs(an2)), ("reciprocal", lambda v: 1.0 / v, an2 + 0.25)):
        x = Tensor.from_numpy(device, src if dtype is DType.F32 else (_as_dtype(src, dtype).view(np.uint32) >> 16)
                              .astype(np.uint16), dtype)
        xs = _as_dtype(src, dtype).astype(np.float64)
        got = values(device, getattr(x, name)(device)).astype(np.float64)
        exact = fn(xs)
        if dtype is DType.F32:
            assert np.all(np.abs(got - exact) <= _ulp32(exact)), name
        else:
            assert np.all(np.abs(got - exact) <= 2.0 ** -8 * np.abs(exact) + 1e-30), name


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_copy_convert_gather_scatter_bit_exact(device, dtype):
    rng = np.random.default_rng(8)
    a, an = _permuted(device, rng, (4, 6, 5), (1, 2, 0), dtype)
    c = a.contiguous(device)
    assert c.layout.is_contiguous() and np.array_equal(values(device, c), an)
    other = DType.F32 if dtype is DType.BF16 else DType.BF16
    conv = a.to_dtype(device, other)
    assert np.array_equal(values(device, conv), _as_dtype(an, other))
    # narrow views read in place
    n = a.narrow(1, 1, 3)
    assert np.array_equal(values(device, n.contiguous(device)), an[:, 1:4, :])
    table, tn = _permuted(device, rng, (9, 5), (1, 0), dtype)
    ids = u32(device, [8, 0, 9, 3, 4294967295, 8])
    got = values(device, table.index_select(device, 0, ids))
    want = np.vstack([tn[i] if i < 9 else np.zeros(5, np.float32) for i in [8, 0, 9, 3, 4294967295, 8]])
    assert np.array_equal(got, want)
    b, bn = _permuted(device, rng, (4, 2, 5), (2, 0, 1), dtype)
    for dim, other_t, other_n in ((1, b, bn),):
        cat = Tensor.cat(device, [a, other_t], dim)
        assert np.array_equal(values(device, cat), np.concatenate([an, other_n], axis=dim))
    target = Tensor.zeros(device, dtype, (4, 9, 5))
    target.slice_scatter(device, a, 1, 2)
    target.slice_scatter(device, b, 1, 7)
    want = np.zeros((4, 9, 5), np.float32)
    want[:, 2:8, :] = an
    want[:, 7:9, :] = bn
    assert np.array_equal(values(device, target), want)


def _reduce_restated(rows, amax):
    """reduce_rows' order for every row at once: thread t folds k = t,
    t + 256, ... in fp32, then the halving tree over the 256 partials
    (reduce.metal:17-40)."""
    op = np.maximum if amax else np.add
    parts = np.full((rows.shape[0], 256), -np.inf if amax else 0.0, np.float32)
    for t in range(min(256, rows.shape[1])):
        for k in range(t, rows.shape[1], 256):
            parts[:, t] = op(parts[:, t], rows[:, k])
    w = 128
    while w > 0:
        parts[:, :w] = op(parts[:, :w], parts[:, w:2 * w])
        w //= 2
    return parts[:, 0]


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_reductions_match_the_restated_order(device, dtype):
    rng = np.random.default_rng(9)
    a, an = _permuted(device, rng, (3, 1000, 2), (2, 0, 1), dtype)
    for dim in (0, 1, 2):
        moved = np.moveaxis(an, dim, -1)
        rows = moved.reshape(-1, moved.shape[-1])
        s = values(device, a.sum_keepdim(device, dim)).ravel()
        m = values(device, a.amax_keepdim(device, dim)).ravel()
        i = a.argmax_keepdim(device, dim).to_numpy(device).ravel()
        want_s = _as_dtype(_reduce_restated(np.ascontiguousarray(rows, np.float32), False), dtype)
        want_m = _as_dtype(_reduce_restated(np.ascontiguousarray(rows, np.float32), True), dtype)
        assert np.array_equal(s, want_s.ravel()), dim
        assert np.array_equal(m, want_m.ravel()), dim
        assert np.array_equal(i, np.array([int(np.flatnonzero(r == r.max())[0]) for r in rows])), dim


def test_reductions_over_more_rows_than_the_grid():
    """More output rows (2^20 + 37) than the reduce grid's 2^20 blocks: the
    blocks stride over the rows, and every row is still reduced in the
    restated order (a row of 3: thread t takes element t, then the tree)."""
    from foundry_amd.device import HipDevice

    dev = HipDevice(0)
    try:
        rows = (1 << 20) + 37
        x = (np.arange(rows * 3, dtype=np.int64) % 251).astype(np.float32).reshape(rows, 3) - 125.0
        t = Tensor.from_numpy(dev, x, DType.F32)
        s = t.sum_keepdim(dev, 1).to_numpy(dev).ravel()
        m = t.amax_keepdim(dev, 1).to_numpy(dev).ravel()
        i = t.argmax_keepdim(dev, 1).to_numpy(dev).ravel()
        assert np.array_equal(s, (x[:, 0] + x[:, 1]) + x[:, 2])
        assert np.array_equal(m, x.max(axis=1))
        assert np.array_equal(i, x.argmax(axis=1).astype(np.uint32))
    finally:
        dev.close()


@pytest.mark.parametrize("dtype", [DType.F32, DType.BF16])
def test_matmul_on_strided_batches(device, dtype):
    rng = np.random.default_rng(10)
    lhs, ln = _permuted(device, rng, (2, 3, 45, 70), (1, 0, 3, 2), dtype)
    rhs, rn = _permuted(device, rng, (2, 3, 70, 37), (0, 1, 3, 2), dtype)
    got = values(device, lhs.matmul(device, rhs)).astype(np.float64)
    want = np.matmul(ln.astype(np.float64), rn.astype(np.float64))
    bound = 1e-5 * np.max(np.abs(want))
    if dtype is DType.BF16:
        bound = bound + 2.0 ** -8 * np.abs(want)
    assert np.all(np.abs(got - want) <= bound)


def test_strided_entry_points_reject_bad_views(device):
    """Out-of-allocation views and mismatched dims are refused on the host."""
    import ctypes
    t = f32(device, np.arange(6), (2, 3))
    out = device.empty(64)
    bad = _lib.View.of((2, 4), (3, 1), 0)  # reads past the 6 elements
    with pytest.raises(_lib.HipError) as e:
        _lib.call("fh_copy_strided", device.handle, int(DType.F32), ctypes.c_void_p(t.storage.ptr),
                  ctypes.byref(bad), ctypes.c_void_p(out.ptr))
    assert e.value.kind == "OutOfBounds"
    ok = _lib.View.of((2, 3), (3, 1), 0)
    other = _lib.View.of((3, 2), (1, 3), 0)
    with pytest.raises(_lib.HipError) as e:
        _lib.call("fh_binary", device.handle, 0, int(DType.F32), ctypes.c_void_p(t.storage.ptr), ctypes.byref(ok),
                  ctypes.c_void_p(t.storage.ptr), ctypes.byref(other), ctypes.c_void_p(out.ptr))
    assert e.value.kind == "InvalidArgument"
