"""Host-side logic, no GPU: op output rules (src/nn/primitive.rs:146-289 for
the q4 ops), layouts, and the C-ABI library contract (loads, exports every
symbol include/foundry_hip.h declares, reports errors without a device)."""
import ctypes
import os
import re

import numpy as np
import pytest

from foundry_amd import _lib
from foundry_amd.device import Layout
from foundry_amd.primitive import (
    DType,
    QuantizedIndexSelect,
    QuantizedMatmul,
    TensorError,
    check_shape,
    output,
    profile_key,
)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "foundry_hip.h")


def q4(n, k, g=64):
    return [(DType.U32, (n, k // 8)), (DType.BF16, (n, k // g)), (DType.BF16, (n, k // g))]


def test_dtype_itemsize_and_float():
    assert [d.itemsize for d in (DType.F32, DType.BF16, DType.U32)] == [4, 2, 4]
    assert [d.is_float for d in (DType.F32, DType.BF16, DType.U32)] == [True, True, False]


def test_q4_matmul_output_shape():
    assert output(QuantizedMatmul(), [(DType.BF16, (1, 3072)), *q4(8192, 3072)]) == ((1, 8192), DType.BF16)
    assert output(QuantizedMatmul(), [(DType.F32, (5, 128)), *q4(7, 128)]) == ((5, 7), DType.F32)
    assert output(QuantizedMatmul(), [(DType.BF16, (0, 64)), *q4(3, 64)]) == ((0, 3), DType.BF16)


@pytest.mark.parametrize(
    "inputs,kind",
    [
        ([(DType.BF16, (1, 3072)), *q4(8192, 3136)], "MatmulIncompatible"),  # K mismatch
        ([(DType.BF16, (2, 1, 64)), *q4(4, 64)], "MatmulIncompatible"),  # x not 2-D
        ([(DType.U32, (1, 64)), *q4(4, 64)], "DTypeNotFloat"),
        ([(DType.BF16, (1, 64)), (DType.BF16, (4, 8)), *q4(4, 64)[1:]], "DTypeMismatch"),
        ([(DType.BF16, (1, 64)), (DType.U32, (4, 8)), (DType.BF16, (4, 2)), (DType.BF16, (4, 1))], "MatmulIncompatible"),
        ([(DType.BF16, (1, 96)), (DType.U32, (4, 12)), (DType.BF16, (4, 1)), (DType.BF16, (4, 1))], "MatmulIncompatible"),
        ([(DType.BF16, (1, 64)), *q4(4, 64)[:2]], "OperandCount"),
    ],
)
def test_q4_matmul_rejections(inputs, kind):
    with pytest.raises(TensorError) as e:
        output(QuantizedMatmul(), inputs)
    assert e.value.kind == kind


def test_q4_index_select_output_and_rejections():
    assert output(QuantizedIndexSelect(), [*q4(128256, 3072), (DType.U32, (4096,))]) == ((4096, 3072), DType.BF16)
    assert output(QuantizedIndexSelect(), [*q4(10, 64), (DType.U32, (0,))]) == ((0, 64), DType.BF16)
    with pytest.raises(TensorError) as e:
        output(QuantizedIndexSelect(), [*q4(10, 64), (DType.F32, (3,))])
    assert e.value.kind == "IndicesNotU32"
    with pytest.raises(TensorError) as e:
        output(QuantizedIndexSelect(), [*q4(10, 64), (DType.U32, (3, 1))])
    assert e.value.kind == "IndexSelectIncompatible"
    with pytest.raises(TensorError) as e:
        output(QuantizedIndexSelect(dim=1), [*q4(10, 64), (DType.U32, (3,))])
    assert e.value.kind == "IndexSelectIncompatible"
    with pytest.raises(TensorError) as e:
        output(QuantizedIndexSelect(bits=8), [*q4(10, 64), (DType.U32, (3,))])
    assert e.value.kind == "IndexSelectIncompatible"


def test_shape_limits():
    with pytest.raises(TensorError) as e:
        check_shape((1, 1, 1, 1, 1))
    assert e.value.kind == "RankTooLarge"
    with pytest.raises(TensorError) as e:
        check_shape((65536, 65536))
    assert e.value.kind == "NumelOverflow"


def test_layout_contiguity():
    lay = Layout.contiguous((2, 3, 4))
    assert lay.strides == (12, 4, 1) and lay.is_contiguous() and lay.numel == 24
    assert not Layout((3, 2), (1, 3)).is_contiguous()


def test_profile_key():
    assert profile_key(QuantizedMatmul(), 1, 3072, 8192) == "q4matmul b1 m1 k3072 n8192 g64"


def _declared_functions():
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(fh_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes table covers the whole header
    assert set(names) == set(_lib.SIGNATURES) | {"fh_last_error"}


def test_abi_version_matches_header():
    with open(HEADER) as f:
        version = int(re.search(r"#define FH_ABI_VERSION (\d+)", f.read()).group(1))
    assert _lib.load().fh_abi_version() == version


def _c_layout(struct: str, fields) -> list[int]:
    """sizeof and offsetof of a header struct, from a C program built with gcc."""
    import shutil
    import subprocess
    import tempfile

    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    body = "".join(f'    printf("%zu\\n", offsetof({struct}, {f}));\n' for f in fields)
    src = (f'#include <stdio.h>\n#include <stddef.h>\n#include "{HEADER}"\n'
           f'int main(void) {{\n    printf("%zu\\n", sizeof({struct}));\n{body}    return 0;\n}}\n')
    with tempfile.TemporaryDirectory() as tmp:
        c, exe = os.path.join(tmp, "layout.c"), os.path.join(tmp, "layout")
        with open(c, "w") as f:
            f.write(src)
        subprocess.run(["gcc", "-std=c99", "-o", exe, c], check=True, capture_output=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return [int(v) for v in out.split()]


@pytest.mark.parametrize("struct, cls", [("fh_q4_weight", _lib.Q4Weight), ("fh_llama_layer", _lib.LlamaLayer),
                                         ("fh_llama_model", _lib.LlamaModel), ("fh_view", _lib.View)])
def test_model_structs_match_the_header(struct, cls):
    fields = [f[0] for f in cls._fields_]
    assert _c_layout(struct, fields) == [ctypes.sizeof(cls)] + [getattr(cls, f).offset for f in fields]


def test_llama_forward_rejects_a_null_device_and_model():
    lib = _lib.load()
    m = _lib.LlamaModel()
    assert lib.fh_llama_forward(None, ctypes.addressof(m), 1, None, None, None) == _lib.ERR_INVALID_ARGUMENT
    assert "fh_llama_forward" in _lib.last_error()


def test_calls_without_a_device_return_errors_not_crashes():
    lib = _lib.load()
    handle = ctypes.c_void_p()
    # no GPU here: creation reports DeviceUnavailable (on a GPU box ordinal -1 does)
    rc = lib.fh_device_create(-1, ctypes.byref(handle))
    assert rc == _lib.ERR_DEVICE_UNAVAILABLE and handle.value is None
    assert "fh_device_create" in _lib.last_error()
    assert lib.fh_synchronize(None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.fh_q4_matmul(None, None, 1, 64, 64, None, None, None, 1, 64, None, 1) == _lib.ERR_INVALID_ARGUMENT
    # the load-time weight copies of the decoder
    assert lib.fh_q4_interleave(None, None, None, 16, 128, 64, None) == _lib.ERR_INVALID_ARGUMENT
    assert "fh_q4_interleave" in _lib.last_error()
    assert lib.fh_q4_tile(None, None, 16, 128, 64, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert "fh_q4_tile" in _lib.last_error()
    assert lib.fh_append_token_advance(None, None, 1, None, None, 0, 0, 1) == _lib.ERR_INVALID_ARGUMENT
    assert "fh_append_token_advance" in _lib.last_error()
    assert lib.fh_device_destroy(None) == _lib.OK
    n = ctypes.c_int(-1)
    assert lib.fh_device_count(ctypes.byref(n)) == _lib.OK and n.value >= 0


def test_hip_error_carries_kind():
    err = _lib.HipError(_lib.ERR_FOREIGN_STORAGE, "x")
    assert err.kind == "ForeignStorage" and "ForeignStorage" in str(err)


def test_product_package_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "foundry_amd")
    for dirpath, _, files in os.walk(pkg):
        for name in files:
            if name.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                with open(os.path.join(dirpath, name)) as f:
                    text = f.read()
                assert not re.search(r"^\s*(import|from)\s+oracle", text, flags=re.M), name
                assert "liboracle" not in text, name


# ---- views and the standard Ops' output rules ----

def test_layout_views_follow_the_reference():
    """src/nn/layout.rs tests (:202-313): permute, narrow, reshape, expand."""
    lay = Layout.contiguous((2, 3, 4))
    p = lay.permute((2, 0, 1))
    assert (p.shape, p.strides, p.is_contiguous()) == ((4, 2, 3), (1, 12, 4), False)
    for bad in ((0, 1), (0, 0, 1), (0, 1, 3)):
        with pytest.raises(TensorError) as e:
            lay.permute(bad)
        assert e.value.kind == "InvalidPermutation"
    n = lay.narrow(1, 1, 2)
    assert (n.shape, n.strides, n.offset) == ((2, 2, 4), (12, 4, 1), 4)
    for args, kind in (((1, 2, 2), "NarrowOutOfBounds"), ((3, 0, 1), "DimOutOfRange")):
        with pytest.raises(TensorError) as e:
            lay.narrow(*args)
        assert e.value.kind == kind
    r = lay.narrow(0, 1, 1).reshape((3, 4))
    assert (r.strides, r.offset) == ((4, 1), 12)
    with pytest.raises(TensorError) as e:
        Layout.contiguous((2, 3)).permute((1, 0)).reshape((6,))
    assert e.value.kind == "ReshapeNonContiguous"
    with pytest.raises(TensorError) as e:
        Layout.contiguous((2, 3)).reshape((5,))
    assert e.value.kind == "NumelMismatch"
    x = Layout.contiguous((3, 1)).expand((2, 3, 4))
    assert (x.shape, x.strides) == ((2, 3, 4), (0, 1, 0))
    with pytest.raises(TensorError) as e:
        Layout.contiguous((3, 2)).expand((3, 4))
    assert e.value.kind == "ExpandIncompatible"
    # a dim of size one may carry any stride and still be contiguous
    assert Layout((2, 1, 3), (3, 99, 1)).is_contiguous()


def test_standard_op_output_rules():
    """src/nn/primitive.rs:146-367 and its tests: shapes, dtypes and the
    TensorError kinds."""
    from foundry_amd.primitive import (Binary, BinaryOp, Cat, Copy, IndexSelect, Matmul, Reduce, ReduceOp,
                                       SliceScatter, ToDtype, Unary, UnaryOp, broadcast)
    F, B, U = DType.F32, DType.BF16, DType.U32
    assert output(Unary(UnaryOp.EXP), [(B, (2, 3))]) == ((2, 3), B)
    assert output(Binary(BinaryOp.ADD), [(F, (2, 3)), (F, (3,))]) == ((2, 3), F)
    assert broadcast((4, 1, 3), (2, 1)) == (4, 2, 3)
    assert output(Reduce(ReduceOp.SUM, 1), [(F, (2, 0))]) == ((2, 1), F)
    assert output(Reduce(ReduceOp.ARGMAX, 0), [(B, (2, 3))]) == ((1, 3), U)
    assert output(Matmul(), [(F, (2, 3, 40)), (F, (2, 40, 5))]) == ((2, 3, 5), F)
    assert output(Copy(), [(U, (7,))]) == ((7,), U)
    assert output(ToDtype(F), [(B, (4,))]) == ((4,), F)
    assert output(IndexSelect(0), [(F, (3, 4)), (U, (2,))]) == ((2, 4), F)
    assert output(Cat(1), [(F, (2, 1)), (F, (2, 3))]) == ((2, 4), F)
    assert output(SliceScatter(1, 2), [(B, (2, 4, 3)), (B, (2, 1, 3))]) == ((2, 4, 3), B)
    cases = [
        (Unary(UnaryOp.NEG), [(U, (2,))], "DTypeNotFloat"),
        (Unary(UnaryOp.NEG), [], "OperandCount"),
        (Binary(BinaryOp.MUL), [(F, (2,)), (B, (2,))], "DTypeMismatch"),
        (Binary(BinaryOp.MUL), [(F, (2, 3)), (F, (3, 2))], "BroadcastIncompatible"),
        (Reduce(ReduceOp.AMAX, 1), [(F, (2, 0))], "EmptyReduction"),
        (Reduce(ReduceOp.SUM, 2), [(F, (2, 3))], "DimOutOfRange"),
        (Matmul(), [(F, (2, 3)), (F, (2, 3))], "MatmulIncompatible"),
        (Matmul(), [(F, (2, 2, 3)), (F, (3, 3, 2))], "MatmulIncompatible"),
        (ToDtype(U), [(F, (2,))], "DTypeNotFloat"),
        (IndexSelect(0), [(F, (3, 4)), (F, (2,))], "IndicesNotU32"),
        (IndexSelect(1), [(F, (3, 4)), (U, (2,))], "IndexSelectIncompatible"),
        (Cat(0), [(F, (1, 3)), (F, (2, 2))], "CatIncompatible"),
        (SliceScatter(1, 3), [(F, (2, 4, 3)), (F, (2, 2, 3))], "SliceScatterOutOfBounds"),
    ]
    for op, inputs, kind in cases:
        with pytest.raises(TensorError) as e:
            output(op, inputs)
        assert e.value.kind == kind, (op, inputs)


# ---- the tiled K cache layout (foundry_amd/kv_layout.py, the kernels' k_tile) ----

@pytest.mark.parametrize("max_len,head_dim", [(40, 64), (300, 128), (768, 128), (17, 256), (16, 32)])
def test_k_tile_index_is_a_permutation_of_the_region(max_len, head_dim):
    from foundry_amd.kv_layout import k_tile_index
    idx = k_tile_index(max_len, head_dim)
    assert idx.shape == (max_len, head_dim)
    assert np.array_equal(np.sort(idx.ravel()), np.arange(max_len * head_dim))


def test_k_tile_index_known_offsets_and_fragment_runs():
    from foundry_amd.kv_layout import k_tile_index
    # key 33 of a 40-key region (group 2, 8 keys), dim 40 (block 1, offset 8):
    # 2 * 16 * 64 + 1 * (8 * 32) + 1 * 32 + 8
    assert k_tile_index(40, 64)[33, 40] == 2344
    assert k_tile_index(40, 64)[0, 0] == 0 and k_tile_index(40, 64)[0, 32] == 16 * 32
    # a full group: the fragment of keys 16..31 x dims 64..95 is one 512-element run
    idx = k_tile_index(64, 128)
    run = np.sort(idx[16:32, 64:96].ravel())
    assert np.array_equal(run, np.arange(16 * 128 + 2 * 16 * 32, 16 * 128 + 3 * 16 * 32))
    # 8 consecutive dims of one key stay consecutive (16-byte accesses)
    assert np.array_equal(idx[5, 24:32], np.arange(idx[5, 24], idx[5, 24] + 8))


def test_tile_k_round_trip():
    from foundry_amd.kv_layout import tile_k, untile_k, k_tile_index
    k = np.arange(2 * 3 * 40 * 64, dtype=np.uint16).reshape(2, 3, 40, 64)
    t = tile_k(k)
    assert np.array_equal(untile_k(t), k)
    flat = t.reshape(2, 3, -1)
    assert flat[1, 2, k_tile_index(40, 64)[33, 40]] == k[1, 2, 33, 40]
