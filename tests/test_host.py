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
                                         ("fh_llama_model", _lib.LlamaModel)])
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
