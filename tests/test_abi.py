"""The C ABI library on the CPU: it loads, exports every symbol the header declares, and its host
helpers (layout, shape validation, errors) behave like the reference's Swift types. No kernel is
launched here."""
import re
from pathlib import Path

import pytest

from splosh_amd import _lib
from splosh_amd.quant import GemmQ4Shape, Q4BufferLayout, K_BY_COLUMNS
from splosh_amd._lib import GemmQ4Error, Q4BufferLayoutError

HEADER = Path(__file__).resolve().parents[1] / "include" / "splosh_q4.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w ]+?\*?\s*(splosh_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 19
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    assert _lib.lib().splosh_version().decode().startswith("splosh-amd")


def test_status_strings_name_the_reference_cases():
    s = _lib.lib().splosh_status_string
    assert s(1) == b"invalidShape" and s(2) == b"layoutMismatch" and s(8) == b"bufferTooSmall"


def test_layout_padded_rows():
    """Q4BufferLayoutTests.swift:7-13: K=65 -> 9 packed words, stride 128 B, 23 padding words."""
    layout = Q4BufferLayout(rows=2, logical_k=65)
    assert layout.packed_words_per_row == 9
    assert layout.row_stride_bytes == 128
    assert layout.padding_words_per_row == 23
    assert layout.groups_per_row == 2 and layout.sidecar_count == 4
    assert layout.word_index(1, 64) == 32 + 8
    assert layout.nibble_shift(1, 63) == 28
    assert layout.sidecar_index(1, 64) == 3


def test_layout_k_by_columns():
    """Q4BufferLayoutTests.swift:29-40: transposed addressing."""
    layout = Q4BufferLayout(rows=3, logical_k=65, orientation=K_BY_COLUMNS)
    assert layout.row_stride_bytes == 128
    assert layout.word_index(2, 0) != layout.word_index(0, 2)
    assert layout.word_index(2, 64) == 64 * layout.row_stride_words + 0
    assert layout.nibble_shift(2, 64) == 8


def test_layout_errors():
    with pytest.raises(Q4BufferLayoutError) as e:
        Q4BufferLayout(rows=0, logical_k=64)
    assert e.value.case == "invalidDimensions"
    with pytest.raises(Q4BufferLayoutError) as e:
        Q4BufferLayout(rows=2, logical_k=65, row_stride_bytes=32)
    assert e.value.case == "invalidRowStride"
    with pytest.raises(Q4BufferLayoutError) as e:
        Q4BufferLayout(rows=2, logical_k=64).word_index(2, 0)
    assert e.value.case == "invalidIndex"


def test_shape_validate_rejects_malformed_layouts():
    """GemmOracleTests.swift:229-238 (malformedLayoutFailsClosed) and Gemm.swift:19-40."""
    shape = GemmQ4Shape(2, 3, 65)
    shape.validate(Q4BufferLayout(rows=3, logical_k=65))
    with pytest.raises(GemmQ4Error) as e:
        shape.validate(Q4BufferLayout(rows=4, logical_k=65))
    assert e.value.case == "layoutMismatch"
    with pytest.raises(GemmQ4Error) as e:
        shape.validate(Q4BufferLayout(rows=3, logical_k=64))
    assert e.value.case == "layoutMismatch"
    with pytest.raises(GemmQ4Error) as e:
        shape.validate(Q4BufferLayout(rows=3, logical_k=65, orientation=K_BY_COLUMNS))
    assert e.value.case == "orientationMismatch"
    with pytest.raises(GemmQ4Error) as e:
        shape.validate(Q4BufferLayout(rows=3, logical_k=65, row_stride_bytes=132))
    assert e.value.case == "invalidRowStride"
    with pytest.raises(GemmQ4Error) as e:
        GemmQ4Shape(0, 3, 65)
    assert e.value.case == "invalidShape"


def test_entry_points_validate_before_launch():
    """Malformed calls are rejected on the host with the reference's error case; no device work."""
    import ctypes
    lib = _lib.lib()
    w = _lib.Q4Weight(0x1000, 0x2000, 0x3000, 200, 512, 0, _lib.TILED128, 0)
    st = lib.splosh_q4_gemm(ctypes.byref(w), ctypes.c_void_p(0x4000), 512, ctypes.c_void_p(0x5000), 200, _lib.BF16,
                            None, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"
    w = _lib.Q4Weight(0, 0x2000, 0x3000, 256, 512, 0, _lib.TILED128, 0)
    st = lib.splosh_q4_gemm(ctypes.byref(w), ctypes.c_void_p(0x4000), 512, ctypes.c_void_p(0x5000), 256, _lib.BF16,
                            None, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "nullPointer"
    w = _lib.Q4Weight(0x1000, 0x2000, 0x3000, 256, 512, 0, _lib.TILED128, 0)
    st = lib.splosh_q4_gemm(ctypes.byref(w), ctypes.c_void_p(0x4000), 500, ctypes.c_void_p(0x5000), 256, _lib.BF16,
                            None, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "invalidShape"
    w = _lib.Q4Weight(0x1000, 0x2000, 0x3000, 256, 512, 10, _lib.ROW_MAJOR, 0)
    st = lib.splosh_q4_gemm(ctypes.byref(w), ctypes.c_void_p(0x4000), 512, ctypes.c_void_p(0x5000), 256, _lib.BF16,
                            None, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "invalidRowStride"
    q = _lib.Q5KWeight(0x1000, 0x2000, 0x3000, 256, 300)
    st = lib.splosh_q5k_gemm(ctypes.byref(q), ctypes.c_void_p(0x4000), 512, ctypes.c_void_p(0x5000), 256, _lib.BF16,
                             None, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"
    assert "256" in _lib.last_error()
    g = _lib.Q4Weight(0x1000, 0x2000, 0x3000, 256, 512, 0, _lib.TILED128, 0)
    u = _lib.Q4Weight(0x1000, 0x2000, 0x3000, 128, 512, 0, _lib.TILED128, 0)
    st = lib.splosh_q4_mlp_in(ctypes.byref(g), ctypes.byref(u), ctypes.c_void_p(0x4000), 512, ctypes.c_void_p(0x5000),
                              256, _lib.BF16, 1, _lib.KERNEL_AUTO, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"


def test_no_undefined_kernel_symbols():
    """Every kernel the launchers reference is defined in the library (a host stub that the
    compiler silently dropped would only show up as a load failure on the GPU box)."""
    import shutil
    import subprocess
    from splosh_amd import _lib
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--undefined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert "splosh" not in out, out
