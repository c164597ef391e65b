"""The ROWS32 order of native GGUF blocks on the host: the test-side restatement
(qcheck.rows32_order) against the layout's defining formula, element by element on small shapes,
and the entry points' host checks (no device work)."""
import ctypes

import numpy as np
import pytest

import oracle
from qcheck import rows32_order
from splosh_amd import _lib

TYPES = [8, 11, 14, 20, 21, 23]


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("rows,inner", [(1, 256), (32, 512), (45, 768)])
def test_rows32_order_formula(t, rows, inner):
    elems, size = oracle.GGUF_BLOCK[t]
    ub, units = 256 // elems * size, inner // 256
    native = np.random.default_rng(rows + t).integers(0, 256, rows * units * ub, dtype=np.uint8)
    got = rows32_order(native, t, rows, inner)
    r32 = (rows + 31) // 32 * 32
    assert got.size == r32 * units * ub
    expect = np.zeros_like(got)
    for n in range(rows):
        for u in range(units):
            dst = ((n // 32) * units * 32 + u * 32 + n % 32) * ub
            expect[dst:dst + ub] = native[(n * units + u) * ub:(n * units + u + 1) * ub]
    assert np.array_equal(got, expect)  # padding rows are zero in both


def test_rows32_bytes_and_checks():
    lib = _lib.lib()
    assert lib.splosh_gguf_rows32_bytes(14, 45, 768) == 64 * 3 * 210
    assert lib.splosh_gguf_rows32_bytes(8, 45, 768) == 64 * 768 // 32 * 34
    assert lib.splosh_gguf_rows32_bytes(8, 45, 800) == 0  # inner % 256 != 0
    assert lib.splosh_gguf_rows32_bytes(13, 45, 768) == 0  # not a native-block type
    assert lib.splosh_gguf_rows32_bytes(14 | 0x100, 45, 768) == 0
    w, o = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)
    st = lib.splosh_gguf_repack_rows32(8, w, 45, 800, o, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"
    st = lib.splosh_gguf_repack_rows32(14 | 0x100, w, 45, 768, o, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"
    st = lib.splosh_gguf_repack_rows32(14, w, 45, 768, None, None)
    assert _lib.STATUS_NAMES[st] == "nullPointer"
    # A GEMM on a ROWS32 weight whose inner is not a multiple of 256 is refused before any launch.
    st = lib.splosh_gguf_gemm(8 | 0x100, w, 45, 800, ctypes.c_void_p(0x4000), 800, ctypes.c_void_p(0x5000), 45,
                              _lib.BF16, None, 1, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "layoutMismatch"
    st = lib.splosh_gguf_gemm(14 | 0x200, w, 45, 768, ctypes.c_void_p(0x4000), 768, ctypes.c_void_p(0x5000), 45,
                              _lib.BF16, None, 1, None, 0, None)
    assert _lib.STATUS_NAMES[st] == "unsupported"
