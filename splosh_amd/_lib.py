"""ctypes binding of libsplosh_q4.so (include/splosh_q4.h).

The library is loaded from this package directory; if it is missing, every call raises
``SploshLibraryError`` -- there is no fallback path.
"""
import ctypes
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libsplosh_q4.so"

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# status codes (splosh_status)
OK = 0
STATUS_NAMES = {
    1: "invalidShape", 2: "layoutMismatch", 3: "invalidRowStride", 4: "orientationMismatch",
    5: "invalidGroupSize", 6: "sidecarGeometryMismatch", 7: "sidecarMismatch", 8: "bufferTooSmall",
    9: "invalidDimensions", 10: "arithmeticOverflow", 11: "invalidIndex", 12: "nullPointer",
    13: "unsupported", 14: "workspaceTooSmall", 15: "hipError",
}

ROWS_BY_K, K_BY_COLUMNS = 0, 1
ROW_MAJOR, TILED128 = 0, 1
F32, BF16 = 0, 1
KERNEL_AUTO, KERNEL_STREAM, KERNEL_DEQUANT, KERNEL_TILE, KERNEL_SCALAR, KERNEL_PREFILL = 0, 1, 2, 3, 4, 5


class SploshLibraryError(RuntimeError):
    pass


class SploshError(RuntimeError):
    """A failure the library reported; ``case`` is the reference's error case name."""

    def __init__(self, status, message):
        self.status = status
        self.case = STATUS_NAMES.get(status, "unknown")
        super().__init__(f"{self.case}: {message}")


class GemmQ4Error(SploshError):
    """GemmQ4Error (Model/Gemm.swift:43-52): statuses 1..8."""


class Q4BufferLayoutError(SploshError):
    """Q4BufferLayoutError (Quant/Q4BufferLayout.swift:16-23): statuses 9..11 (and 3)."""


class Layout(ctypes.Structure):
    _fields_ = [("rows", _i64), ("logical_k", _i64), ("orientation", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("packed_words_per_row", _i64),
                ("row_stride_bytes", _i64), ("row_stride_words", _i64),
                ("padding_words_per_row", _i64), ("groups_per_row", _i64), ("group_stride", _i64)]


class Q4Weight(ctypes.Structure):
    _fields_ = [("packed", _vp), ("scales", _vp), ("biases", _vp), ("rows", _i64), ("inner", _i64),
                ("row_stride_words", _i64), ("order", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Q5KWeight(ctypes.Structure):
    _fields_ = [("plane0", _vp), ("plane1", _vp), ("meta", _vp), ("rows", _i64), ("inner", _i64)]


# name -> (restype, argtypes); every symbol include/splosh_q4.h declares.
SIGNATURES = {
    "splosh_q4_layout_init": (_int, [_i64, _i64, _int, _i64, _i64, ctypes.POINTER(Layout)]),
    "splosh_q4_layout_word_index": (_int, [ctypes.POINTER(Layout), _i64, _i64, ctypes.POINTER(_i64)]),
    "splosh_q4_layout_nibble_shift": (_int, [ctypes.POINTER(Layout), _i64, _i64, ctypes.POINTER(ctypes.c_uint32)]),
    "splosh_q4_layout_sidecar_index": (_int, [ctypes.POINTER(Layout), _i64, _i64, ctypes.POINTER(_i64)]),
    "splosh_q4_shape_validate": (_int, [_i64, _i64, _i64, ctypes.POINTER(Layout)]),
    "splosh_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "splosh_status_string": (ctypes.c_char_p, [_int]),
    "splosh_last_error": (ctypes.c_char_p, []),
    "splosh_version": (ctypes.c_char_p, []),
    "splosh_gemm_q4": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, ctypes.POINTER(Layout), _vp]),
    "splosh_q4_gemm": (_int, [ctypes.POINTER(Q4Weight), _vp, _i64, _vp, _i64, _int, _vp, _i64, _int, _vp, _sz, _vp]),
    "splosh_q5k_embed": (_int, [ctypes.POINTER(Q5KWeight), _vp, _i64, _vp, _i64, _int, _vp]),
    "splosh_q4k_embed": (_int, [ctypes.POINTER(Q5KWeight), _vp, _i64, _vp, _i64, _int, _vp]),
    "splosh_gguf_embed": (_int, [_int, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _int, _vp]),
    "splosh_q4_gemm_emit": (_int, [ctypes.POINTER(Q4Weight), _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp,
                                     _vp, _int, _vp, _sz, _vp]),
    "splosh_q4_gemm_noalloc": (_int, [ctypes.POINTER(Q4Weight), _vp, _i64, _vp, _i64, _int, _vp, _i64, _int, _vp]),
    "splosh_q4_mlp_in": (_int, [ctypes.POINTER(Q4Weight), ctypes.POINTER(Q4Weight), _vp, _i64, _vp, _i64, _int,
                                _i64, _int, _vp, _sz, _vp]),
    "splosh_q4_dequant": (_int, [ctypes.POINTER(Q4Weight), _vp, _vp]),
    "splosh_q4_gemm_group": (_int, [ctypes.POINTER(Q4Weight), _int, _vp, _i64, ctypes.POINTER(_vp),
                                    ctypes.POINTER(_i64), _int, _i64, _int, _vp, _sz, _vp]),
    "splosh_tile128": (_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "splosh_untile128": (_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "splosh_q5k_gemm": (_int, [ctypes.POINTER(Q5KWeight), _vp, _i64, _vp, _i64, _int, _vp, _i64, _int, _vp, _sz,
                               _vp]),
    "splosh_q5k_dequant": (_int, [ctypes.POINTER(Q5KWeight), _vp, _vp]),
    "splosh_q5k_repack": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "splosh_q5k_unpack": (_int, [_vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "splosh_q4k_gemm": (_int, [ctypes.POINTER(Q5KWeight), _vp, _i64, _vp, _i64, _int, _vp, _i64, _int, _vp, _sz,
                               _vp]),
    "splosh_q4k_dequant": (_int, [ctypes.POINTER(Q5KWeight), _vp, _vp]),
    "splosh_gguf_gemm": (_int, [_int, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _int, _vp, _i64, _vp, _sz, _vp]),
    "splosh_gguf_dequant": (_int, [_int, _vp, _i64, _i64, _vp, _vp]),
    "splosh_gguf_rows32_bytes": (_sz, [_int, _i64, _i64]),
    "splosh_gguf_repack_rows32": (_int, [_int, _vp, _i64, _i64, _vp, _vp]),
    "splosh_q5k_gemm_heads": (_int, [ctypes.POINTER(Q5KWeight), _int, _vp, _i64, _vp, _i64, _int, _vp, _i64, _int,
                                     _vp, _sz, _vp]),
    "splosh_q4k_gemm_heads": (_int, [ctypes.POINTER(Q5KWeight), _int, _vp, _i64, _vp, _i64, _int, _vp, _i64, _int,
                                     _vp, _sz, _vp]),
    "splosh_gguf_gemm_heads": (_int, [_int, _vp, _i64, _i64, _int, _vp, _i64, _vp, _i64, _int, _vp, _i64, _vp, _sz,
                                      _vp]),
    "splosh_heads_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "splosh_q4k_repack": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "splosh_q4k_unpack": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "splosh_q4_embed": (_int, [ctypes.POINTER(Q4Weight), _vp, _i64, _vp, _i64, _int, _vp]),
    "splosh_prepare_operand": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "splosh_silu_mul_operand": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "splosh_emit_operand": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "splosh_row_inv": (_int, [_vp, _i64, _i64, _i64, ctypes.c_float, _vp, _vp]),
}

_lib = None


def lib():
    """The loaded library. Raises SploshLibraryError if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise SploshLibraryError(
                f"{LIB_PATH} is missing: build it with `python -m splosh_amd.build` (no fallback exists)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def last_error():
    return lib().splosh_last_error().decode()


def check(status, error_class=None):
    if status == OK:
        return
    msg = last_error()
    if error_class is None:
        error_class = GemmQ4Error if 1 <= status <= 8 else (Q4BufferLayoutError if 9 <= status <= 11 else SploshError)
    raise error_class(status, msg)
