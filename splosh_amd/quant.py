"""Format contract of the q4 path, as the reference's SploshQuant / SploshModel types expose it.

``Q4BufferLayout`` and ``GemmQ4Shape`` are thin views of the C++ implementations behind the C ABI
(``splosh_q4_layout_init`` and ``splosh_q4_shape_validate``), so the host checks that guard every
launch are the ones tested here. Errors raise the reference's error cases by name.
"""
import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import GemmQ4Error, Q4BufferLayoutError  # noqa: F401

GROUP_SIZE = 64             # MlxAffine.groupSize (Quant/MlxAffine.swift:22)
WORD_BYTES = 4              # Q4BufferLayout.wordBytes (Quant/Q4BufferLayout.swift:31)
DEFAULT_ROW_ALIGNMENT = 128  # Q4BufferLayout.defaultRowAlignment (:32)
TILE_ROWS = 128             # Converter.tileRows (Model/Retile.swift:17)

ROWS_BY_K = _lib.ROWS_BY_K
K_BY_COLUMNS = _lib.K_BY_COLUMNS


class Q4BufferLayout:
    """Q4BufferLayout (Quant/Q4BufferLayout.swift:29-130)."""

    def __init__(self, rows, logical_k, orientation=ROWS_BY_K, row_stride_bytes=None,
                 row_alignment=DEFAULT_ROW_ALIGNMENT):
        self._c = _lib.Layout()
        st = _lib.lib().splosh_q4_layout_init(rows, logical_k, orientation, row_stride_bytes or 0,
                                              row_alignment, ctypes.byref(self._c))
        _lib.check(st, Q4BufferLayoutError)

    def __getattr__(self, name):
        c = object.__getattribute__(self, "_c")
        return getattr(c, name)

    @property
    def packed_word_count(self):
        return (self.rows if self.orientation == ROWS_BY_K else self.logical_k) * self.row_stride_words

    @property
    def sidecar_count(self):
        return self.rows * self.group_stride

    def word_index(self, row, k):
        out = ctypes.c_int64()
        _lib.check(_lib.lib().splosh_q4_layout_word_index(ctypes.byref(self._c), row, k, ctypes.byref(out)),
                   Q4BufferLayoutError)
        return out.value

    def nibble_shift(self, row, k):
        out = ctypes.c_uint32()
        _lib.check(_lib.lib().splosh_q4_layout_nibble_shift(ctypes.byref(self._c), row, k, ctypes.byref(out)),
                   Q4BufferLayoutError)
        return out.value

    def sidecar_index(self, row, k):
        out = ctypes.c_int64()
        _lib.check(_lib.lib().splosh_q4_layout_sidecar_index(ctypes.byref(self._c), row, k, ctypes.byref(out)),
                   Q4BufferLayoutError)
        return out.value

    @property
    def c(self):
        return self._c


@dataclass(frozen=True)
class GemmQ4Shape:
    """GemmQ4Shape (Model/Gemm.swift:8-41): A[rows, inner] x dequant(Q)[inner, columns]."""

    rows: int
    columns: int
    inner: int

    def __post_init__(self):
        if self.rows <= 0 or self.columns <= 0 or self.inner <= 0:
            raise GemmQ4Error(1, "rows, columns and inner must be positive")

    def validate(self, layout: Q4BufferLayout):
        _lib.check(_lib.lib().splosh_q4_shape_validate(self.rows, self.columns, self.inner,
                                                        ctypes.byref(layout.c)), GemmQ4Error)


def q4_bytes(n, k):
    """Algorithmic bytes of an N x K q4 g64 weight: N K / 2 codes plus N (K / 64) bf16 scale and bias."""
    return n * k // 2 + n * (k // GROUP_SIZE) * 4


def q5k_bytes(n, k):
    """Bytes of an N x K Q5_K weight: 176 bytes per 256 elements (plane0 + plane1 + meta)."""
    return n * (k // 256) * 176
