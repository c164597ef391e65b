"""splosh_amd -- MI355X (gfx950) quantized-weight matmul path: MLX affine q4 (group 64) and GGUF
Q5_K GEMV/GEMM as hand-written HIP kernels behind a C ABI (include/splosh_q4.h).

The compute is in libsplosh_q4.so; this package binds it (``_lib``), mirrors the reference's
format contract (``quant``) and exposes operator entry points on torch device tensors
(``runtime``). Build the library with ``python -m splosh_amd.build``.
"""
from . import _lib, quant  # noqa: F401
from ._lib import GemmQ4Error, Q4BufferLayoutError, SploshError, SploshLibraryError  # noqa: F401
from .quant import GemmQ4Shape, Q4BufferLayout  # noqa: F401

__version__ = "0.1.0"


def library_path():
    return str(_lib.LIB_PATH)
