"""Operator entry points of the q4 / Q5_K path on torch device tensors.

PyTorch-ROCm supplies device memory and streams only; every computation is a call into
libsplosh_q4.so through its C ABI. The names follow the reference's host API:

* ``Q4GemmRuntime.dispatch`` -- Runtime/Q4Runtime.swift:94-145 (gemm_q4, fp32 out, synchronous).
* ``Engine.gemm`` / ``Engine.mlp_in`` -- Runtime/Engine.swift:1652, :1911 (stream-ordered).
* ``dequant``, ``tile128``, ``q5k_repack`` -- DequantOracle.dequantize, Converter.tile,
  GgufPlanes.repack on the device.

Buffer-size checks (GemmQ4Error.bufferTooSmall) happen here because the C ABI sees raw pointers.
"""
import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import GemmQ4Error, SploshError
from .quant import GROUP_SIZE, TILE_ROWS, GemmQ4Shape, Q4BufferLayout

AUTO = _lib.KERNEL_AUTO
STREAM = _lib.KERNEL_STREAM
DEQUANT = _lib.KERNEL_DEQUANT
TILE = _lib.KERNEL_TILE
SCALAR = _lib.KERNEL_SCALAR
PREFILL = _lib.KERNEL_PREFILL
ROW_MAJOR = _lib.ROW_MAJOR
TILED128 = _lib.TILED128


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _require(t, nbytes, name):
    # The bytes the pointer may address: to the end of the tensor's storage (a strided view of a
    # larger buffer reaches past its own elements).
    have = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()
    if have < nbytes:
        raise GemmQ4Error(8, f"bufferTooSmall(name: {name}, expected: {nbytes}, observed: {have})")
    if not t.is_cuda:
        raise SploshError(12, f"{name} is not a device tensor")


def _dtype_code(dtype):
    if dtype == torch.float32:
        return _lib.F32
    if dtype == torch.bfloat16:
        return _lib.BF16
    raise SploshError(13, f"unsupported output dtype {dtype}")


@dataclass
class Q4Weight:
    """A resident MLX affine q4 weight (the reference's Q4Handle): int32 packed words, bf16 scale
    and bias sidecars (as int16 or bfloat16 tensors), `rows` outputs x `inner` inputs."""

    packed: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    rows: int
    inner: int
    order: int = TILED128
    row_stride_words: int = 0

    def __post_init__(self):
        groups = (self.inner + GROUP_SIZE - 1) // GROUP_SIZE
        if self.order == TILED128:
            words = self.rows * groups * 8
        else:
            if self.row_stride_words == 0:
                self.row_stride_words = ((self.inner + 7) // 8 * 4 + 127) // 128 * 32
            words = self.rows * self.row_stride_words
        _require(self.packed, words * 4, "packed")
        _require(self.scales, self.rows * groups * 2, "scales")
        _require(self.biases, self.rows * groups * 2, "biases")

    def c(self):
        return _lib.Q4Weight(self.packed.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr(), self.rows,
                             self.inner, self.row_stride_words, self.order, 0)

    @property
    def nbytes(self):
        """Algorithmic bytes: N K / 2 codes + N (K / 64) * 4 sidecar bytes."""
        return self.rows * self.inner // 2 + self.rows * (self.inner // GROUP_SIZE) * 4


@dataclass
class Q5KWeight:
    """A GGUF Q5_K weight in plane form (Model/GgufPlanes.swift:8-20)."""

    plane0: torch.Tensor
    plane1: torch.Tensor
    meta: torch.Tensor
    rows: int
    inner: int

    def __post_init__(self):
        groups = self.inner // 32
        _require(self.plane0, self.rows * groups * 16, "plane0")
        _require(self.plane1, self.rows * groups * 4, "plane1")
        _require(self.meta, self.rows * (self.inner // 256) * 16, "meta")

    def c(self):
        return _lib.Q5KWeight(self.plane0.data_ptr(), self.plane1.data_ptr(), self.meta.data_ptr(), self.rows,
                              self.inner)

    @property
    def nbytes(self):
        return self.rows * (self.inner // 256) * 176


@dataclass
class Q4KWeight:
    """A GGUF Q4_K weight in plane form (GgufPlanes.swift:64: plane0 and meta, no plane1)."""

    plane0: torch.Tensor
    meta: torch.Tensor
    rows: int
    inner: int

    def __post_init__(self):
        _require(self.plane0, self.rows * (self.inner // 32) * 16, "plane0")
        _require(self.meta, self.rows * (self.inner // 256) * 16, "meta")

    def c(self):
        return _lib.Q5KWeight(self.plane0.data_ptr(), None, self.meta.data_ptr(), self.rows, self.inner)

    @property
    def nbytes(self):
        return self.rows * (self.inner // 256) * 144


def _on(stream):
    """The stream a call's kernels run on (the caller's, else torch's current one)."""
    return stream if stream is not None else torch.cuda.current_stream()


def _out(a, rows, n, out, out_dtype, stream=None):
    if out is None:
        # Allocated on the stream the kernel writes it from, so torch's caching allocator orders
        # any reuse of the block after that kernel.
        with torch.cuda.stream(_on(stream)):
            out = torch.empty((rows, n), dtype=out_dtype, device=a.device)
    return out


# ggml type id -> (block elements, block bytes) of the formats kept in native blocks
# (GgufQuant.swift:13-48): Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS.
GGUF_NATIVE = {8: (32, 34), 11: (256, 110), 14: (256, 210), 20: (32, 18), 21: (256, 110), 23: (256, 136)}


# splosh_gguf_gemm's layout flag: the ROWS32 order of the native blocks (splosh_gguf_repack_rows32).
GGUF_ROWS32 = 0x100


@dataclass
class GgufWeight:
    """A GGUF weight in native blocks (rows x inner): in the order its file holds them (rows back to
    back), or with rows32=True in the ROWS32 order of gguf_repack_rows32 (the units of 256
    elements of 32 consecutive rows interleaved, rows padded to a multiple of 32)."""

    native: torch.Tensor
    gguf_type: int
    rows: int
    inner: int
    rows32: bool = False

    def __post_init__(self):
        if self.gguf_type not in GGUF_NATIVE:
            raise SploshError(13, f"ggml type {self.gguf_type} is not kept in native blocks")
        elems, size = GGUF_NATIVE[self.gguf_type]
        stored = (self.rows + 31) // 32 * 32 if self.rows32 else self.rows
        _require(self.native, stored * (self.inner // elems) * size, "native")

    @property
    def type_id(self):
        """The type id the entry points take: the ggml id, with the layout flag for ROWS32."""
        return self.gguf_type | (GGUF_ROWS32 if self.rows32 else 0)


def gguf_repack_rows32(w, stream=None):
    """splosh_gguf_repack_rows32: the same weight in the ROWS32 order (a new device tensor)."""
    if w.rows32:
        raise SploshError(2, "the weight is already in the ROWS32 order")
    nbytes = _lib.lib().splosh_gguf_rows32_bytes(w.gguf_type, w.rows, w.inner)
    if nbytes == 0:
        raise SploshError(2, "no ROWS32 form for this type or shape (inner % 256 != 0)")
    out = torch.empty(nbytes, dtype=torch.uint8, device=w.native.device)
    _lib.check(_lib.lib().splosh_gguf_repack_rows32(w.gguf_type, _ptr(w.native), w.rows, w.inner, _ptr(out),
                                                    _stream(stream)))
    return GgufWeight(out, w.gguf_type, w.rows, w.inner, rows32=True)


def workspace_bytes(rows, columns, inner):
    """splosh_workspace_bytes: the split-K scratch the kernels can use for this shape (0: none)."""
    return _lib.lib().splosh_workspace_bytes(rows, columns, inner)


def heads_workspace_bytes(rows, columns, inner):
    """splosh_heads_workspace_bytes: the workspace a head-ordered GGUF GEMM needs."""
    return _lib.lib().splosh_heads_workspace_bytes(rows, columns, inner)


class _Scratch:
    """The split-K scratch of one call: (pointer, bytes), and the tensor that owns it, held by the
    caller until the kernel has been launched."""

    def __init__(self, ptr, nbytes, owner=None):
        self.ptr, self.nbytes, self.owner = ptr, nbytes, owner

    def __iter__(self):
        return iter((self.ptr, self.nbytes))


def _workspace(workspace, rows, n, inner, device, stream=None, heads=False):
    """The split-K scratch of the kernels: the caller's tensor (an empty one: none), or a fresh one
    from torch's stream-ordered allocator sized by splosh_workspace_bytes. A fresh one is
    zero-filled and allocated on the stream the kernel runs on, so the fill is ordered before the
    kernel; the caller keeps the returned object (and with it the tensor) until the kernel has
    been launched, after which the allocator hands the block out again only to work ordered after
    that kernel on the same stream."""
    if workspace is not None and workspace.numel() == 0:
        return _Scratch(None, 0)
    if workspace is not None:
        return _Scratch(_ptr(workspace), workspace.numel() * workspace.element_size(), workspace)
    need = (_lib.lib().splosh_heads_workspace_bytes if heads else _lib.lib().splosh_workspace_bytes)(rows, n, inner)
    if need == 0:
        return _Scratch(None, 0)
    with torch.cuda.stream(_on(stream)):
        buf = torch.zeros(need, dtype=torch.uint8, device=device)
    return _Scratch(_ptr(buf), need, buf)


def gemm(w, a, out=None, residual=None, out_dtype=torch.bfloat16, kernel=AUTO, rows=None, stream=None,
         workspace=None, key_heads=0):
    """Engine.gemm (Runtime/Engine.swift:1652-1806): out = a @ dequant(w)^T (+ residual).

    ``a`` is bf16 [rows, inner] (row stride a.stride(0)); ``out`` [rows, w.rows] in fp32 or bf16;
    ``residual`` may be ``out`` itself. ``key_heads`` > 0 (GGUF weights only): the weight's inner
    columns are in a GGUF file's value-head order and the activations in the engine's (the `heads`
    kernels, engine_gguf.metal:55-72)."""
    rows = a.shape[0] if rows is None else rows
    if a.dtype != torch.bfloat16:
        raise SploshError(13, "activations must be bf16")
    if a.stride(-1) != 1:
        raise SploshError(1, "activation rows must be contiguous")
    out = _out(a, rows, w.rows, out, out_dtype, stream)
    _require(a, ((rows - 1) * a.stride(0) + w.inner) * 2, "a")
    _require(out, ((rows - 1) * out.stride(0) + w.rows) * out.element_size(), "output")
    if residual is not None:
        if residual.dtype != out.dtype or residual.stride(0) != out.stride(0):
            raise SploshError(13, "residual must match the output's dtype and row stride")
    if key_heads and isinstance(w, Q4Weight):
        raise SploshError(13, "the value-head order applies to GGUF weights only")
    scratch = _workspace(workspace, rows, w.rows, w.inner, a.device, stream, heads=bool(key_heads))  # held until the launch
    ws, ws_bytes = scratch
    if isinstance(w, GgufWeight):
        if key_heads:
            st = _lib.lib().splosh_gguf_gemm_heads(w.type_id, _ptr(w.native), w.rows, w.inner, key_heads, _ptr(a),
                                                   a.stride(0), _ptr(out), out.stride(0), _dtype_code(out.dtype),
                                                   _ptr(residual), rows, ws, ws_bytes, _stream(stream))
        else:
            st = _lib.lib().splosh_gguf_gemm(w.type_id, _ptr(w.native), w.rows, w.inner, _ptr(a), a.stride(0),
                                             _ptr(out), out.stride(0), _dtype_code(out.dtype), _ptr(residual),
                                             rows, ws, ws_bytes, _stream(stream))
        _lib.check(st)
        return out
    wc = w.c()
    if key_heads:
        fn = _lib.lib().splosh_q4k_gemm_heads if isinstance(w, Q4KWeight) else _lib.lib().splosh_q5k_gemm_heads
        _lib.check(fn(ctypes.byref(wc), key_heads, _ptr(a), a.stride(0), _ptr(out), out.stride(0),
                      _dtype_code(out.dtype), _ptr(residual), rows, kernel, ws, ws_bytes, _stream(stream)))
        return out
    if isinstance(w, Q4Weight):
        st = _lib.lib().splosh_q4_gemm(ctypes.byref(wc), _ptr(a), a.stride(0), _ptr(out), out.stride(0),
                                       _dtype_code(out.dtype), _ptr(residual), rows, kernel, ws, ws_bytes,
                                       _stream(stream))
    else:
        fn = _lib.lib().splosh_q4k_gemm if isinstance(w, Q4KWeight) else _lib.lib().splosh_q5k_gemm
        st = fn(ctypes.byref(wc), _ptr(a), a.stride(0), _ptr(out), out.stride(0), _dtype_code(out.dtype),
                _ptr(residual), rows, kernel, ws, ws_bytes, _stream(stream))
    _lib.check(st)
    return out


def gemm_group(weights, a, outs=None, out_dtype=torch.bfloat16, kernel=AUTO, rows=None, stream=None,
               workspace=None):
    """Several projections of one activation in one launch (the reference's concurrent encoder of a
    layer's independent projections, Engine.swift:1402, 1131-1140): [a @ dequant(w)^T for w in
    weights], each in its own output. Returns the outputs."""
    rows = a.shape[0] if rows is None else rows
    if a.dtype != torch.bfloat16 or a.stride(-1) != 1:
        raise SploshError(13, "activations must be bf16 with contiguous rows")
    weights = list(weights)
    if outs is None:
        outs = [None] * len(weights)
    outs = [_out(a, rows, w.rows, o, out_dtype, stream) for w, o in zip(weights, outs)]
    _require(a, ((rows - 1) * a.stride(0) + weights[0].inner) * 2, "a")
    for w, o in zip(weights, outs):
        _require(o, ((rows - 1) * o.stride(0) + w.rows) * o.element_size(), "output")
        if o.dtype != outs[0].dtype:
            raise SploshError(13, "grouped outputs must share one dtype")
    scratch = _workspace(workspace, rows, sum(w.rows for w in weights), weights[0].inner, a.device, stream)
    ws, ws_bytes = scratch
    wcs = (_lib.Q4Weight * len(weights))(*[w.c() for w in weights])
    out_ptrs = (ctypes.c_void_p * len(outs))(*[_ptr(o) for o in outs])
    ldcs = (ctypes.c_int64 * len(outs))(*[o.stride(0) for o in outs])
    _lib.check(_lib.lib().splosh_q4_gemm_group(wcs, len(weights), _ptr(a), a.stride(0), out_ptrs, ldcs,
                                               _dtype_code(outs[0].dtype), rows, kernel, ws, ws_bytes,
                                               _stream(stream)))
    return outs


def gemm_emit(w, a, norm_weight, out=None, residual=None, kernel=AUTO, rows=None, stream=None, workspace=None):
    """Engine.gemm with emit (engine_na.metal:322-473): out = a @ dequant(w)^T (+ residual), fp32,
    and the next RMSNorm's operand from it: (bf16 out * norm_weight, per-64 sums of those values,
    per-64 sums of out^2). Returns (out, values, sums, squares)."""
    rows = a.shape[0] if rows is None else rows
    if a.dtype != torch.bfloat16 or a.stride(-1) != 1:
        raise SploshError(13, "activations must be contiguous bf16 rows")
    out = _out(a, rows, w.rows, out, torch.float32, stream)
    if out.dtype != torch.float32:
        raise SploshError(13, "the emitting projection writes fp32")
    _require(a, ((rows - 1) * a.stride(0) + w.inner) * 2, "a")
    _require(out, ((rows - 1) * out.stride(0) + w.rows) * 4, "output")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() < w.rows:
        raise SploshError(13, "norm_weight must be bf16 with one value a column")
    with torch.cuda.stream(_on(stream)):
        values = torch.empty((rows, w.rows), dtype=torch.bfloat16, device=a.device)
        sums = torch.empty((rows, w.rows // 64), dtype=torch.float32, device=a.device)
        squares = torch.empty_like(sums)
    wc = w.c()
    scratch = _workspace(workspace, rows, w.rows, w.inner, a.device, stream)  # held until the launch
    ws, ws_bytes = scratch
    _lib.check(_lib.lib().splosh_q4_gemm_emit(ctypes.byref(wc), _ptr(a), a.stride(0), _ptr(out), out.stride(0),
                                              _ptr(residual), rows, _ptr(norm_weight), _ptr(values), values.stride(0),
                                              _ptr(sums), _ptr(squares), kernel, ws, ws_bytes, _stream(stream)))
    return out, values, sums, squares


def mlp_in(gate, up, a, out=None, out_dtype=torch.bfloat16, kernel=AUTO, rows=None, stream=None, workspace=None):
    """Engine.mlpIn (Runtime/Engine.swift:1911-1966): out = silu(a @ gate^T) * (a @ up^T), one
    pass over the activations for both weights."""
    rows = a.shape[0] if rows is None else rows
    if a.dtype != torch.bfloat16 or a.stride(-1) != 1:
        raise SploshError(13, "activations must be contiguous bf16 rows")
    out = _out(a, rows, gate.rows, out, out_dtype, stream)
    _require(a, ((rows - 1) * a.stride(0) + gate.inner) * 2, "a")
    _require(out, ((rows - 1) * out.stride(0) + gate.rows) * out.element_size(), "output")
    gc, uc = gate.c(), up.c()
    scratch = _workspace(workspace, rows, gate.rows, gate.inner, a.device, stream)  # held until the launch
    ws, ws_bytes = scratch
    st = _lib.lib().splosh_q4_mlp_in(ctypes.byref(gc), ctypes.byref(uc), _ptr(a), a.stride(0), _ptr(out),
                                     out.stride(0), _dtype_code(out.dtype), rows, kernel, ws, ws_bytes,
                                     _stream(stream))
    _lib.check(st)
    return out


def dequant(w, out=None, stream=None):
    """DequantOracle.dequantize / GgufTensorType.decode on the device: fp32 [rows, inner]."""
    if out is None:
        dev = (w.packed.device if isinstance(w, Q4Weight) else w.native.device if isinstance(w, GgufWeight)
               else w.plane0.device)
        out = torch.empty((w.rows, w.inner), dtype=torch.float32, device=dev)
    _require(out, w.rows * w.inner * 4, "output")
    if isinstance(w, GgufWeight):
        _lib.check(_lib.lib().splosh_gguf_dequant(w.type_id, _ptr(w.native), w.rows, w.inner, _ptr(out),
                                                  _stream(stream)))
        return out
    wc = w.c()
    fn = (_lib.lib().splosh_q4_dequant if isinstance(w, Q4Weight) else
          _lib.lib().splosh_q4k_dequant if isinstance(w, Q4KWeight) else _lib.lib().splosh_q5k_dequant)
    _lib.check(fn(ctypes.byref(wc), _ptr(out), _stream(stream)))
    return out


def tile128(src, rows, groups, element_bytes, inverse=False, out=None, stream=None):
    """Converter.tile (Model/Retile.swift:135-153) on the device (or its inverse)."""
    if out is None:
        out = torch.empty_like(src)
    nbytes = rows * groups * element_bytes
    _require(src, nbytes, "src")
    _require(out, nbytes, "dst")
    fn = _lib.lib().splosh_untile128 if inverse else _lib.lib().splosh_tile128
    _lib.check(fn(_ptr(src), _ptr(out), rows, groups, element_bytes, _stream(stream)))
    return out


def q4_to_tiled(w, stream=None):
    """A row-major (unpadded) q4 weight retiled to the 128-row layout the kernels prefer."""
    if w.order == TILED128:
        return w
    groups = w.inner // GROUP_SIZE
    if w.row_stride_words != w.inner // 8:
        packed = w.packed.view(w.rows, -1)[:, : w.inner // 8].contiguous()
    else:
        packed = w.packed
    tp = tile128(packed, w.rows, groups, 32, stream=stream)
    ts = tile128(w.scales, w.rows, groups, 2, stream=stream)
    tb = tile128(w.biases, w.rows, groups, 2, stream=stream)
    return Q4Weight(tp, ts, tb, w.rows, w.inner, TILED128)


def q5k_repack(native, rows, inner, stream=None):
    """GgufPlanes.repack for Q5_K on the device: native uint8 blocks -> Q5KWeight."""
    groups = inner // 32
    dev = native.device
    p0 = torch.empty(rows * groups * 16, dtype=torch.uint8, device=dev)
    p1 = torch.empty(rows * groups * 4, dtype=torch.uint8, device=dev)
    meta = torch.empty(rows * (inner // 256) * 16, dtype=torch.uint8, device=dev)
    _require(native, rows * (inner // 256) * 176, "native")
    _lib.check(_lib.lib().splosh_q5k_repack(_ptr(native), rows, inner, _ptr(p0), _ptr(p1), _ptr(meta),
                                            _stream(stream)))
    return Q5KWeight(p0, p1, meta, rows, inner)


def q5k_unpack(w, stream=None):
    native = torch.empty(w.rows * (w.inner // 256) * 176, dtype=torch.uint8, device=w.plane0.device)
    _lib.check(_lib.lib().splosh_q5k_unpack(_ptr(w.plane0), _ptr(w.plane1), _ptr(w.meta), w.rows, w.inner,
                                            _ptr(native), _stream(stream)))
    return native


def q4k_repack(native, rows, inner, stream=None):
    """GgufPlanes.repack for Q4_K on the device: native 144-byte blocks -> Q4KWeight."""
    dev = native.device
    p0 = torch.empty(rows * (inner // 32) * 16, dtype=torch.uint8, device=dev)
    meta = torch.empty(rows * (inner // 256) * 16, dtype=torch.uint8, device=dev)
    _require(native, rows * (inner // 256) * 144, "native")
    _lib.check(_lib.lib().splosh_q4k_repack(_ptr(native), rows, inner, _ptr(p0), _ptr(meta), _stream(stream)))
    return Q4KWeight(p0, meta, rows, inner)


def q4k_unpack(w, stream=None):
    native = torch.empty(w.rows * (w.inner // 256) * 144, dtype=torch.uint8, device=w.plane0.device)
    _lib.check(_lib.lib().splosh_q4k_unpack(_ptr(w.plane0), _ptr(w.meta), w.rows, w.inner, _ptr(native),
                                            _stream(stream)))
    return native


class Q4GemmRuntime:
    """Q4GemmRuntime (Runtime/Q4Runtime.swift:29-157): the oracle-grade gemm_q4 submission API."""

    def dispatch(self, shape: GemmQ4Shape, layout: Q4BufferLayout, a, packed, scales, biases, output, stream=None):
        """Validate, encode gemm_q4 (one thread per output), and wait (Q4Runtime.swift:94-145)."""
        shape.validate(layout)
        _require(a, shape.rows * shape.inner * 2, "a")
        _require(packed, layout.packed_word_count * 4, "packed")
        _require(scales, layout.sidecar_count * 2, "scales")
        _require(biases, layout.sidecar_count * 2, "biases")
        _require(output, shape.rows * shape.columns * 4, "output")
        st = _lib.lib().splosh_gemm_q4(_ptr(a), _ptr(packed), _ptr(scales), _ptr(biases), _ptr(output), shape.rows,
                                       shape.columns, shape.inner, ctypes.byref(layout.c), _stream(stream))
        _lib.check(st)
        (stream or torch.cuda.current_stream()).synchronize()


class Engine:
    """The GEMM entry points of the reference's Engine (Runtime/Engine.swift:1652, :1911), stream
    ordered; `kernel` replaces the reference's SPLOSH_* kernel-selection environment variables."""

    def __init__(self, kernel=AUTO, stream=None):
        self.kernel = kernel
        self.stream = stream

    def gemm(self, w, input, output, residual=False, rows=None):
        return gemm(w, input, out=output, residual=output if residual else None, kernel=self.kernel, rows=rows,
                    stream=self.stream)

    def mlp_in(self, gate, up, input, output, rows=None):
        return mlp_in(gate, up, input, out=output, kernel=self.kernel, rows=rows, stream=self.stream)


def version():
    return _lib.lib().splosh_version().decode()


# ---- operand producers (the steps either side of a GEMM) ----------------------------------------


def _f32_rows(t, name):
    if t.dtype != torch.float32 or t.dim() != 2 or t.stride(1) != 1:
        raise SploshError(13, f"{name} must be fp32 [rows, dim] with contiguous rows")
    return t


def _operand_out(x, out, sums):
    rows, dim = x.shape
    if out is None:
        out = torch.empty((rows, dim), dtype=torch.bfloat16, device=x.device)
    if sums is None:
        sums = torch.empty((rows, dim // 64), dtype=torch.float32, device=x.device)
    return out, sums


def prepare_operand(x, out=None, sums=None, stream=None):
    """sp_na_prepare (engine_na.metal:38-56): fp32 [rows, dim] -> (bf16 operand, per-64 sums)."""
    x = _f32_rows(x, "x")
    out, sums = _operand_out(x, out, sums)
    _lib.check(_lib.lib().splosh_prepare_operand(_ptr(x), x.stride(0), x.shape[0], x.shape[1], _ptr(out),
                                                 out.stride(0), _ptr(sums), _stream(stream)))
    return out, sums


def silu_mul_operand(gate, up, row_inv=None, out=None, sums=None, stream=None):
    """sp_silu_mul_na (engine.metal:200-218): bf16(silu(g s) (u s)) and its per-64 sums."""
    gate, up = _f32_rows(gate, "gate"), _f32_rows(up, "up")
    if up.shape != gate.shape or up.stride(0) != gate.stride(0):
        raise SploshError(13, "gate and up must share shape and row stride")
    out, sums = _operand_out(gate, out, sums)
    _lib.check(_lib.lib().splosh_silu_mul_operand(_ptr(gate), _ptr(up), gate.stride(0), _ptr(row_inv), gate.shape[0],
                                                  gate.shape[1], _ptr(out), out.stride(0), _ptr(sums),
                                                  _stream(stream)))
    return out, sums


def emit_operand(hidden, norm_weight, values=None, sums=None, squares=None, stream=None):
    """The next RMSNorm-ed GEMM's operand (engine_na.metal:26-36, 365-411): (bf16 hidden * weight,
    per-64 sums of it, per-64 sums of hidden^2)."""
    hidden = _f32_rows(hidden, "hidden")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() < hidden.shape[1]:
        raise SploshError(13, "norm_weight must be bf16 with dim values")
    values, sums = _operand_out(hidden, values, sums)
    if squares is None:
        squares = torch.empty_like(sums)
    _lib.check(_lib.lib().splosh_emit_operand(_ptr(hidden), hidden.stride(0), _ptr(norm_weight), hidden.shape[0],
                                              hidden.shape[1], _ptr(values), values.stride(0), _ptr(sums),
                                              _ptr(squares), _stream(stream)))
    return values, sums, squares


def row_inv(squares, dim, eps, out=None, stream=None):
    """sp_row_inv (engine.metal:222-233): 1 / sqrt(sum(squares[row]) / dim + eps)."""
    if squares.dtype != torch.float32 or not squares.is_contiguous():
        raise SploshError(13, "squares must be contiguous fp32 [rows, groups]")
    rows, groups = squares.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=squares.device)
    _lib.check(_lib.lib().splosh_row_inv(_ptr(squares), rows, groups, dim, float(eps), _ptr(out), _stream(stream)))
    return out


def embed(w, tokens, out=None, out_dtype=torch.float32, stream=None):
    """sp_embed_q4 (engine.metal:39-57) for a q4 table, sp_gguf_embed (engine_gguf.metal:302-318)
    for a GGUF one (planes or native blocks): rows tokens[i] of the decoded table, [count, inner].
    tokens: uint32 ids on the device (int32 tensors are taken as their bits); an id past the table
    gives zeros."""
    if tokens.dtype not in (torch.int32,) or not tokens.is_contiguous():
        raise SploshError(13, "tokens must be a contiguous int32 tensor of uint32 ids")
    count = tokens.numel()
    if out is None:
        out = torch.empty((count, w.inner), dtype=out_dtype, device=tokens.device)
    _require(out, ((count - 1) * out.stride(0) + w.inner) * out.element_size(), "output")
    if isinstance(w, GgufWeight):
        _lib.check(_lib.lib().splosh_gguf_embed(w.type_id, _ptr(w.native), w.rows, w.inner, _ptr(tokens), count,
                                                _ptr(out), out.stride(0), _dtype_code(out.dtype), _stream(stream)))
        return out
    wc = w.c()
    fn = (_lib.lib().splosh_q4_embed if isinstance(w, Q4Weight) else
          _lib.lib().splosh_q4k_embed if isinstance(w, Q4KWeight) else _lib.lib().splosh_q5k_embed)
    _lib.check(fn(ctypes.byref(wc), _ptr(tokens), count, _ptr(out), out.stride(0), _dtype_code(out.dtype),
                  _stream(stream)))
    return out
