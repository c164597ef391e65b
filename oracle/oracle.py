"""numpy front end of the C oracle (liborc_splosh.so) -- TEST INFRASTRUCTURE ONLY.

Every function here calls the C restatement in ``splosh_oracle.c``, which cites the reference
file:line it follows. Only tests, ``__graft_entry__.smoke()`` and bench.py's CPU baseline use it.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liborc_splosh.so"
_lib = None

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def build(force=False):
    """Compile the oracle with its Makefile (gcc -O2 -ffp-contract=off)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        L = _lib
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_bf16_halfup.restype = ctypes.c_uint16
        L.or_f32_to_bf16_halfup.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.or_f32_to_bf16_rne.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16_rne_n.argtypes = [_ptr, _ptr, _i64]
        L.or_q4_dequant_rowmajor.argtypes = [_ptr, _i64, _ptr, _ptr, _i64, _i64, _ptr]
        L.or_q4_dequant_tiled.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _ptr]
        L.or_tile128.argtypes = [_ptr, _ptr, _i64, _i64, _i64]
        L.or_gguf_decode.restype = ctypes.c_int
        L.or_gguf_decode.argtypes = [ctypes.c_int, _ptr, _i64, _ptr]
        L.or_gguf_block_bytes.restype = ctypes.c_int
        L.or_gguf_block_bytes.argtypes = [ctypes.c_int]
        L.or_iq3s_grid.restype = None
        L.or_iq3s_grid.argtypes = [_ptr]
        L.or_untile128.argtypes = [_ptr, _ptr, _i64, _i64, _i64]
        L.or_gemm_a_bf16_w_f32.argtypes = [_ptr, _i64, _ptr, _i64, _i64, _i64, _ptr]
        L.or_gemm_bf16.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _ptr]
        L.or_q4_gemm_rowmajor.argtypes = [_ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64,
                                          _i64, _i64, _ptr, ctypes.c_int]
        L.or_silu_mul.argtypes = [_ptr, _ptr, _i64, _ptr]
        L.or_q45k_decode.argtypes = [_ptr, _i64, ctypes.c_int, _ptr]
        L.or_q45k_repack.restype = ctypes.c_int
        L.or_q45k_repack.argtypes = [_ptr, _i64, _i64, ctypes.c_int, _ptr, _ptr, _ptr]
        L.or_q45k_unpack.restype = ctypes.c_int
        L.or_q45k_unpack.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, ctypes.c_int, _ptr]
        L.or_gguf_slot.restype = ctypes.c_int
        L.or_gguf_slot.argtypes = [ctypes.c_int]
        L.or_q45k_gemm_native.argtypes = [_ptr, _i64, _ptr, ctypes.c_int, _i64, _i64, _i64, _i64,
                                          _i64, _ptr, ctypes.c_int]
        L.or_prepare_operand.argtypes = [_ptr, _i64, _i64, _ptr, _ptr]
        L.or_silu_mul_operand.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr]
        L.or_emit_operand.argtypes = [_ptr, _ptr, _i64, _i64, _ptr, _ptr, _ptr]
        L.or_row_inv.argtypes = [_ptr, _i64, _i64, _i64, ctypes.c_float, _ptr]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- bf16 -----------------------------------------------------------------------------------

def bf16_to_f32(bits):
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(values):
    values = _c(values, np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_rne_n(_p(values), _p(out), values.size)
    return out


def f32_to_bf16_halfup(value):
    return int(lib().or_f32_to_bf16_halfup(float(value)))


# ---- MLX affine q4 --------------------------------------------------------------------------

def q4_dequant_rowmajor(words, stride_words, scales, biases, N, K):
    words = _c(words, np.uint32)
    scales = _c(scales, np.uint16)
    biases = _c(biases, np.uint16)
    out = np.empty((N, K), dtype=np.float32)
    lib().or_q4_dequant_rowmajor(_p(words), stride_words, _p(scales), _p(biases), N, K, _p(out))
    return out


def q4_dequant_tiled(words, scales, biases, N, K):
    words = _c(words, np.uint32)
    scales = _c(scales, np.uint16)
    biases = _c(biases, np.uint16)
    out = np.empty((N, K), dtype=np.float32)
    lib().or_q4_dequant_tiled(_p(words), _p(scales), _p(biases), N, K, _p(out))
    return out


def tile128(src, rows, groups, element_bytes):
    src = np.ascontiguousarray(src)
    dst = np.empty_like(src)
    lib().or_tile128(_p(src), _p(dst), rows, groups, element_bytes)
    return dst


def untile128(src, rows, groups, element_bytes):
    src = np.ascontiguousarray(src)
    dst = np.empty_like(src)
    lib().or_untile128(_p(src), _p(dst), rows, groups, element_bytes)
    return dst


def gemm_a_bf16_w_f32(a_bf16, w_f32):
    a = _c(a_bf16, np.uint16)
    w = _c(w_f32, np.float32)
    M, K = a.shape
    N = w.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    lib().or_gemm_a_bf16_w_f32(_p(a), K, _p(w), M, N, K, _p(out))
    return out


def gemm_bf16(a_bf16, b_bf16, M, N, K):
    a = _c(a_bf16, np.uint16)
    b = _c(b_bf16, np.uint16)
    out = np.empty((M, N), dtype=np.float32)
    lib().or_gemm_bf16(_p(a), _p(b), M, N, K, _p(out))
    return out


def q4_gemm_rowmajor(a_bf16, words, stride_words, scales, biases, N, K, n0=0, n1=None, threads=1):
    """Fused dequant + sequential fp32 dot over output columns [n0, n1); others are left NaN."""
    a = _c(a_bf16, np.uint16)
    M = a.shape[0]
    n1 = N if n1 is None else n1
    out = np.full((M, N), np.nan, dtype=np.float32)
    lib().or_q4_gemm_rowmajor(_p(a), a.shape[1], _p(_c(words, np.uint32)), stride_words,
                              _p(_c(scales, np.uint16)), _p(_c(biases, np.uint16)), M, N, K,
                              n0, n1, _p(out), threads)
    return out


def silu_mul(gate, up):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.empty_like(g)
    lib().or_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


# ---- operand producers (engine_na.metal:38-56, engine.metal:200-233, engine_na.metal:365-411) --

def prepare_operand(x):
    """sp_na_prepare: (bf16 bits [rows, inner], per-64 sums of the rounded values [rows, inner/64])."""
    x = _c(x, np.float32)
    rows, inner = x.shape
    out = np.empty((rows, inner), np.uint16)
    sums = np.empty((rows, inner // 64), np.float32)
    lib().or_prepare_operand(_p(x), rows, inner, _p(out), _p(sums))
    return out, sums


def silu_mul_operand(gate, up, row_inv=None):
    """sp_silu_mul_na: bf16(silu(g s) (u s)) and its per-64 sums; s = row_inv[row] or 1."""
    g, u = _c(gate, np.float32), _c(up, np.float32)
    rows, dim = g.shape
    inv = None if row_inv is None else _c(row_inv, np.float32)
    out = np.empty((rows, dim), np.uint16)
    sums = np.empty((rows, dim // 64), np.float32)
    lib().or_silu_mul_operand(_p(g), _p(u), None if inv is None else _p(inv), rows, dim, _p(out), _p(sums))
    return out, sums


def emit_operand(hidden, norm_weight_bits):
    """The next RMSNorm-ed GEMM's operand: (bf16 values, per-64 sums, per-64 sums of squares)."""
    h = _c(hidden, np.float32)
    w = _c(norm_weight_bits, np.uint16)
    rows, dim = h.shape
    values = np.empty((rows, dim), np.uint16)
    sums = np.empty((rows, dim // 64), np.float32)
    squares = np.empty((rows, dim // 64), np.float32)
    lib().or_emit_operand(_p(h), _p(w), rows, dim, _p(values), _p(sums), _p(squares))
    return values, sums, squares


def row_inv(squares, dim, eps):
    """sp_row_inv: 1 / sqrt(sum(squares[row]) / dim + eps)."""
    q = _c(squares, np.float32)
    rows, groups = q.shape
    inv = np.empty(rows, np.float32)
    lib().or_row_inv(_p(q), rows, groups, dim, eps, _p(inv))
    return inv


# ---- GGUF Q4_K / Q5_K -----------------------------------------------------------------------

def q45k_decode(blocks, fifth_bit=True):
    blocks = _c(blocks, np.uint8)
    size = 176 if fifth_bit else 144
    n = blocks.size // size
    out = np.empty(n * 256, dtype=np.float32)
    lib().or_q45k_decode(_p(blocks), n, int(fifth_bit), _p(out))
    return out


GGUF_BLOCK = {8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 20: (32, 18),
              21: (256, 110), 23: (256, 136)}


def iq3s_grid():
    """The oracle's IQ3_S codebook, 512 uint32 entries."""
    out = np.empty(512, dtype=np.uint32)
    lib().or_iq3s_grid(_p(out))
    return out


def gguf_decode(gguf_type, blocks):
    """Native GGUF blocks to float32 (or_gguf_decode: the reference decoder's op order)."""
    blocks = _c(blocks, np.uint8)
    elems, size = GGUF_BLOCK[gguf_type]
    n = blocks.size // size
    out = np.empty(n * elems, dtype=np.float32)
    if lib().or_gguf_decode(int(gguf_type), _p(blocks), n, _p(out)) != 0:
        raise ValueError(f"ggml type {gguf_type} is not decoded by the oracle")
    return out


def gguf_random_native(gguf_type, n, k, seed):
    """Rows of random native blocks with sane fp16 scales: every byte random, then each fp16
    field (Q8_0 / IQ4_NL / IQ4_XS / IQ3_S: d at 0; Q6_K: d at 208; Q3_K: d at 108) set to about 1e-3 (sign random in one
    block of four)."""
    elems, size = GGUF_BLOCK[gguf_type]
    blocks = n * k // elems
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(blocks, size), dtype=np.uint8)
    at = {14: 208, 11: 108}.get(gguf_type, 0)
    v = 1e-3 * (1 + 0.25 * rng.uniform(-1, 1, size=blocks))
    v = np.where(rng.integers(0, 4, size=blocks) == 0, -v, v).astype(np.float16)
    raw[:, at:at + 2] = v.view(np.uint8).reshape(blocks, 2)
    return raw.reshape(-1)


def gguf_slot(e):
    return int(lib().or_gguf_slot(int(e)))


def q45k_plane_sizes(N, K, fifth_bit=True):
    groups = K // 32
    return N * groups * 16, (N * groups * 4 if fifth_bit else 0), N * (K // 256) * 16


def q45k_repack(native, N, K, fifth_bit=True):
    native = _c(native, np.uint8)
    s0, s1, sm = q45k_plane_sizes(N, K, fifth_bit)
    p0 = np.zeros(s0, np.uint8)
    p1 = np.zeros(max(s1, 1), np.uint8)
    meta = np.zeros(sm, np.uint8)
    rc = lib().or_q45k_repack(_p(native), N, K, int(fifth_bit), _p(p0), _p(p1), _p(meta))
    if rc != 0:
        raise ValueError(f"Q{'5' if fifth_bit else '4'}_K {N} x {K} has no plane form")
    return p0, p1[:s1], meta


def q45k_unpack(p0, p1, meta, N, K, fifth_bit=True):
    size = 176 if fifth_bit else 144
    native = np.zeros(N * (K // 256) * size, np.uint8)
    p1 = _c(p1, np.uint8) if fifth_bit else np.zeros(1, np.uint8)
    rc = lib().or_q45k_unpack(_p(_c(p0, np.uint8)), _p(p1), _p(_c(meta, np.uint8)), N, K,
                              int(fifth_bit), _p(native))
    if rc != 0:
        raise ValueError("no plane form")
    return native


def q45k_gemm_native(a_bf16, native, N, K, fifth_bit=True, n0=0, n1=None, threads=1):
    a = _c(a_bf16, np.uint16)
    M = a.shape[0]
    n1 = N if n1 is None else n1
    out = np.full((M, N), np.nan, dtype=np.float32)
    lib().or_q45k_gemm_native(_p(a), a.shape[1], _p(_c(native, np.uint8)), int(fifth_bit), M, N, K,
                              n0, n1, _p(out), threads)
    return out


# ---- seeded synthetic inputs (the BASELINE distributions) -----------------------------------

def q4_random_weight(N, K, seed, stride_words=None):
    """Row-major padded MLX q4 weight: uniform random code words, scale = bf16(|N(0, 0.02)|),
    bias = bf16(N(0, 0.01)), generated with numpy's PCG64 from ``seed``."""
    rng = np.random.default_rng(seed)
    wpr = (K + 7) // 8
    stride = stride_words or ((wpr * 4 + 127) // 128 * 128) // 4
    words = np.zeros((N, stride), np.uint32)
    words[:, :wpr] = rng.integers(0, 2**32, size=(N, wpr), dtype=np.uint64).astype(np.uint32)
    if K % 8:
        words[:, wpr - 1] &= np.uint32((1 << (4 * (K % 8))) - 1)
    groups = (K + 63) // 64
    scales = f32_to_bf16_rne(np.abs(rng.normal(0, 0.02, size=(N, groups))).astype(np.float32))
    biases = f32_to_bf16_rne(rng.normal(0, 0.01, size=(N, groups)).astype(np.float32))
    return words, stride, scales, biases


def bf16_normal(shape, seed, std=1.0):
    rng = np.random.default_rng(seed)
    return f32_to_bf16_rne(rng.normal(0, std, size=shape).astype(np.float32))


class SplitMix64:
    """The seeded generator of the reference's GGUF kernel tests (GgufKernelTests.swift:35-46)."""

    MASK = (1 << 64) - 1

    def __init__(self, state):
        self.state = state & self.MASK

    def next(self):
        self.state = (self.state + 0x9E3779B97F4A7C15) & self.MASK
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & self.MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & self.MASK
        return z ^ (z >> 31)

    def unit(self):
        return np.float32((self.next() >> 40) - (1 << 23)) / np.float32(1 << 23)


def q45k_random_native(N, K, seed, fifth_bit=True):
    """Rows of random native blocks with the reference test's fp16 scale fields
    (GgufKernelTests.swift:49-82): every byte random, then d ~ 1e-4 (Q5_K; 2e-4 Q4_K) and
    dmin ~ 1.5e-3, each times (1 + 0.25 u), negative in one block of four.

    Vectorised: the byte stream is drawn from numpy's PCG64 (not SplitMix64, which is the
    reference's, used by ``q45k_random_native_splitmix`` for small cases)."""
    size = 176 if fifth_bit else 144
    blocks = N * K // 256
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(blocks, size), dtype=np.uint8)
    mags = (1e-4 if fifth_bit else 2e-4, 1.5e-3)
    for field, mag in zip((0, 2), mags):
        v = mag * (1 + 0.25 * rng.uniform(-1, 1, size=blocks))
        neg = rng.integers(0, 4, size=blocks) == 0
        v = np.where(neg, -v, v).astype(np.float16)
        raw[:, field:field + 2] = v.view(np.uint8).reshape(blocks, 2)
    return raw.reshape(-1)


def q45k_random_native_splitmix(N, K, seed, fifth_bit=True):
    """Exactly the reference test's generator (GgufKernelTests.swift:63-82), for small shapes."""
    size = 176 if fifth_bit else 144
    blocks = N * K // 256
    g = SplitMix64(seed)
    raw = np.array([g.next() & 0xFF for _ in range(blocks * size)], dtype=np.uint8).reshape(blocks, size)
    mags = (1e-4 if fifth_bit else 2e-4, 1.5e-3)
    for b in range(blocks):
        for field, mag in zip((0, 2), mags):
            value = np.float32(mag) * (np.float32(1) + np.float32(0.25) * g.unit())
            if g.next() & 3 == 0:
                value = -value
            raw[b, field:field + 2] = np.array([value], dtype=np.float16).view(np.uint8)
    return raw.reshape(-1)


# ---- GGUF conversion: value-head order and Q8_0 requantisation (GgufNames.swift, GgufConvert.swift)

def mlx_value_head(i, key_heads=16, value_heads=48):
    return lib().or_mlx_value_head(int(i), key_heads, value_heads)


def head_destination(unit, first, span, key_heads=16, value_heads=48):
    lib().or_head_destination.restype = _i64
    lib().or_head_destination.argtypes = [_i64, _i64, _i64, ctypes.c_int, ctypes.c_int]
    return lib().or_head_destination(unit, first, span, key_heads, value_heads)


def order_rows(native, rows, row_bytes, first=0, span=0, stored=None, key_heads=16, value_heads=48):
    """GgufConvert's row order: file row r at row head_destination(r); span 0: rows unchanged."""
    native = _c(native, np.uint8)
    stored = rows if stored is None else stored
    out = np.empty(stored * row_bytes, np.uint8)
    f = lib().or_order_rows
    f.argtypes = [_ptr, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _i64, _ptr]
    f(_p(native), rows, row_bytes, first, span, key_heads, value_heads, stored, _p(out))
    return out


def f32_to_f16_rne(values):
    v = np.ascontiguousarray(np.asarray(values, np.float32).reshape(-1))
    f = lib().or_f32_to_f16_rne
    f.restype = ctypes.c_uint16
    f.argtypes = [ctypes.c_float]
    return np.array([f(float(x)) for x in v], np.uint16)


def q8_0_blocks(values):
    v = _c(np.asarray(values, np.float32).reshape(-1), np.float32)
    out = np.empty(v.size // 32 * 34, np.uint8)
    f = lib().or_q8_0_blocks
    f.argtypes = [_ptr, _i64, _ptr]
    f(_p(v), v.size // 32, _p(out))
    return out


def head_gather(a_bits, key_heads=16):
    """out[m][k] = a[m][mlx_value_head(k / 128) 128 + k % 128]: the activations a head-ordered weight meets."""
    a = _c(a_bits, np.uint16)
    m, inner = a.shape
    out = np.empty_like(a)
    f = lib().or_head_gather
    f.argtypes = [_ptr, _i64, _i64, _i64, ctypes.c_int, _ptr]
    f(_p(a), inner, m, inner, key_heads, _p(out))
    return out
