"""GGUF files (llama.cpp's container, version 3), read the way Model/GgufFile.swift reads them, and
their Q4_K / Q5_K weights loaded into the plane form the kernels read.

A GGUF file is the magic "GGUF" (little-endian word 0x46554747), the version (3), the tensor and
metadata counts (u64), the metadata pairs (a string key, a u32 value type, the value), one record
per tensor (name, rank, u64 extents with the row -- ggml's first dimension -- first, u32 ggml type,
u64 offset relative to the data), and the tensor data from the end of the header rounded up to
`general.alignment` (32 when absent). Parsing restates GgufFile.init (GgufFile.swift:99-175) with
its checks: version 3 only, rank 1..4, rows a whole number of blocks, no duplicate keys or
tensors, every tensor inside the file. String arrays and arrays longer than 4096 elements are
skipped, as there (:292-325).

`load_weight` turns a Q4_K / Q5_K tensor into a runtime.Q5KWeight / Q4KWeight through the device
repack (GgufPlanes.repack), with the rows rounded up to whole 128-row tiles by zero blocks
(GgufConvert.storedRows, GgufConvert.swift:259-262), and a Q8_0 / Q6_K / IQ4_NL / IQ4_XS tensor into
a runtime.GgufWeight of its native blocks. A weight the file holds in a float type (f32, f16, bf16)
is quantised to Q8_0 first (GgufConvert.storedType / q8_0Blocks, GgufConvert.swift:229-257). The rows
of a gated-delta layer's head-ordered weights are moved into the engine's order of the value heads
(GgufConvert.swift:56-70, 326-345, 381-395: `block_head_order`); the out projection keeps its
columns in the file's order and is multiplied with runtime.gemm(..., key_heads=16). `dense_bf16`
converts the dense tensors the same way (GgufConvert.ggufDense, :432-457). `write_gguf` writes the
file form (the tests' fixtures).
"""
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

MAGIC = 0x46554747
# ggml type id -> (block elements, block bytes) for the types GgufTensorType knows
# (GgufQuant.swift:13-45).
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 20: (32, 18), 21: (256, 110), 23: (256, 136), 30: (1, 2)}
Q4_K, Q5_K = 12, 13
Q8_0 = 8
FLOAT_TYPES = (0, 1, 30)  # f32, f16, bf16: kept as Q8_0 (GgufConvert.storedType, GgufConvert.swift:229-234)
_MAX_KEPT_ARRAY = 4096
_WIDTH = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class GgufError(Exception):
    """GgufError (GgufFile.swift:12-35)."""


@dataclass
class Tensor:
    name: str
    type: int
    dims: list
    offset: int       # absolute byte offset in the file
    byte_length: int

    @property
    def rows(self):
        """The matrix's rows (ggml's second extent) of a [inner, rows] tensor."""
        return int(np.prod(self.dims[1:])) if len(self.dims) > 1 else 1

    @property
    def inner(self):
        return self.dims[0]


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def read(self, fmt):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise GgufError("GGUF header is truncated")
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += n
        return v

    def string(self):
        n = self.read("<Q")
        if n > len(self.buf) - self.pos:
            raise GgufError("GGUF header is truncated")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", "replace")
        self.pos += n
        return s

    def value(self, t):
        if t in _FMT:
            v = self.read(_FMT[t])
            return bool(v) if t == 7 else v
        if t == 8:
            return self.string()
        if t == 9:
            et, count = self.read("<I"), self.read("<Q")
            if et == 8:
                for _ in range(count):
                    self.string()
                return ("skipped", count)
            if et not in _WIDTH:
                raise GgufError(f"GGUF header is malformed: array of metadata value type {et}")
            if count * _WIDTH[et] > len(self.buf) - self.pos:
                raise GgufError("GGUF header is truncated")
            if et == 7 or count > _MAX_KEPT_ARRAY:
                self.pos += count * _WIDTH[et]
                return ("skipped", count)
            return [self.value(et) for _ in range(count)]
        raise GgufError(f"GGUF header is malformed: unknown metadata value type {t}")


class GgufFile:
    """GgufFile(url:) (GgufFile.swift:99-175): the header parsed and every tensor bounds-checked
    on open; tensor bytes are views of a read-only memory map."""

    def __init__(self, path):
        self.path = Path(path)
        try:
            self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        except (OSError, ValueError) as e:
            raise GgufError(f"GGUF file unreadable: {self.path}: {e}") from None
        r = _Reader(self._map)
        if r.read("<I") != MAGIC:
            raise GgufError("not a GGUF file: bad magic")
        self.version = r.read("<I")
        if self.version != 3:
            raise GgufError(f"unsupported GGUF version {self.version}; only version 3 is read")
        n_tensors, n_pairs = r.read("<Q"), r.read("<Q")
        self.metadata = {}
        for _ in range(n_pairs):
            key = r.string()
            value = r.value(r.read("<I"))
            if key in self.metadata:
                raise GgufError(f"GGUF header is malformed: duplicate metadata key {key}")
            self.metadata[key] = value
        self.alignment = 32
        if "general.alignment" in self.metadata:
            a = self.metadata["general.alignment"]
            if not isinstance(a, int) or isinstance(a, bool) or a <= 0:
                raise GgufError("GGUF header is malformed: general.alignment is not a positive integer")
            self.alignment = a
        pending = []
        for _ in range(n_tensors):
            name = r.string()
            rank = r.read("<I")
            if not 1 <= rank <= 4:
                raise GgufError(f"GGUF header is malformed: tensor {name} has {rank} dimensions")
            dims = [r.read("<Q") for _ in range(rank)]
            tid, rel = r.read("<I"), r.read("<Q")
            if tid not in BLOCK:
                raise GgufError(f"tensor {name} has ggml type {tid}, which is not supported")
            be, bb = BLOCK[tid]
            if dims[0] % be:
                raise GgufError(f"GGUF header is malformed: tensor {name}: a row of {dims[0]} elements is not a "
                                f"whole number of {be}-element blocks")
            pending.append((name, tid, dims, rel, int(np.prod(dims, dtype=np.int64)) // be * bb))
        self.data_start = -(-r.pos // self.alignment) * self.alignment
        self.tensors = {}
        for name, tid, dims, rel, length in pending:
            start = self.data_start + rel
            if start + length > len(self._map):
                raise GgufError(f"tensor {name} ends at byte {start + length}, past the end of the file "
                                f"({len(self._map)} bytes)")
            if name in self.tensors:
                raise GgufError(f"GGUF header is malformed: duplicate tensor {name}")
            self.tensors[name] = Tensor(name, tid, dims, start, length)

    def tensor(self, name):
        t = self.tensors.get(name)
        if t is None:
            raise GgufError(f"no tensor named {name} in the GGUF file")
        return t

    def bytes(self, name):
        t = self.tensor(name)
        return self._map[t.offset:t.offset + t.byte_length]


# ---- the gated-delta value heads (GgufNames.swift, GgufConvert.swift) -------------------------

GDN_KEY_HEADS, GDN_VALUE_HEADS, GDN_HEAD_DIM = 16, 48, 128   # ModelGeometry (ModelWeights.swift:78-82)
GDN_CHANNELS, GDN_VALUE_DIM = 10240, 6144
CONV_TAPS = 4


def mlx_value_head(i, key_heads=GDN_KEY_HEADS, value_heads=GDN_VALUE_HEADS):
    """GgufNames.mlxValueHead: the engine's index of the value head a GGUF file stores as head i,
    3 (i % 16) + i / 16 for 48 heads over 16 key heads."""
    return (value_heads // key_heads) * (i % key_heads) + i // key_heads


@dataclass(frozen=True)
class HeadOrder:
    """GgufConvert.HeadOrder: a tensor's value heads are `span` units each from unit `first` (a unit
    being a row of a weight, a channel of the convolution or an element of a per-head vector)."""

    first: int
    span: int

    def destination(self, unit, heads=GDN_VALUE_HEADS):
        """The engine-order place of the file's unit `unit` (units outside the heads stay)."""
        h = (unit - self.first) // self.span
        if unit < self.first or h >= heads:
            return unit
        return self.first + mlx_value_head(h, value_heads=heads) * self.span + (unit - self.first) % self.span


_VALUE_CHANNELS = HeadOrder(GDN_CHANNELS - GDN_VALUE_DIM, GDN_HEAD_DIM)
# GgufConvert.ggufRole(ofBlockTensor:) for a gated-delta layer (GgufConvert.swift:340-352): the
# weights whose rows, and the dense tensors whose units, are by value head.
WEIGHT_HEAD_ORDER = {
    "attn_qkv.weight": _VALUE_CHANNELS,
    "attn_gate.weight": HeadOrder(0, GDN_HEAD_DIM),
    "ssm_alpha.weight": HeadOrder(0, 1),
    "ssm_beta.weight": HeadOrder(0, 1),
}
DENSE_HEAD_ORDER = {  # tail: (unit, head order, negated log)
    "ssm_conv1d.weight": (CONV_TAPS, _VALUE_CHANNELS, False),
    "ssm_a": (1, HeadOrder(0, 1), True),
    "ssm_dt.bias": (1, HeadOrder(0, 1), False),
}
# The out projection has the heads as its inner columns, left in the file's order: its GEMM reads
# the activations in that order instead (runtime.gemm(..., key_heads=GDN_KEY_HEADS)).
COLUMN_HEAD_ORDER = ("ssm_out.weight",)


def block_tail(name):
    """The tensor's name below `blk.<n>.`, or None outside the blocks."""
    if not name.startswith("blk."):
        return None
    rest = name[4:]
    digits = len(rest) - len(rest.lstrip("0123456789"))
    if digits == 0 or rest[digits:digits + 1] != ".":
        return None
    return rest[digits + 1:]


def block_head_order(name, full_attention=False):
    """The HeadOrder of a gated-delta layer's weight rows, or None (a full-attention layer has none)."""
    tail = block_tail(name)
    return None if full_attention or tail is None else WEIGHT_HEAD_ORDER.get(tail)


def order_rows(native, rows, row_bytes, head_order, stored_rows=None, heads=GDN_VALUE_HEADS):
    """GgufConvert.ggufPlanes' `order` (GgufConvert.swift:381-395): row r of the file goes to row
    head_order.destination(r), whole rows of native blocks (lossless); rows past `rows` up to
    `stored_rows` are zero blocks."""
    native = np.asarray(native, np.uint8).reshape(rows, row_bytes)
    stored = rows if stored_rows is None else stored_rows
    out = np.zeros((stored, row_bytes), np.uint8)
    if head_order is None:
        out[:rows] = native
    else:
        dest = np.array([head_order.destination(r, heads) for r in range(rows)], np.int64)
        out[dest] = native
    return out.reshape(-1)


def q8_0_blocks(values):
    """GgufConvert.q8_0Blocks (GgufConvert.swift:236-257): fp32 values, 32 a block, as Q8_0 blocks
    the way llama.cpp quantises: scale = largest magnitude / 127 (fp32), kept as fp16 (RNE); each
    code = value x (1 / scale), rounded half away from zero, clamped to int8 (0 for a zero block)."""
    v = np.asarray(values, np.float32).reshape(-1, 32)
    largest = np.abs(v).max(axis=1)
    scale = (largest / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inverse = np.where(scale > 0, np.float32(1) / scale, np.float32(0)).astype(np.float32)
    x = (v * inverse[:, None]).astype(np.float32).astype(np.float64)
    code = np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5))
    code = np.clip(code, -128, 127).astype(np.int8)
    out = np.empty((v.shape[0], 34), np.uint8)
    out[:, 0:2] = scale.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = code.view(np.uint8)
    return out.reshape(-1)


def float_values(f, name):
    """A float-typed tensor's values as fp32 (f32, f16, bf16)."""
    t = f.tensor(name)
    raw = np.array(f.bytes(name))
    if t.type == 0:
        return raw.view(np.float32).copy()
    if t.type == 1:
        return raw.view(np.float16).astype(np.float32)
    if t.type == 30:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise GgufError(f"tensor {name} has ggml type {t.type}, not a float type")


def bf16_rne(values):
    """GgufConvert.bf16Bits(roundingToEven:) (GgufConvert.swift:264-268) for each value."""
    bits = np.asarray(values, np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def dense_bf16(values, unit=1, head_order=None, negated_log=False, heads=GDN_VALUE_HEADS):
    """GgufConvert.ggufDense (GgufConvert.swift:432-457): fp32 values -> bf16 (RNE), the decay
    turned back into A_log (the file holds -exp(A_log)), each unit of `unit` values moved to its
    engine-order place."""
    v = np.asarray(values, np.float32).reshape(-1)
    if negated_log:
        if not (v < 0).all():
            raise GgufError("the decay holds a value that is not negative, so is not -exp of anything")
        v = np.log(-v).astype(np.float32)
    if not np.isfinite(v).all():
        raise GgufError("a dense tensor holds a value that is not finite")
    bits = bf16_rne(v)
    out = np.empty_like(bits)
    idx = np.arange(v.size)
    dest_unit = idx // unit if head_order is None else np.array(
        [head_order.destination(u, heads) for u in range(v.size // unit)], np.int64)[idx // unit]
    out[dest_unit * unit + idx % unit] = bits
    return out


def load_weight(f, name, device="cuda", full_attention=False, rows32=False):
    """A packed matrix [rows, inner] on the device in the form its kernels read: Q4_K / Q5_K as planes
    (GgufPlanes.repack on the GPU), the other formats in their native blocks, a float type as Q8_0
    blocks; a gated-delta layer's head-ordered rows in the engine's order (GgufConvert.ggufPlanes,
    GgufConvert.swift:370-430). Planes round the rows up to whole tiles by zero blocks
    (GgufConvert.swift:259-262). rows32=True puts native blocks in the ROWS32 order
    (runtime.gguf_repack_rows32; faster from about 16 activation rows) where inner % 256 == 0."""
    import torch
    from . import runtime as rt
    t = f.tensor(name)
    order = block_head_order(name, full_attention)
    if t.type in FLOAT_TYPES:
        if len(t.dims) != 2 or t.inner % 32:
            raise GgufError(f"tensor {name} is a dense float tensor (dims {t.dims}); the device kernels take packed "
                            "matrices (a float matrix is requantised to Q8_0, whole 32-element blocks a row); "
                            "dense tensors convert with dense_bf16")
        native = q8_0_blocks(float_values(f, name))
        gtype = Q8_0
    else:
        native = np.array(f.bytes(name))
        gtype = t.type
    if gtype in rt.GGUF_NATIVE:
        # Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS stay in their native blocks.
        elems, size = rt.GGUF_NATIVE[gtype]
        if order is not None:
            native = order_rows(native, t.rows, t.inner // elems * size, order)
        w = rt.GgufWeight(torch.from_numpy(np.ascontiguousarray(native)).to(device), gtype, t.rows, t.inner)
        return rt.gguf_repack_rows32(w) if rows32 and t.inner % 256 == 0 else w
    if t.type not in (Q4_K, Q5_K):
        raise GgufError(f"tensor {name} has ggml type {t.type}; the device kernels take Q4_K, Q5_K, Q3_K, "
                        "Q6_K, Q8_0, IQ4_NL, IQ3_S and IQ4_XS")
    rows, inner = t.rows, t.inner
    stored = -(-rows // 128) * 128
    block = BLOCK[t.type][1]
    native = order_rows(native, rows, inner // 256 * block, order, stored_rows=stored)
    dev = torch.from_numpy(native).to(device)
    if t.type == Q5_K:
        return rt.q5k_repack(dev, stored, inner)
    return rt.q4k_repack(dev, stored, inner)


def write_gguf(path, metadata, tensors, alignment=32):
    """Write a version-3 GGUF file. metadata: [(key, type, value)] with the GGUF value type ids
    (arrays as (9, (element type, [values]))); tensors: [(name, ggml type, dims, bytes)]."""
    out = bytearray(struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(metadata)))

    def put_string(s):
        b = s.encode()
        out.extend(struct.pack("<Q", len(b)) + b)

    def put_value(t, v):
        if t in _FMT:
            out.extend(struct.pack(_FMT[t], int(v) if t == 7 else v))
        elif t == 8:
            put_string(v)
        elif t == 9:
            et, values = v
            out.extend(struct.pack("<IQ", et, len(values)))
            for x in values:
                put_value(et, x)
        else:
            raise GgufError(f"unknown value type {t}")

    for key, t, v in metadata:
        put_string(key)
        out.extend(struct.pack("<I", t))
        put_value(t, v)
    offsets, rel = [], 0
    for name, tid, dims, data in tensors:
        put_string(name)
        out.extend(struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims))
        rel = -(-rel // alignment) * alignment
        out.extend(struct.pack("<IQ", tid, rel))
        offsets.append(rel)
        rel += len(data)
    start = -(-len(out) // alignment) * alignment
    out.extend(b"\0" * (start - len(out)))
    for (name, tid, dims, data), off in zip(tensors, offsets):
        out.extend(b"\0" * (start + off - len(out)))
        out.extend(bytes(data))
    Path(path).write_bytes(bytes(out))
    return path
