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
a runtime.GgufWeight of its native blocks. `write_gguf` writes the same form (the tests'
fixtures).
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


def load_weight(f, name, device="cuda"):
    """A Q4_K or Q5_K matrix [rows, inner] as planes on the device (GgufPlanes.repack on the GPU),
    rows rounded up to whole tiles by zero blocks (GgufConvert.swift:259-262)."""
    import torch
    from . import runtime as rt
    t = f.tensor(name)
    if t.type in rt.GGUF_NATIVE:
        # Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS stay in their native blocks.
        native = torch.from_numpy(np.array(f.bytes(name))).to(device)
        return rt.GgufWeight(native, t.type, t.rows, t.inner)
    if t.type not in (Q4_K, Q5_K):
        raise GgufError(f"tensor {name} has ggml type {t.type}; the device kernels take Q4_K, Q5_K, Q3_K, "
                        "Q6_K, Q8_0, IQ4_NL, IQ3_S and IQ4_XS")
    rows, inner = t.rows, t.inner
    stored = -(-rows // 128) * 128
    block = BLOCK[t.type][1]
    native = np.zeros(stored * (inner // 256) * block, np.uint8)
    native[: t.byte_length] = f.bytes(name)
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
