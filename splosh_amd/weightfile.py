"""SPLW weight containers: the reference's on-disk form of the weights this path consumes.

Restates the container contract of Model/WeightFile.swift (reader, :78-125 framing and record
checks, :134-185 GGUF plane resolution, :188-226 q4 triplet resolution), Model/Converter.swift
(:23-81, the header's fields) and Model/Retile.swift (:12-36, the row-major and tiled q4 formats),
and loads the resolved weights into device memory in the layouts the kernels read
(`runtime.Q4Weight`, `runtime.Q5KWeight`, `runtime.Q4KWeight`).

A container is "SPLW", a little-endian u32 version (1) and u64 header length, the JSON header,
then the payload from the next `pointerAlignmentBytes` boundary: tensor records in increasing
offset order, each at an aligned offset, the gap before it recorded as its `alignmentPadding`,
and nothing after the last one.

`write_splw` writes the same form (the tests' fixtures; the reference's Converter writes it from
safetensors shards, which this build does not read).
"""
import json
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

FORMAT_ROW_MAJOR = "mlxAffine4"
FORMAT_TILED = "mlxAffine4.tiled128"
FORMAT_GGUF = "gguf.tiled128"
TILE_ROWS = 128
GGUF_Q4_K, GGUF_Q5_K = 12, 13  # ggml type ids (Model/GgufQuant.swift:19-20)
_DTYPE_BYTES = {"BF16": 2, "F32": 4, "F16": 2, "U32": 4, "I32": 4, "I64": 8, "U8": 1}


class WeightFileError(Exception):
    """WeightFileError / TensorInventoryError (Model/WeightFile.swift:4-11)."""


def _align(n, a):
    return n + (a - n % a) % a


def _layout(fmt):
    """Converter.layout(ofFormat:) (Retile.swift:19-25): (bits, tiled) or None."""
    for bits in (4, 8):
        if fmt == f"mlxAffine{bits}":
            return bits, False
        if fmt == f"mlxAffine{bits}.tiled128":
            return bits, True
    return None


def is_tiled_weight(name, rows):
    """Converter.isTiledWeight (Retile.swift:28-32): stored tiled in a tiled artifact."""
    return name.startswith("language_model.") and name.endswith(".weight") and "embed_tokens" not in name \
        and rows % TILE_ROWS == 0


def gguf_plane_sizes(gguf_type, rows, inner):
    """GgufPlanes.geometry / sizes (GgufPlanes.swift:61-86) for Q4_K and Q5_K: (plane0, plane1, meta)."""
    if gguf_type not in (GGUF_Q4_K, GGUF_Q5_K) or inner % 256:
        return None
    groups = inner // 32
    return rows * groups * 16, rows * groups * (4 if gguf_type == GGUF_Q5_K else 0), rows * (inner // 256) * 16


@dataclass
class Record:
    name: str
    dtype: str
    shape: list
    physical_shape: list
    logical_shape: list
    offset: int
    length: int
    row_stride: int
    gguf_type: int


@dataclass
class Q4Record:
    """Q4WeightRecord (WeightFile.swift:13-27): the triplet's records and geometry."""
    weight: Record
    scales: Record
    biases: Record
    rows: int
    inner: int
    tiled: bool
    stride_words: int


@dataclass
class GgufRecord:
    """GgufWeightRecord (WeightFile.swift:29-47): the planes' records, logical shape, stored rows."""
    gguf_type: int
    plane0: Record
    plane1: Record
    meta: Record
    logical_shape: list
    stored_rows: int


class SplwFile:
    """WeightFile(splwURL:) (WeightFile.swift:78-125): the framing, header and every record are
    validated on open; tensors are read on demand (memory-mapped, never the whole file)."""

    def __init__(self, path):
        self.path = Path(path)
        if not self.path.exists():
            raise WeightFileError(f"weight file missing: {self.path}")
        size = self.path.stat().st_size
        if size < 16:
            raise WeightFileError("truncated framing")
        with open(self.path, "rb") as f:
            framing = f.read(16)
            if framing[:4] != b"SPLW":
                raise WeightFileError("bad magic")
            version, header_length = struct.unpack_from("<IQ", framing, 4)
            if version != 1:
                raise WeightFileError("unsupported version")
            if header_length > size - 16:
                raise WeightFileError("header length overflow")
            raw = f.read(header_length)
        if len(raw) != header_length:
            raise WeightFileError("truncated framing")
        try:
            h = json.loads(raw)
        except ValueError as e:
            raise WeightFileError(f"malformed header: {e}") from None
        if h.get("magic") != "SPLW" or h.get("version") != 1 or h.get("headerLength") != header_length:
            raise WeightFileError("contradictory header framing")
        q = h["quantization"]
        affine = q["bits"] in (4, 8) and q["groupSize"] == 64 and q["mode"] == "affine"
        gguf = q == {"bits": 0, "groupSize": 32, "mode": "gguf"}
        if not (gguf if h["format"] == FORMAT_GGUF else affine):
            raise WeightFileError("unsupported quantization")
        align = h["alignment"]["pointerAlignmentBytes"]
        if align <= 0:
            raise WeightFileError("invalid alignment")
        payload_start = _align(16 + header_length, align)
        if payload_start > size or h["payloadLength"] > size - payload_start or payload_start + h["payloadLength"] != size:
            raise WeightFileError("payload size mismatch")
        previous, names, records = payload_start, set(), {}
        for r in h["tensorRecords"]:
            name = r["name"]
            if name in names:
                raise WeightFileError(f"duplicate tensor: {name}")
            names.add(name)
            if r["dtype"] not in _DTYPE_BYTES:
                raise WeightFileError(f"unknown dtype: {name}")
            off, length = r["payloadOffset"], r["rawByteLength"]
            if not name or any(d < 0 for d in r["shape"]) or off < payload_start or off < previous or off > size \
                    or length > size - off:
                raise WeightFileError(f"tensor bounds: {name}")
            if off % align:
                raise WeightFileError(f"unaligned tensor: {name}")
            if r["alignmentPadding"] != off - previous:
                raise WeightFileError(f"padding mismatch: {name}")
            previous = off + length
            records[name] = Record(name, r["dtype"], list(r["shape"]), list(r.get("physicalShape") or r["shape"]),
                                   r.get("logicalShape"), off, length, r.get("rowStride", 0), r.get("ggufType"))
        if previous > size or (records and previous != size):
            raise WeightFileError("unaccounted payload bytes")
        self.header, self.size, self.records = h, size, records
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")

    @property
    def format(self):
        return self.header["format"]

    @property
    def is_gguf(self):
        return self.format == FORMAT_GGUF

    def _record(self, name, dtype=None):
        r = self.records.get(name)
        if r is None:
            raise WeightFileError(f"missing tensor: {name}")
        if dtype is not None and r.dtype != dtype:
            raise WeightFileError(f"dtype mismatch for {name}: expected {dtype}, observed {r.dtype}")
        return r

    def read(self, name):
        """The record's bytes (a view of the memory map)."""
        r = self._record(name)
        return self._map[r.offset:r.offset + r.length]

    def resolve_q4(self, name):
        """WeightFile.q4 (WeightFile.swift:188-226): a validated MLX affine q4 triplet (Q4Record)."""
        r = self._record(name, "U32")
        if self.is_gguf:
            raise WeightFileError(f"{name} is in a GGUF-derived artifact, which has no affine triplets")
        layout = _layout(self.format)
        bits = self.header["quantization"]["bits"]
        phys, logical = r.physical_shape, r.logical_shape
        if layout is None or bits != 4 or phys != r.shape or len(phys) != 2 or min(phys) <= 0 or not logical \
                or len(logical) != 2 or logical[0] != phys[0] or logical[1] != phys[1] * (32 // bits):
            raise WeightFileError(f"invalid physical/logical shape metadata for {name}")
        base = name[: -len(".weight")] if name.endswith(".weight") else name
        sc, bi = self.records.get(base + ".scales"), self.records.get(base + ".biases")
        if sc is None or bi is None:
            raise WeightFileError(f"missing sidecar for {name}; expected {base}.scales and {base}.biases")
        if sc.dtype != "BF16" or bi.dtype != "BF16":
            raise WeightFileError(f"sidecars for {name} must be BF16")
        rows, inner = logical
        expected = [rows, (inner + 63) // 64]
        if sc.shape != expected or bi.shape != expected:
            raise WeightFileError(f"sidecar shape for {name} must be {expected}")
        return Q4Record(r, sc, bi, rows, inner, layout[1] and is_tiled_weight(name, rows), phys[1])

    def q4(self, name, device="cuda"):
        """The resolved triplet loaded as a runtime.Q4Weight in the container's layout (TILED128 for
        the tiled format's eligible weights, row-major with MLX's unpadded row otherwise)."""
        import torch
        from . import runtime as rt
        q = self.resolve_q4(name)
        dev = lambda rec, dt: torch.from_numpy(np.array(self.read(rec.name)).view(dt)).to(device)  # noqa: E731
        packed, scales, biases = dev(q.weight, np.int32), dev(q.scales, np.int16), dev(q.biases, np.int16)
        if q.tiled:
            return rt.Q4Weight(packed, scales, biases, q.rows, q.inner, rt.TILED128)
        return rt.Q4Weight(packed, scales, biases, q.rows, q.inner, rt.ROW_MAJOR, q.stride_words)

    def resolve_gguf(self, name):
        """WeightFile.gguf (WeightFile.swift:134-185): a GGUF weight's planes, validated against its
        type and logical shape (GgufRecord; stored rows are whole tiles)."""
        r = self._record(name, "U8")
        if not self.is_gguf or r.gguf_type not in (GGUF_Q4_K, GGUF_Q5_K):
            raise WeightFileError(f"{name} is not a GGUF weight of a type this build reads (Q4_K, Q5_K)")
        logical = r.logical_shape
        if not logical or len(logical) != 2 or min(logical) <= 0:
            raise WeightFileError(f"{name} has no logical shape [rows, inner]")
        stored = -(-logical[0] // TILE_ROWS) * TILE_ROWS
        sizes = gguf_plane_sizes(r.gguf_type, stored, logical[1])
        if sizes is None:
            raise WeightFileError(f"{name}: a row of {logical[1]} is not a whole number of blocks")
        base = name[: -len(".weight")] if name.endswith(".weight") else name

        def plane(pname, nbytes):
            p = r if pname == name else self.records.get(pname)
            if p is None:
                raise WeightFileError(f"{name} has no {pname}")
            if p.dtype != "U8" or p.length != nbytes or p.shape != [stored, nbytes // stored]:
                raise WeightFileError(f"{pname} is {p.length} bytes of shape {p.shape}; needs {nbytes}")
            return p

        if r.gguf_type == GGUF_Q4_K and (base + ".plane1") in self.records:
            raise WeightFileError(f"{name} is Q4_K, which has no second plane, yet {base}.plane1 exists")
        plane1 = plane(base + ".plane1", sizes[1]) if r.gguf_type == GGUF_Q5_K else None
        return GgufRecord(r.gguf_type, plane(name, sizes[0]), plane1, plane(base + ".meta", sizes[2]),
                          list(logical), stored)

    def gguf(self, name, device="cuda"):
        """The resolved planes loaded as a runtime.Q5KWeight or Q4KWeight."""
        import torch
        from . import runtime as rt
        g = self.resolve_gguf(name)
        dev = lambda rec: torch.from_numpy(np.array(self.read(rec.name))).to(device)  # noqa: E731
        if g.gguf_type == GGUF_Q4_K:
            return rt.Q4KWeight(dev(g.plane0), dev(g.meta), g.stored_rows, g.logical_shape[1])
        return rt.Q5KWeight(dev(g.plane0), dev(g.plane1), dev(g.meta), g.stored_rows, g.logical_shape[1])

    def dense_bf16(self, name, shape=None):
        """WeightFile.denseBF16 (WeightFile.swift:228-242): the bytes of a BF16 component."""
        r = self._record(name, "BF16")
        if shape is not None and r.shape != list(shape):
            raise WeightFileError(f"shape mismatch for {name}: expected {list(shape)}, observed {r.shape}")
        return np.array(self.read(name)).view(np.uint16).reshape(r.shape)


def write_splw(path, tensors, fmt=FORMAT_ROW_MAJOR, alignment=128):
    """Write an SPLW container in the form SplwFile reads (Converter's framing and padding rules).

    tensors: [(name, dtype, array, extra)] with dtype one of the record dtypes, array a numpy array
    of the record's bytes and shape, extra a dict of optional record fields (physicalShape,
    logicalShape, rowStride, ggufType)."""
    quant = {"bits": 0, "groupSize": 32, "mode": "gguf"} if fmt == FORMAT_GGUF else \
        {"bits": 4, "groupSize": 64, "mode": "affine"}
    header = {"magic": "SPLW", "version": 1, "format": fmt, "dtype": "mixed", "quantization": quant,
              "alignment": {"rowStrideBytes": 128, "pointerAlignmentBytes": alignment, "padded": True},
              "configHash": "", "tokenizerHash": "", "tensorRecords": [], "headerLength": 0, "payloadLength": 0}
    blobs = [np.ascontiguousarray(a).view(np.uint8).reshape(-1) for _, _, a, _ in tensors]
    # The header holds its own length and the offsets, which depend on it: iterate to a fixed point.
    for _ in range(8):
        start = _align(16 + header["headerLength"], alignment)
        records, off = [], start
        for (name, dtype, a, extra), blob in zip(tensors, blobs):
            aligned = _align(off, alignment)
            rec = {"name": name, "dtype": dtype, "shape": list(a.shape), "physicalShape": list(a.shape),
                   "logicalShape": None, "payloadOffset": aligned, "rawByteLength": int(blob.size),
                   "rowStride": 0, "alignmentPadding": aligned - off, "sourceShard": "fixture"}
            rec.update(extra or {})
            records.append(rec)
            off = aligned + blob.size
        header["tensorRecords"], header["payloadLength"] = records, off - start
        raw = json.dumps(header, separators=(",", ":")).encode()
        if len(raw) == header["headerLength"]:
            break
        header["headerLength"] = len(raw)
    else:
        raise WeightFileError("header length did not settle")
    with open(path, "wb") as f:
        f.write(b"SPLW" + struct.pack("<IQ", 1, len(raw)) + raw)
        pos = 16 + len(raw)
        for rec, blob in zip(records, blobs):
            f.write(b"\0" * (rec["payloadOffset"] - pos))
            f.write(blob.tobytes())
            pos = rec["payloadOffset"] + blob.size
    return path
