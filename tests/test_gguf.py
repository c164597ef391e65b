"""GGUF files on the CPU (Model/GgufFile.swift): a written file parsed back with its metadata,
tensor records and bytes, and each header check the reference makes rejects a file that breaks it."""
import struct

import numpy as np
import pytest

import oracle
from splosh_amd import gguf

META = [("general.architecture", 8, "qwen3"), ("general.alignment", 4, 64), ("a.count", 10, 7),
        ("a.neg", 5, -3), ("a.flag", 7, True), ("a.ratio", 6, 0.5), ("a.ints", 9, (5, [1, 2, 3])),
        ("a.words", 9, (8, ["x", "yz"])), ("a.big", 9, (0, list(range(256)) * 17))]


def _tensors():
    q5 = oracle.q45k_random_native(200, 512, seed=1, fifth_bit=True)
    q4 = oracle.q45k_random_native(3, 256, seed=2, fifth_bit=False)
    f32 = np.arange(10, dtype=np.float32)
    return [("blk.0.ffn_down.weight", gguf.Q5_K, [512, 200], q5.tobytes()),
            ("blk.0.attn_q.weight", gguf.Q4_K, [256, 3], q4.tobytes()),
            ("output_norm.weight", 0, [10], f32.tobytes())]


def test_roundtrip(tmp_path):
    t = _tensors()
    f = gguf.GgufFile(gguf.write_gguf(tmp_path / "m.gguf", META, t, alignment=64))
    assert f.version == 3 and f.alignment == 64 and f.data_start % 64 == 0
    m = f.metadata
    assert m["general.architecture"] == "qwen3" and m["a.count"] == 7 and m["a.neg"] == -3
    assert m["a.flag"] is True and m["a.ratio"] == 0.5 and m["a.ints"] == [1, 2, 3]
    assert m["a.words"] == ("skipped", 2) and m["a.big"] == ("skipped", 256 * 17)
    for name, tid, dims, data in t:
        r = f.tensor(name)
        assert (r.type, r.dims, r.byte_length) == (tid, dims, len(data))
        assert r.offset % 64 == 0
        assert f.bytes(name).tobytes() == data
    assert (f.tensor("blk.0.ffn_down.weight").rows, f.tensor("blk.0.ffn_down.weight").inner) == (200, 512)
    with pytest.raises(gguf.GgufError, match="no tensor named"):
        f.tensor("missing")


def test_default_alignment(tmp_path):
    f = gguf.GgufFile(gguf.write_gguf(tmp_path / "d.gguf", [], _tensors()[2:]))
    assert f.alignment == 32 and f.data_start % 32 == 0
    assert np.array_equal(f.bytes("output_norm.weight").view(np.float32), np.arange(10, dtype=np.float32))


def _good(tmp_path):
    return bytearray(gguf.write_gguf(tmp_path / "g.gguf", META[:2], _tensors()[1:]).read_bytes())


def _load(tmp_path, data):
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(data))
    return gguf.GgufFile(p)


def test_bad_magic_and_version(tmp_path):
    d = _good(tmp_path)
    d[0] ^= 1
    with pytest.raises(gguf.GgufError, match="bad magic"):
        _load(tmp_path, d)
    d = _good(tmp_path)
    d[4:8] = struct.pack("<I", 2)
    with pytest.raises(gguf.GgufError, match="version 2"):
        _load(tmp_path, d)


def test_truncated(tmp_path):
    d = _good(tmp_path)
    for cut in (3, 20, 60):
        with pytest.raises(gguf.GgufError, match="truncated"):
            _load(tmp_path, d[:cut])


def test_tensor_past_end(tmp_path):
    d = _good(tmp_path)
    with pytest.raises(gguf.GgufError, match="past the end"):
        _load(tmp_path, d[:-1])


def test_duplicates(tmp_path):
    p = gguf.write_gguf(tmp_path / "k.gguf", META[:1] + META[:1], [])
    with pytest.raises(gguf.GgufError, match="duplicate metadata key"):
        gguf.GgufFile(p)
    t = _tensors()[2:]
    p = gguf.write_gguf(tmp_path / "t.gguf", [], t + t)
    with pytest.raises(gguf.GgufError, match="duplicate tensor"):
        gguf.GgufFile(p)


def test_header_checks(tmp_path):
    cases = [([("general.alignment", 4, 0)], [], "alignment"),
             ([("general.alignment", 8, "x")], [], "alignment"),
             ([("x", 13, 0)], [], "unknown metadata value type"),
             ([], [("w", 99, [32], b"")], "ggml type 99"),
             ([], [("w", gguf.Q4_K, [100, 2], b"")], "whole number"),
             ([], [("w", 0, [1, 1, 1, 1, 1], b"\0" * 4)], "5 dimensions")]
    for meta, tensors, match in cases:
        p = tmp_path / "h.gguf"
        try:
            gguf.write_gguf(p, meta, tensors)
        except gguf.GgufError:
            # The writer knows no value type 13: write the pair by hand.
            p.write_bytes(struct.pack("<IIQQ", gguf.MAGIC, 3, 0, 1) + struct.pack("<Q", 1) + b"x"
                          + struct.pack("<I", 13))
        with pytest.raises(gguf.GgufError, match=match):
            gguf.GgufFile(p)


def test_unreadable(tmp_path):
    with pytest.raises(gguf.GgufError, match="unreadable"):
        gguf.GgufFile(tmp_path / "absent.gguf")


def test_load_weight_rejects_other_types(tmp_path):
    f = gguf.GgufFile(gguf.write_gguf(tmp_path / "o.gguf", [], _tensors()[2:]))
    with pytest.raises(gguf.GgufError, match="device kernels take"):
        gguf.load_weight(f, "output_norm.weight", device="cpu")
