"""SPLW containers on the CPU (Model/WeightFile.swift): written, read back byte-exact, resolved into
q4 triplets and GGUF planes, and every framing and record check the reference makes rejects a
container that breaks it."""
import json
import struct

import numpy as np
import pytest

import oracle
from splosh_amd import weightfile as wf

NAME = "language_model.layers.0.mlp.up_proj"


def _q4_tensors(rows, inner, seed, tiled=False):
    words, stride, sc, bi = oracle.q4_random_weight(rows, inner, seed)
    words = np.ascontiguousarray(words.reshape(rows, -1)[:, : inner // 8])  # MLX's [rows, K/8], unpadded
    groups = inner // 64
    if tiled:
        words = oracle.tile128(words.reshape(-1).view(np.uint8), rows, groups, 32).view(np.uint32)
        sc = oracle.tile128(sc.reshape(-1).view(np.uint8), rows, groups, 2).view(np.uint16)
        bi = oracle.tile128(bi.reshape(-1).view(np.uint8), rows, groups, 2).view(np.uint16)
    return [(NAME + ".weight", "U32", np.asarray(words, np.uint32).reshape(rows, -1),
             {"logicalShape": [rows, inner]}),
            (NAME + ".scales", "BF16", np.asarray(sc, np.uint16).reshape(rows, groups), {}),
            (NAME + ".biases", "BF16", np.asarray(bi, np.uint16).reshape(rows, groups), {})]


def test_roundtrip_q4_and_dense(tmp_path):
    t = _q4_tensors(128, 320, seed=1) + [("language_model.norm.weight", "BF16", np.arange(320, dtype=np.uint16), {})]
    path = wf.write_splw(tmp_path / "a.splw", t)
    f = wf.SplwFile(path)
    assert f.format == wf.FORMAT_ROW_MAJOR and not f.is_gguf
    for name, _, a, _ in t:
        assert np.array_equal(np.asarray(f.read(name)), a.view(np.uint8).reshape(-1)), name
        assert f.records[name].offset % 128 == 0
    q = f.resolve_q4(NAME + ".weight")
    assert (q.rows, q.inner, q.tiled, q.stride_words) == (128, 320, False, 40)
    assert np.array_equal(f.dense_bf16("language_model.norm.weight", [320]), np.arange(320))


def test_tiled_format_marks_eligible_weights(tmp_path):
    path = wf.write_splw(tmp_path / "t.splw", _q4_tensors(256, 256, seed=2, tiled=True), fmt=wf.FORMAT_TILED)
    assert wf.SplwFile(path).resolve_q4(NAME + ".weight").tiled
    assert wf.is_tiled_weight("language_model.x.weight", 256) and not wf.is_tiled_weight(
        "language_model.embed_tokens.weight", 256) and not wf.is_tiled_weight("language_model.x.weight", 48)


def test_gguf_planes(tmp_path):
    n, k = 128, 512
    t = []
    for base, fifth in (("language_model.a", True), ("language_model.b", False)):
        native = oracle.q45k_random_native(n, k, seed=3, fifth_bit=fifth)
        p0, p1, meta = oracle.q45k_repack(native, n, k, fifth_bit=fifth)
        gt = wf.GGUF_Q5_K if fifth else wf.GGUF_Q4_K
        t.append((base + ".weight", "U8", p0.reshape(n, -1), {"logicalShape": [n, k], "ggufType": gt}))
        if fifth:
            t.append((base + ".plane1", "U8", p1.reshape(n, -1), {}))
        t.append((base + ".meta", "U8", meta.reshape(n, -1), {}))
    f = wf.SplwFile(wf.write_splw(tmp_path / "g.splw", t, fmt=wf.FORMAT_GGUF))
    a, b = f.resolve_gguf("language_model.a.weight"), f.resolve_gguf("language_model.b.weight")
    assert (a.gguf_type, a.stored_rows, b.gguf_type, b.plane1) == (wf.GGUF_Q5_K, n, wf.GGUF_Q4_K, None)
    assert np.array_equal(np.asarray(f.read(a.plane1.name)), t[1][2].reshape(-1))
    with pytest.raises(wf.WeightFileError):
        f.resolve_q4("language_model.a.weight")  # no affine triplets in a GGUF artifact


def _corrupt(path, fn):
    raw = bytearray(path.read_bytes())
    hl = struct.unpack_from("<Q", raw, 8)[0]
    header = json.loads(raw[16:16 + hl])
    raw = fn(raw, header, hl)
    path.write_bytes(bytes(raw))


def _rewrite_header(raw, header, hl):
    new = json.dumps(header, separators=(",", ":")).encode()
    assert len(new) <= hl
    new = new + b" " * (hl - len(new))  # same length: offsets stay valid
    raw[16:16 + hl] = new
    return raw


@pytest.mark.parametrize("case,message", [
    ("magic", "bad magic"), ("version", "unsupported version"), ("truncate", "payload size mismatch"),
    ("padding", "padding mismatch"), ("duplicate", "duplicate tensor"), ("quant", "unsupported quantization"),
    ("extra", "payload size mismatch")])
def test_framing_checks(tmp_path, case, message):
    path = wf.write_splw(tmp_path / "c.splw", _q4_tensors(128, 128, seed=4))

    def edit(raw, header, hl):
        if case == "magic":
            raw[0:4] = b"SPLX"
        elif case == "version":
            raw[4:8] = struct.pack("<I", 2)
        elif case == "truncate":
            raw = raw[:-1]
        elif case == "extra":
            raw = raw + b"\0"
        elif case == "padding":
            header["tensorRecords"][1]["alignmentPadding"] += 1
            raw = _rewrite_header(raw, header, hl)
        elif case == "duplicate":
            header["tensorRecords"][2]["name"] = header["tensorRecords"][1]["name"]
            raw = _rewrite_header(raw, header, hl)
        elif case == "quant":
            header["quantization"]["groupSize"] = 32
            raw = _rewrite_header(raw, header, hl)
        return raw

    _corrupt(path, edit)
    with pytest.raises(wf.WeightFileError, match=message):
        wf.SplwFile(path)


def test_record_checks(tmp_path):
    t = _q4_tensors(128, 128, seed=5)
    bad_sidecar = [t[0], (t[1][0], "F32", t[1][2].astype(np.float32), {}), t[2]]
    f = wf.SplwFile(wf.write_splw(tmp_path / "s.splw", bad_sidecar))
    with pytest.raises(wf.WeightFileError, match="must be BF16"):
        f.resolve_q4(NAME + ".weight")
    bad_shape = [(t[0][0], "U32", t[0][2], {"logicalShape": [128, 100]}), t[1], t[2]]
    f = wf.SplwFile(wf.write_splw(tmp_path / "l.splw", bad_shape))
    with pytest.raises(wf.WeightFileError, match="physical/logical"):
        f.resolve_q4(NAME + ".weight")
    n, k = 128, 256
    p0, _, meta = oracle.q45k_repack(oracle.q45k_random_native(n, k, seed=6, fifth_bit=False), n, k, fifth_bit=False)
    q4k_with_plane1 = [("language_model.c.weight", "U8", p0.reshape(n, -1), {"logicalShape": [n, k], "ggufType": 12}),
                       ("language_model.c.plane1", "U8", np.zeros((n, 32), np.uint8), {}),
                       ("language_model.c.meta", "U8", meta.reshape(n, -1), {})]
    f = wf.SplwFile(wf.write_splw(tmp_path / "p.splw", q4k_with_plane1, fmt=wf.FORMAT_GGUF))
    with pytest.raises(wf.WeightFileError, match="no second plane"):
        f.resolve_gguf("language_model.c.weight")
    with pytest.raises(wf.WeightFileError, match="missing tensor"):
        f.resolve_gguf("language_model.d.weight")
