"""Weights loaded from SPLW containers (Model/WeightFile.swift) run through the GEMM entry points
and match the oracle on the bytes that were written: a tiled q4 triplet, a row-major one (MLX's
unpadded rows), and GGUF Q5_K and Q4_K planes."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import abs_gemm, bf16_tensor, check_close, to_f32
from splosh_amd import weightfile as wf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


def test_q4_triplets_from_containers(rt, tmp_path):
    n, k, rows = 256, 512, 3
    words, stride, sc, bi = oracle.q4_random_weight(n, k, seed=60)
    dense = oracle.q4_dequant_rowmajor(words, stride, sc, bi, n, k)
    raw = np.ascontiguousarray(words.reshape(n, -1)[:, : k // 8])
    g = k // 64
    tiled = (oracle.tile128(raw.reshape(-1).view(np.uint8), n, g, 32).view(np.uint32).reshape(n, -1),
             oracle.tile128(sc.reshape(-1).view(np.uint8), n, g, 2).view(np.uint16).reshape(n, g),
             oracle.tile128(bi.reshape(-1).view(np.uint8), n, g, 2).view(np.uint16).reshape(n, g))
    a_bits = oracle.bf16_normal((rows, k), seed=61)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    for fmt, (pw, ps, pb) in ((wf.FORMAT_ROW_MAJOR, (raw, sc.reshape(n, g), bi.reshape(n, g))), (wf.FORMAT_TILED, tiled)):
        name = "language_model.layers.3.self_attn.q_proj"
        path = wf.write_splw(tmp_path / f"{fmt}.splw", [
            (name + ".weight", "U32", pw, {"logicalShape": [n, k]}), (name + ".scales", "BF16", ps, {}),
            (name + ".biases", "BF16", pb, {})], fmt=fmt)
        w = wf.SplwFile(path).q4(name + ".weight")
        assert w.order == (rt.TILED128 if fmt == wf.FORMAT_TILED else rt.ROW_MAJOR)
        assert np.array_equal(rt.dequant(w).cpu().numpy().view(np.uint32), dense.view(np.uint32))
        got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32))
        check_close(got, ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, dense), label=fmt)


@pytest.mark.parametrize("fifth", [True, False])
def test_gguf_planes_from_container(rt, tmp_path, fifth):
    n, k, rows = 128, 1024, 1
    native = oracle.q45k_random_native(n, k, seed=62, fifth_bit=fifth)
    p0, p1, meta = oracle.q45k_repack(native, n, k, fifth_bit=fifth)
    dense = oracle.q45k_decode(native, fifth_bit=fifth).reshape(n, k)
    base = "language_model.layers.0.mlp.down_proj"
    t = [(base + ".weight", "U8", p0.reshape(n, -1), {"logicalShape": [n, k], "ggufType": 13 if fifth else 12})]
    if fifth:
        t.append((base + ".plane1", "U8", p1.reshape(n, -1), {}))
    t.append((base + ".meta", "U8", meta.reshape(n, -1), {}))
    w = wf.SplwFile(wf.write_splw(tmp_path / "g.splw", t, fmt=wf.FORMAT_GGUF)).gguf(base + ".weight")
    assert np.array_equal(rt.dequant(w).cpu().numpy().view(np.uint32), dense.view(np.uint32))
    a_bits = oracle.bf16_normal((rows, k), seed=63)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32))
    check_close(got, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label=f"gguf fifth={fifth}")
