"""The remaining weight consumers of a step: the q4 embedding lookup (sp_embed_q4,
engine.metal:39-57) against rows of the pinned dequant, bit-exact; and the 48-row a/b projections
of the gated-delta layer (sp_gemm_q4_b, engine.metal:240-270: row-major, N not a multiple of 32)
through Engine.gemm at every row count the step uses."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import Q4Case, abs_gemm, bf16_tensor, check_close, to_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


@pytest.mark.parametrize("tiled", [False, True])
def test_embed_rows_bit_exact(rt, tiled):
    n, k = 384, 320
    case = Q4Case(n, k, seed=31)
    w = case.w_tiled if tiled else case.w_rm
    ids = np.array([0, 5, 383, 127, 128, 5, 200], np.uint32)
    got = rt.embed(w, torch.from_numpy(ids.view(np.int32)).cuda()).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), case.dense[ids].view(np.uint32))
    got16 = rt.embed(w, torch.from_numpy(ids.view(np.int32)).cuda(), out_dtype=torch.bfloat16)
    assert np.array_equal(got16.view(torch.int16).cpu().numpy().view(np.uint16),
                          oracle.f32_to_bf16_rne(case.dense[ids]).reshape(len(ids), k))


def test_embed_odd_k_and_out_of_range(rt):
    """K = 65 (a partial word and group, the row-major padded layout) and ids past the table."""
    n, k = 7, 65
    words, stride, sc, bi = oracle.q4_random_weight(n, k, seed=32)
    from qcheck import dev_u16, dev_u32
    w = rt.Q4Weight(dev_u32(words), dev_u16(sc), dev_u16(bi), n, k, rt.ROW_MAJOR, stride)
    dense = oracle.q4_dequant_rowmajor(words, stride, sc, bi, n, k)
    ids = np.array([6, 0, 7, 0xFFFFFFFF, 3], np.uint32)
    out = torch.full((5, 80), 7.0, device="cuda")
    rt.embed(w, torch.from_numpy(ids.view(np.int32)).cuda(), out=out)  # row stride 80, K columns written
    got = out.cpu().numpy()
    assert np.array_equal(got[[0, 1, 4], :k].view(np.uint32), dense[[6, 0, 3]].view(np.uint32))
    assert np.all(got[[2, 3], :k] == 0) and np.all(got[:, k:] == 7.0)


@pytest.mark.parametrize("kind", ["q5k", "q4k", 8, 11, 14, 20, 21, 23])
def test_gguf_embed_rows_bit_exact(rt, kind):
    """sp_gguf_embed (engine_gguf.metal:302-318) on Q5_K / Q4_K planes and on every native-block
    format: the rows of the pinned decoder, bit-exact in fp32 and RNE in bf16; ids past the table
    give zeros; the output row stride is honoured."""
    from qcheck import dev_u8
    n, k = 256, 512
    if kind in ("q5k", "q4k"):
        fifth = kind == "q5k"
        native = oracle.q45k_random_native(n, k, seed=41, fifth_bit=fifth)
        w = (rt.q5k_repack if fifth else rt.q4k_repack)(dev_u8(native), n, k)
        dense = oracle.q45k_decode(native, fifth_bit=fifth).reshape(n, k)
    else:
        native = oracle.gguf_random_native(kind, n, k, seed=42)
        w = rt.GgufWeight(dev_u8(native), kind, n, k)
        dense = oracle.gguf_decode(kind, native).reshape(n, k)
    ids = np.array([0, 255, 17, 300, 128, 17, 0xFFFFFFFF], np.uint32)
    tokens = torch.from_numpy(ids.view(np.int32)).cuda()
    out = torch.full((len(ids), k + 8), 5.0, device="cuda")
    rt.embed(w, tokens, out=out)
    got = out.cpu().numpy()
    inside = ids < n
    assert np.array_equal(got[inside, :k].view(np.uint32), dense[ids[inside]].view(np.uint32))
    assert np.all(got[~inside, :k] == 0) and np.all(got[:, k:] == 5.0)
    got16 = rt.embed(w, tokens, out_dtype=torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got16[inside], oracle.f32_to_bf16_rne(dense[ids[inside]]).reshape(int(inside.sum()), k))


@pytest.mark.parametrize("rows", [1, 2, 16, 64])
def test_small_projection_48_rows(rt, rows):
    """The gated-delta a and b projections: 48 outputs from 5120, row-major (the engine keeps them
    untiled, Retile.swift:33-36)."""
    n, k = 48, 5120
    words, stride, sc, bi = oracle.q4_random_weight(n, k, seed=40 + rows)
    from qcheck import dev_u16, dev_u32
    w = rt.Q4Weight(dev_u32(words), dev_u16(sc), dev_u16(bi), n, k, rt.ROW_MAJOR, stride)
    dense = oracle.q4_dequant_rowmajor(words, stride, sc, bi, n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=41 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    for out_dtype in (torch.float32, torch.bfloat16):
        got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype))
        check_close(got, ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=abs_gemm(a_bits, dense),
                    label=f"48-row projection rows={rows}")
