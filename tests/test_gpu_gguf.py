"""Q4_K and Q5_K weights read out of a GGUF file (Model/GgufFile.swift), repacked on the device with
their rows rounded up to whole 128-row tiles (GgufConvert.swift:259-262), dequantised bit-exact and
multiplied to the oracle's tolerance; the padding rows come out zero."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import abs_gemm, bf16_tensor, check_close, to_f32
from splosh_amd import gguf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fifth,rows", [(True, 200), (False, 128), (False, 72)])
def test_gguf_file_weights(tmp_path, fifth, rows):
    from splosh_amd import runtime as rt
    k = 1024
    native = oracle.q45k_random_native(rows, k, seed=70 + rows, fifth_bit=fifth)
    tid = gguf.Q5_K if fifth else gguf.Q4_K
    path = gguf.write_gguf(tmp_path / "w.gguf", [("general.architecture", 8, "qwen3")],
                           [("blk.0.ffn_up.weight", tid, [k, rows], native.tobytes())])
    w = gguf.load_weight(gguf.GgufFile(path), "blk.0.ffn_up.weight")
    stored = -(-rows // 128) * 128
    assert (w.rows, w.inner) == (stored, k)
    assert isinstance(w, rt.Q5KWeight if fifth else rt.Q4KWeight)
    dense = oracle.q45k_decode(native, fifth_bit=fifth).reshape(rows, k)
    got = rt.dequant(w).cpu().numpy()
    assert np.array_equal(got[:rows].view(np.uint32), dense.view(np.uint32))
    assert not got[rows:].any()
    for m in (1, 5):
        a_bits = oracle.bf16_normal((m, k), seed=71 + m)
        out = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32))
        assert not out[:, rows:].any()
        check_close(out[:, :rows], oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                    absref=abs_gemm(a_bits, dense), label=f"gguf fifth={fifth} rows={rows} m={m}")
