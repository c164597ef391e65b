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


# ---- the value-head order of a gated-delta out projection (engine_gguf.metal:55-72) ----------

def _heads_case(m, n, seed):
    a_bits = oracle.bf16_normal((m, 6144), seed=seed)
    return a_bits, oracle.head_gather(a_bits)


@pytest.mark.parametrize("m", [1, 2, 16, 64, 100])
@pytest.mark.parametrize("fifth", [True, False])
def test_heads_gemm_planes(m, fifth):
    """A head-ordered Q5_K / Q4_K weight (inner 6144 = 48 value heads of 128, in the file's order)
    times activations in the engine's order equals the plain GEMM with the activations gathered
    into the file's order: in-kernel at one and two rows (decode kernel), through the permuted copy
    above (the M <= 64 and prefill kernels)."""
    from splosh_amd import runtime as rt
    from qcheck import dev_u8
    n, k = 256, 6144
    native = oracle.q45k_random_native(n, k, seed=80 + m, fifth_bit=fifth)
    w = (rt.q5k_repack if fifth else rt.q4k_repack)(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native, fifth_bit=fifth).reshape(n, k)
    a_bits, a_file = _heads_case(m, n, 81 + m)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, key_heads=16))
    check_close(got, oracle.gemm_a_bf16_w_f32(a_file, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_file, dense), label=f"heads fifth={fifth} m={m}")
    # and it is not the unpermuted product
    plain = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    assert np.abs(got - plain).max() > 1e-3 * np.abs(plain).max()


@pytest.mark.parametrize("gtype,m", [(14, 1), (14, 4), (8, 1), (8, 5), (11, 7), (21, 2), (14, 16), (8, 16), (14, 256)])
def test_heads_gemm_native(gtype, m):
    """The same for native blocks: the streaming kernels read the activations in head order
    directly, the tiled (16 rows) and prefill (256 rows) kernels get the permuted copy."""
    from splosh_amd import runtime as rt
    n, k = 256 if m < 256 else 128, 6144
    native = oracle.gguf_random_native(gtype, n, k, seed=90 + m)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), gtype, n, k)
    dense = oracle.gguf_decode(gtype, native).reshape(n, k)
    a_bits, a_file = _heads_case(m, n, 91 + m)
    ws = torch.zeros(rt.heads_workspace_bytes(m, n, k), dtype=torch.uint8, device="cuda")
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, key_heads=16, workspace=ws))
    check_close(got, oracle.gemm_a_bf16_w_f32(a_file, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_file, dense), label=f"heads type={gtype} m={m}")
    # The same weight in the ROWS32 order: the same result, bit for bit.
    got32 = to_f32(rt.gemm(rt.gguf_repack_rows32(w), bf16_tensor(a_bits), out_dtype=torch.float32, key_heads=16,
                           workspace=ws))
    assert np.array_equal(got, got32)


@pytest.mark.parametrize("m", [1, 64])
def test_heads_gemm_out_projection_full_size(m):
    """The gated-delta out projection at its real shape, 6144 -> 5120 in Q5_K, head-ordered: every
    output column at one row, a sample of 256 columns at 64 rows, against the oracle with the
    activations gathered into the file's head order."""
    from splosh_amd import runtime as rt
    from qcheck import dev_u8
    n, k = 5120, 6144
    native = oracle.q45k_random_native(n, k, seed=95)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits, a_file = _heads_case(m, n, 96 + m)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, key_heads=16))
    cols = np.arange(n) if m == 1 else np.sort(np.random.default_rng(97).choice(n, 256, replace=False))
    blocks = native.reshape(n, k // 256, 176)[cols].reshape(-1)
    dense = oracle.q45k_decode(blocks).reshape(len(cols), k)
    check_close(got[:, cols], oracle.gemm_a_bf16_w_f32(a_file, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_file, dense), label=f"out projection heads m={m}")


def test_heads_workspace_too_small():
    from splosh_amd import runtime as rt
    from splosh_amd._lib import SploshError
    from qcheck import dev_u8
    n, k, m = 128, 6144, 16
    w = rt.q5k_repack(dev_u8(oracle.q45k_random_native(n, k, seed=98)), n, k)
    a = bf16_tensor(oracle.bf16_normal((m, k), seed=99))
    with pytest.raises(SploshError) as e:
        rt.gemm(w, a, key_heads=16, workspace=torch.zeros(1024, dtype=torch.uint8, device="cuda"))
    assert e.value.case == "workspaceTooSmall"
    with pytest.raises(SploshError):
        rt.gemm(w, a, key_heads=3)  # not a power of two


def test_gguf_file_head_ordered_and_float_weights(tmp_path):
    """load_weight on a gated-delta layer's tensors: attn_gate (Q5_K, 128 rows a head) and ssm_beta
    (f32, one row a head) come out with their rows in the engine's head order, the f32 one
    requantised to Q8_0 exactly as GgufConvert.q8_0Blocks; ssm_out keeps its columns (file order)."""
    from splosh_amd import runtime as rt
    k = 512
    gate_rows = 48 * 128
    gate = oracle.q45k_random_native(gate_rows, k, seed=100)
    beta = np.random.default_rng(101).standard_normal(48 * k).astype(np.float32)
    path = gguf.write_gguf(tmp_path / "g.gguf", [("general.architecture", 8, "qwen35")],
                           [("blk.0.attn_gate.weight", gguf.Q5_K, [k, gate_rows], gate.tobytes()),
                            ("blk.0.ssm_beta.weight", 0, [k, 48], beta.tobytes())])
    f = gguf.GgufFile(path)
    wg = gguf.load_weight(f, "blk.0.attn_gate.weight")
    got = rt.dequant(wg).cpu().numpy()
    want = oracle.order_rows(gate, gate_rows, k // 256 * 176, 0, 128)
    assert np.array_equal(got.view(np.uint32), oracle.q45k_decode(want).reshape(gate_rows, k).view(np.uint32))
    wb = gguf.load_weight(f, "blk.0.ssm_beta.weight")
    assert (wb.gguf_type, wb.rows, wb.inner) == (8, 48, k)
    q8 = oracle.order_rows(oracle.q8_0_blocks(beta), 48, k // 32 * 34, 0, 1)
    assert np.array_equal(wb.native.cpu().numpy(), q8)
    a_bits = oracle.bf16_normal((3, k), seed=102)
    out = to_f32(rt.gemm(wb, bf16_tensor(a_bits), out_dtype=torch.float32))
    dense = oracle.gguf_decode(8, q8).reshape(48, k)
    check_close(out, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label="requantised beta")
