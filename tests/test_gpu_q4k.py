"""GGUF Q4_K on the GPU (GgufQuant.swift:44,151,191-212: decodeQ45K without fifth bits; planes per
GgufPlanes.swift:64, no plane1) against the CPU oracle: repack/unpack and decode bit-exact
(including the real Q4_K golden block), GEMM to the path's tolerance at every row-count path
(decode, MFMA, streaming)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from qcheck import abs_gemm, bf16_tensor, check_close, dev_u8, to_f32

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "gguf_golden_blocks.json"


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


def _native(n, k, seed):
    """Seeded native Q4_K rows with the real golden block (GgufGoldenBlocks.swift) at row 3, block 1."""
    native = oracle.q45k_random_native(n, k, seed=seed, fifth_bit=False).reshape(n, -1)
    golden = json.loads(GOLDEN.read_text())["q4K"]
    native[3, 144:288] = np.array(golden["bytes"], np.uint8)
    return native.reshape(-1), golden


def test_repack_unpack_and_dequant_bit_exact(rt):
    n, k = 256, 1024
    native, golden = _native(n, k, seed=5)
    w = rt.q4k_repack(dev_u8(native), n, k)
    p0, _, meta = oracle.q45k_repack(native, n, k, fifth_bit=False)
    assert np.array_equal(w.plane0.cpu().numpy(), p0)
    assert np.array_equal(w.meta.cpu().numpy(), meta)
    assert np.array_equal(rt.q4k_unpack(w).cpu().numpy(), native)
    got = rt.dequant(w).cpu().numpy()
    want = oracle.q45k_decode(native, fifth_bit=False).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    values = np.array([np.float32(v) for v in golden["values"]], np.float32)
    assert np.array_equal(got[3, 256:512].view(np.uint32), values.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 2, 16, 64, 100, 200, 300])
def test_gemm_paths(rt, rows):
    n, k = 384, 2048
    native, _ = _native(n, k, seed=10 + rows)
    w = rt.q4k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native, fifth_bit=False).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=20 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype))
        check_close(got, ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"q4k rows={rows} {out_dtype}")
    if rows == 1:
        base = np.random.default_rng(3).normal(size=(1, n)).astype(np.float32)
        out = torch.from_numpy(base.copy()).cuda()
        rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out)
        check_close(out.cpu().numpy(), ref + base, bf16_out=False, tight=True, absref=absref, label="q4k residual")


@pytest.mark.parametrize("kernel", ["STREAM", "SCALAR", "DEQUANT", "TILE", "PREFILL"])
def test_gemm_explicit_kernels(rt, kernel):
    n, k, rows = 256, 1280, 5
    native, _ = _native(n, k, seed=30)
    w = rt.q4k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native, fifth_bit=False).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=31)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=getattr(rt, kernel)))
    check_close(got, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label=f"q4k {kernel}")
