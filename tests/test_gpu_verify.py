"""The verify kernel (tiled q4, 2 < rows <= 64) against the oracle: single weights and fused
gate+up pairs, every row count class (partial 16-row tiles, one to four of them), shapes whose
tiles all split along K, shapes with a whole group a workgroup plus split leftover tiles, the
residual and both output types, a deterministic split, and the BASELINE shapes at full size
through sampled columns."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import Q4Case, abs_gemm, bf16_tensor, check_close, to_f32
from test_gpu_q4 import _full_size_weight, _sampled_reference

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


@pytest.mark.parametrize("rows", [3, 16, 17, 40, 64])
@pytest.mark.parametrize("n,k", [(384, 512), (2048, 1280), (17408 // 4, 1024)])
def test_verify_gemm(rt, rows, n, k):
    case = Q4Case(n, k, seed=rows + n)
    a_bits = oracle.bf16_normal((rows, k), seed=rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    absref = abs_gemm(a_bits, case.dense)
    a = bf16_tensor(a_bits)
    got = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY)
    check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=absref, label=f"f32 {rows}x{n}x{k}")
    got = rt.gemm(case.w_tiled, a, kernel=rt.VERIFY)
    check_close(to_f32(got), ref, bf16_out=True, tight=True, absref=absref, label=f"bf16 {rows}x{n}x{k}")
    res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=7).astype(np.float32)).cuda()
    got = rt.gemm(case.w_tiled, a, out=res.clone(), out_dtype=torch.float32, kernel=rt.VERIFY, residual=res)
    check_close(got.cpu().numpy(), ref + res.cpu().numpy(), bf16_out=False, label=f"residual {rows}x{n}x{k}")


@pytest.mark.parametrize("rows", [3, 33, 64])
@pytest.mark.parametrize("n,k", [(384, 512), (17408 // 4, 1280)])
def test_verify_mlp_in(rt, rows, n, k):
    gate, up = Q4Case(n, k, seed=90 + rows), Q4Case(n, k, seed=91 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=92)
    ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, gate.dense), oracle.gemm_a_bf16_w_f32(a_bits, up.dense))
    a = bf16_tensor(a_bits)
    got = rt.mlp_in(gate.w_tiled, up.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY)
    check_close(got.cpu().numpy(), ref, bf16_out=False, label=f"mlp f32 {rows}x{n}x{k}")
    got = rt.mlp_in(gate.w_tiled, up.w_tiled, a, kernel=rt.VERIFY)
    check_close(to_f32(got), ref, bf16_out=True, label=f"mlp bf16 {rows}x{n}x{k}")


@pytest.mark.parametrize("split", [1, 2])
@pytest.mark.parametrize("rows", [5, 24, 48, 64])
def test_verify_long_k(rt, monkeypatch, split, rows):
    """Whole-K (or two-piece) tiles over K = 4096: each wave runs eight (gate+up) or four chunks
    through the pipelined loop and its remainder, for every count of 16-row tiles."""
    monkeypatch.setenv("SPLOSH_VERIFY_SPLIT", str(split))
    n, k = 384, 4096
    gate, up = Q4Case(n, k, seed=97 + rows), Q4Case(n, k, seed=98 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=99)
    g = oracle.gemm_a_bf16_w_f32(a_bits, gate.dense)
    a = bf16_tensor(a_bits)
    got = rt.gemm(gate.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY)
    check_close(got.cpu().numpy(), g, bf16_out=False, tight=True, absref=abs_gemm(a_bits, gate.dense),
                label=f"long k rows={rows} split={split}")
    ref = oracle.silu_mul(g, oracle.gemm_a_bf16_w_f32(a_bits, up.dense))
    got = rt.mlp_in(gate.w_tiled, up.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY)
    check_close(got.cpu().numpy(), ref, bf16_out=False, label=f"long k mlp rows={rows} split={split}")


def test_verify_split_is_deterministic_and_needs_workspace(rt):
    rows, n, k = 64, 256, 4096
    case = Q4Case(n, k, seed=93)
    a = bf16_tensor(oracle.bf16_normal((rows, k), seed=94))
    need = rt.workspace_bytes(rows, n, k)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    first = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY, workspace=ws).cpu().numpy()
    for _ in range(3):
        again = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, kernel=rt.VERIFY, workspace=ws).cpu().numpy()
        assert np.array_equal(first, again)
    with pytest.raises(RuntimeError, match="verify kernel"):
        rt.gemm(case.w_tiled, a, kernel=rt.VERIFY, workspace=torch.zeros(16, dtype=torch.uint8, device="cuda"))
    # AUTO without room for the split falls back to another kernel.
    got = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, workspace=torch.zeros(16, dtype=torch.uint8, device="cuda"))
    check_close(got.cpu().numpy(), first, bf16_out=False, label="fallback")


def test_verify_rejects_row_major_and_out_of_range_rows(rt):
    case = Q4Case(384, 512, seed=95)
    for rows, w in ((64, case.w_rm), (2, case.w_tiled), (65, case.w_tiled)):
        a = bf16_tensor(oracle.bf16_normal((rows, 512), seed=96))
        with pytest.raises(RuntimeError, match="verify kernel"):
            rt.gemm(w, a, kernel=rt.VERIFY)


@pytest.mark.parametrize("rows", [8, 64])
def test_verify_baseline_mlp_sampled(rt, rows):
    """Config 1's fused gate+up (K=5120 -> 2 x 17408) at full size through the verify kernel:
    512 sampled output columns against the oracle."""
    n, k = 17408, 5120
    gate, up = _full_size_weight(rt, n, k, seed=101), _full_size_weight(rt, n, k, seed=102)
    a_bits = oracle.bf16_normal((rows, k), seed=103)
    got = to_f32(rt.mlp_in(gate, up, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=rt.VERIFY))
    cols = np.sort(np.random.default_rng(rows).choice(n, 512, replace=False))
    g, _ = _sampled_reference(gate, a_bits, cols)
    u, _ = _sampled_reference(up, a_bits, cols)
    check_close(got[:, cols], oracle.silu_mul(g, u), bf16_out=False, label=f"mlp full rows={rows}")
