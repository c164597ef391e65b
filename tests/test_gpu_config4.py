"""Config 4 (every projection of one hybrid layer set at M=64, and the 5120 -> 248320 lm_head at
M=1 and M=64) and config 1's fused gate+up at full size, all through AUTO -- the kernels the bench
times -- against the oracle on sampled output columns. Also: one workspace shared by calls of
different shapes, row counts and kernels (the split-K arrival counters sit at a fixed place)."""
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


# (name, N, K): attention q/o 5120 x 5120, k/v 5120 -> 1024, gated-delta input projections
# 5120 -> 12288 and output 6144 -> 5120, and the MLP down projection.
LAYER_SET = [("attn_q", 5120, 5120), ("attn_kv", 1024, 5120), ("gdn_in", 12288, 5120), ("gdn_out", 5120, 6144),
             ("mlp_down", 5120, 17408)]


@pytest.mark.parametrize("name,n,k", LAYER_SET)
def test_layer_set_projection_m64(rt, name, n, k):
    rows = 64
    w = _full_size_weight(rt, n, k, seed=n + 3 * k)
    a_bits = oracle.bf16_normal((rows, k), seed=n % 97)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    cols = np.sort(np.random.default_rng(n + k).choice(n, 384, replace=False))
    ref, absref = _sampled_reference(w, a_bits, cols)
    check_close(got[:, cols], ref, bf16_out=True, tight=True, absref=absref, label=f"{name} {n}x{k}")


@pytest.mark.parametrize("rows", [1, 64])
def test_lm_head_sampled(rt, rows):
    n, k = 248320, 5120
    w = _full_size_weight(rt, n, k, seed=31 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=33)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    cols = np.sort(np.random.default_rng(rows).choice(n, 256, replace=False))
    ref, absref = _sampled_reference(w, a_bits, cols)
    check_close(got[:, cols], ref, bf16_out=True, tight=True, absref=absref, label=f"lm_head rows={rows}")
    del w, got
    torch.cuda.empty_cache()


@pytest.mark.parametrize("rows", [8, 64])
def test_fused_gate_up_full_size_auto(rt, rows):
    """Config 1's fused gate+up (K=5120 -> 2 x 17408) through AUTO (the stream-K MFMA kernel the
    bench times), bf16 out: 512 sampled columns against silu(gate) * up of the oracle."""
    n, k = 17408, 5120
    gate, up = _full_size_weight(rt, n, k, seed=201), _full_size_weight(rt, n, k, seed=202)
    a_bits = oracle.bf16_normal((rows, k), seed=203)
    got = to_f32(rt.mlp_in(gate, up, bf16_tensor(a_bits)))
    cols = np.sort(np.random.default_rng(rows + 5).choice(n, 512, replace=False))
    g, _ = _sampled_reference(gate, a_bits, cols)
    u, _ = _sampled_reference(up, a_bits, cols)
    check_close(got[:, cols], oracle.silu_mul(g, u), bf16_out=True, label=f"gate+up rows={rows}")


def test_workspace_shared_across_shapes(rt):
    """One zero-filled workspace, sized for the largest call, used in turn by fused and single
    GEMMs, Q5_K, and row counts 8 -> 64 -> 8, each call twice: every result matches the oracle
    (and itself), so no call reads another's partials as arrival counters."""
    cases = {}
    gate, up = Q4Case(2176, 5120, seed=61), Q4Case(2176, 5120, seed=62)
    single = Q4Case(640, 4352, seed=63)
    native = oracle.q45k_random_native(640, 4352, seed=64)
    from qcheck import dev_u8
    w5 = rt.q5k_repack(dev_u8(native), 640, 4352)
    dense5 = oracle.q45k_decode(native).reshape(640, 4352)
    need = max(rt.workspace_bytes(r, n, k) for r in (8, 64, 96) for n, k in ((2176, 5120), (640, 4352)))
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    # 96 rows: one tiled weight and a row-major pair go to the split-K tile kernel, whose partials
    # must stay clear of the counters the M <= 64 calls after it rely on.
    seq = [("mlp", 8), ("gemm", 64), ("q5k", 64), ("gemm", 96), ("mlp", 64), ("mlp_rm", 96), ("gemm", 8),
           ("q5k", 16), ("mlp", 8), ("gemm", 64)]
    for kind, rows in seq:
        k = 5120 if kind.startswith("mlp") else 4352
        a_bits = oracle.bf16_normal((rows, k), seed=rows + len(kind))
        a = bf16_tensor(a_bits)
        if kind == "mlp":
            ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, gate.dense), oracle.gemm_a_bf16_w_f32(a_bits, up.dense))
            run = lambda: rt.mlp_in(gate.w_tiled, up.w_tiled, a, out_dtype=torch.float32, workspace=ws)
        elif kind == "mlp_rm":
            ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, gate.dense), oracle.gemm_a_bf16_w_f32(a_bits, up.dense))
            run = lambda: rt.mlp_in(gate.w_rm, up.w_rm, a, out_dtype=torch.float32, workspace=ws)
        elif kind == "gemm":
            ref = oracle.gemm_a_bf16_w_f32(a_bits, single.dense)
            run = lambda: rt.gemm(single.w_tiled, a, out_dtype=torch.float32, workspace=ws)
        else:
            ref = oracle.gemm_a_bf16_w_f32(a_bits, dense5)
            run = lambda: rt.gemm(w5, a, out_dtype=torch.float32, workspace=ws)
        first = run().cpu().numpy()
        check_close(first, ref, bf16_out=False, label=f"{kind} rows={rows}")
        again = run().cpu().numpy()
        assert np.array_equal(first, again), f"{kind} rows={rows}: second call differs"
    # Every counter is back at zero.
    assert int(ws[:16384].view(torch.int32).abs().sum().item()) == 0
