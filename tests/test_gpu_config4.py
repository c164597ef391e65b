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


@pytest.mark.parametrize("order", ["tiled", "rowmajor"])
@pytest.mark.parametrize("rows", [8, 33, 64])
def test_wide_weight_as_split_pair(rt, order, rows):
    """A single weight with at least four bands of 64 columns a CU runs as the pair of its column
    halves (rows [0, N/2) and [N/2, N) of the weight through the fused-pair kernel, each half's sums
    stored to its own columns). N = 66048: sampled columns of both halves, and the columns next to
    the seam, against the oracle; with a workspace (stream-K) and without (whole bands); bf16 and
    fp32 out with a residual."""
    n, k = 66048, 512
    g = k // 64
    if order == "tiled":
        w = _full_size_weight(rt, n, k, seed=400 + rows)
    else:
        gen = torch.Generator(device="cuda").manual_seed(401 + rows)
        stride = 64  # 512 codes a row = 256 bytes, a whole number of 128-byte lines
        packed = torch.randint(-2**31, 2**31, (n * stride,), dtype=torch.int64, device="cuda", generator=gen).to(torch.int32)
        scales = (torch.randn(n * g, device="cuda", generator=gen) * 0.02).abs().to(torch.bfloat16).view(torch.int16)
        biases = (torch.randn(n * g, device="cuda", generator=gen) * 0.01).to(torch.bfloat16).view(torch.int16)
        w = rt.Q4Weight(packed, scales, biases, n, k, rt.ROW_MAJOR, stride)
    a_bits = oracle.bf16_normal((rows, k), seed=402 + rows)
    half = n // 2
    cols = np.unique(np.concatenate([np.random.default_rng(rows).choice(n, 256, replace=False),
                                     np.arange(half - 3, half + 3), [0, n - 1]]))
    if order == "tiled":
        ref, absref = _sampled_reference(w, a_bits, cols)
    else:
        words = w.packed.cpu().numpy().view(np.uint32).reshape(n, -1)
        sc = w.scales.cpu().numpy().view(np.uint16).reshape(n, g)
        bi = w.biases.cpu().numpy().view(np.uint16).reshape(n, g)
        dense = oracle.q4_dequant_rowmajor(words[cols], words.shape[1], sc[cols], bi[cols], len(cols), k)
        ref, absref = oracle.gemm_a_bf16_w_f32(a_bits, dense), abs_gemm(a_bits, dense)
    a = bf16_tensor(a_bits)
    for ws in (None, torch.empty(0, dtype=torch.uint8, device="cuda")):
        got = to_f32(rt.gemm(w, a, workspace=ws))
        check_close(got[:, cols], ref, bf16_out=True, tight=True, absref=absref,
                    label=f"split {order} rows={rows} split-K={ws is None}")
    res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=403).astype(np.float32)).cuda()
    got = rt.gemm(w, a, out=res.clone(), out_dtype=torch.float32, residual=res).cpu().numpy()
    check_close(got[:, cols], ref + res.cpu().numpy()[:, cols], bf16_out=False, label=f"split {order} residual")


@pytest.mark.parametrize("rows", [8, 64, 96])
def test_fused_gate_up_full_size_auto(rt, rows):
    """Config 1's fused gate+up (K=5120 -> 2 x 17408) through AUTO (the stream-K MFMA kernel the
    bench times; 96 rows as two calls of it), bf16 out: 512 sampled columns against silu(gate) * up
    of the oracle."""
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
    # 96 rows: under AUTO two calls of the M <= 64 kernel (64 + 32 rows) on the one workspace; by
    # name, the split-K tile kernel, whose partials must stay clear of the counters the M <= 64
    # calls after it rely on.
    seq = [("mlp", 8), ("gemm", 64), ("q5k", 64), ("gemm", 96), ("mlp", 64), ("mlp_rm", 96), ("gemm_tile", 96),
           ("mlp_tile", 96), ("gemm", 8), ("q5k", 16), ("mlp", 8), ("gemm", 64)]
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
        elif kind == "mlp_tile":
            ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, gate.dense), oracle.gemm_a_bf16_w_f32(a_bits, up.dense))
            run = lambda: rt.mlp_in(gate.w_tiled, up.w_tiled, a, out_dtype=torch.float32, workspace=ws, kernel=rt.TILE)
        elif kind == "gemm":
            ref = oracle.gemm_a_bf16_w_f32(a_bits, single.dense)
            run = lambda: rt.gemm(single.w_tiled, a, out_dtype=torch.float32, workspace=ws)
        elif kind == "gemm_tile":
            ref = oracle.gemm_a_bf16_w_f32(a_bits, single.dense)
            run = lambda: rt.gemm(single.w_tiled, a, out_dtype=torch.float32, workspace=ws, kernel=rt.TILE)
        else:
            ref = oracle.gemm_a_bf16_w_f32(a_bits, dense5)
            run = lambda: rt.gemm(w5, a, out_dtype=torch.float32, workspace=ws)
        first = run().cpu().numpy()
        check_close(first, ref, bf16_out=False, label=f"{kind} rows={rows}")
        again = run().cpu().numpy()
        assert np.array_equal(first, again), f"{kind} rows={rows}: second call differs"
    # Every counter is back at zero.
    assert int(ws[:16384].view(torch.int32).abs().sum().item()) == 0


@pytest.mark.parametrize("rows", [1, 8, 33, 64, 100])
def test_gemm_group_attention_qkv(rt, rows):
    """Config 4's attention inputs, q (5120 x 5120), k and v (5120 -> 1024), as one grouped call:
    one launch of the M <= 64 kernel over their joined bands (rows <= 64), three calls above; each
    output against the oracle on sampled columns (bf16 out)."""
    k = 5120
    shapes = (5120, 1024, 1024)
    ws = [_full_size_weight(rt, n, k, seed=300 + i) for i, n in enumerate(shapes)]
    a_bits = oracle.bf16_normal((rows, k), seed=310 + rows)
    outs = rt.gemm_group(ws, bf16_tensor(a_bits))
    for i, (w, out, n) in enumerate(zip(ws, outs, shapes)):
        assert tuple(out.shape) == (rows, n)
        cols = np.sort(np.random.default_rng(320 + i).choice(n, 192, replace=False))
        ref, absref = _sampled_reference(w, a_bits, cols)
        check_close(to_f32(out)[:, cols], ref, bf16_out=True, tight=True, absref=absref,
                    label=f"group weight {i} rows={rows}")


def test_gemm_group_small_shapes_and_workspace(rt):
    """Four small tiled weights of different widths into strided fp32 outputs of one buffer, twice
    on one shared workspace (same results; every counter back at zero), against the oracle on
    every column; and the argument checks."""
    k = 1024
    cases = [Q4Case(n, k, seed=330 + n) for n in (128, 384, 256, 640)]
    ws = [c.w_tiled for c in cases]
    total = sum(c.n for c in cases)
    rows = 40
    a_bits = oracle.bf16_normal((rows, k), seed=341)
    buf = torch.zeros(rows, total + 16, dtype=torch.float32, device="cuda")
    views, c0 = [], 0
    for c in cases:
        views.append(buf[:, c0:c0 + c.n])
        c0 += c.n
    need = rt.workspace_bytes(rows, total, k)
    scratch = torch.zeros(max(need, 16384), dtype=torch.uint8, device="cuda")
    rt.gemm_group(ws, bf16_tensor(a_bits), outs=views, workspace=scratch)
    first = buf.cpu().numpy().copy()
    c0 = 0
    for c in cases:
        ref = oracle.gemm_a_bf16_w_f32(a_bits, c.dense)
        check_close(first[:, c0:c0 + c.n], ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, c.dense),
                    label=f"group n={c.n}")
        c0 += c.n
    assert not first[:, total:].any()  # columns past the views untouched
    rt.gemm_group(ws, bf16_tensor(a_bits), outs=views, workspace=scratch)
    assert np.array_equal(first, buf.cpu().numpy())
    assert int(scratch[:16384].view(torch.int32).abs().sum().item()) == 0
    from splosh_amd._lib import SploshError
    with pytest.raises(SploshError):
        rt.gemm_group(ws + [Q4Case(128, 512, seed=1).w_tiled], bf16_tensor(a_bits))  # inner differs
    with pytest.raises(SploshError):
        rt.gemm_group(ws * 3, bf16_tensor(a_bits))  # more than SPLOSH_MAX_GROUP
