"""q4 (MLX affine, group 64) on the GPU against the CPU oracle.

Dequantization and retiling are bit-exact; GEMMs are held to the path's tolerance and the
streaming kernel to one bf16 rounding of the fp32-accumulate reference (qcheck.check_close)."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import Q4Case, abs_gemm, bf16_tensor, check_close, dev_u16, dev_u32, to_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


def test_q4_dequant_bit_exact(rt):
    case = Q4Case(256, 320, seed=1)
    got = rt.dequant(case.w_rm).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), case.dense.view(np.uint32))
    case = Q4Case(256, 512, seed=2)
    got = rt.dequant(case.w_tiled).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), case.dense.view(np.uint32))


def test_tile128_matches_converter(rt):
    rows, groups = 384, 5
    src = np.random.default_rng(3).integers(0, 2**32, size=rows * groups * 8, dtype=np.uint64).astype(np.uint32)
    want = oracle.tile128(src.view(np.uint8), rows, groups, 32).view(np.uint32)
    got = rt.tile128(dev_u32(src), rows, groups, 32).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want)
    back = rt.tile128(dev_u32(want), rows, groups, 32, inverse=True).cpu().numpy().view(np.uint32)
    assert np.array_equal(back, src)
    s16 = np.arange(rows * groups, dtype=np.uint16)
    assert np.array_equal(rt.tile128(dev_u16(s16), rows, groups, 2).cpu().numpy().view(np.uint16),
                          oracle.tile128(s16.view(np.uint8), rows, groups, 2).view(np.uint16))


def test_device_retile_of_a_weight(rt):
    case = Q4Case(256, 512, seed=4)
    tiled = rt.q4_to_tiled(case.w_rm)
    ref = case.w_tiled
    for name in ("packed", "scales", "biases"):
        assert torch.equal(getattr(tiled, name).view(-1)[: getattr(ref, name).numel()], getattr(ref, name).view(-1))


@pytest.mark.parametrize("rows,columns,inner", [(2, 3, 65), (3, 2, 128), (1, 1, 64)])
def test_gemm_q4_named_cases(rt, rows, columns, inner):
    """GemmOracleTests.swift:160-214 through Q4GemmRuntime.dispatch (fp32 out)."""
    from test_oracle import named_q4_case
    from splosh_amd.quant import GemmQ4Shape, Q4BufferLayout
    words, stride, sc, bi, a = named_q4_case(oracle, rows, columns, inner)
    layout = Q4BufferLayout(rows=columns, logical_k=inner)
    out = torch.full((rows, columns), float("nan"), device="cuda")
    rt.Q4GemmRuntime().dispatch(GemmQ4Shape(rows, columns, inner), layout, bf16_tensor(a), dev_u32(words),
                                dev_u16(sc), dev_u16(bi), out)
    w = oracle.q4_dequant_rowmajor(words, stride, sc, bi, columns, inner)
    ref = oracle.gemm_a_bf16_w_f32(a, w)
    assert np.allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)


def test_gemm_q4_runtime_rejects_small_buffers(rt):
    from splosh_amd.quant import GemmQ4Shape, Q4BufferLayout
    layout = Q4BufferLayout(rows=3, logical_k=65)
    small = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(rt.GemmQ4Error) as e:
        rt.Q4GemmRuntime().dispatch(GemmQ4Shape(2, 3, 65), layout, torch.zeros(130, dtype=torch.int16, device="cuda"),
                                    small, torch.zeros(6, dtype=torch.int16, device="cuda"),
                                    torch.zeros(6, dtype=torch.int16, device="cuda"),
                                    torch.zeros(6, device="cuda"))
    assert e.value.case == "bufferTooSmall"


ROWS = [1, 2, 3, 4, 5, 8, 16, 17, 31, 33, 64, 65, 100]


@pytest.mark.parametrize("kernel", ["STREAM", "TILE"])
@pytest.mark.parametrize("order", ["tiled", "rowmajor"])
@pytest.mark.parametrize("rows", ROWS)
def test_stream_gemm_rows(rt, kernel, order, rows):
    case = Q4Case(384, 768, seed=10 + rows)
    w = case.w_tiled if order == "tiled" else case.w_rm
    a_bits = oracle.bf16_normal((rows, case.k), seed=100 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    absref = abs_gemm(a_bits, case.dense)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=getattr(rt, kernel))
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"{kernel} {order} rows={rows} {out_dtype}")


@pytest.mark.parametrize("order", ["tiled", "rowmajor"])
@pytest.mark.parametrize("rows", [1, 3, 32, 33, 64])
def test_dequant_kernel(rt, order, rows):
    """Group counts that are not a multiple of the workgroup's K waves (K = 1216: 19 groups)."""
    case = Q4Case(384, 1216, seed=40 + rows)
    w = case.w_tiled if order == "tiled" else case.w_rm
    a_bits = oracle.bf16_normal((rows, case.k), seed=41)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    got = rt.gemm(w, bf16_tensor(a_bits), kernel=rt.DEQUANT)
    check_close(to_f32(got), ref, bf16_out=True, tight=True, absref=abs_gemm(a_bits, case.dense))


@pytest.mark.parametrize("kernel", ["TILE", "DEQUANT"])
@pytest.mark.parametrize("mlp", [False, True])
def test_split_k(rt, kernel, mlp):
    """Few output blocks and a long K: the tiled kernel splits K over a workspace and sums the
    slices in a second pass; with a workspace that is too small it must not split. Both agree with
    the oracle, and the split result is deterministic."""
    rows, n, k = 64, 256, 4096
    gate, up = Q4Case(n, k, seed=50), Q4Case(n, k, seed=51)
    a_bits = oracle.bf16_normal((rows, k), seed=52)
    g = oracle.gemm_a_bf16_w_f32(a_bits, gate.dense)
    ref = oracle.silu_mul(g, oracle.gemm_a_bf16_w_f32(a_bits, up.dense)) if mlp else g
    absref = abs_gemm(a_bits, gate.dense)
    need = rt.workspace_bytes(rows, n, k)
    assert need > 0
    a = bf16_tensor(a_bits)
    outs = []
    for ws in (torch.zeros(need, dtype=torch.uint8, device="cuda"), torch.zeros(16, dtype=torch.uint8, device="cuda"),
               None):
        if mlp:
            got = rt.mlp_in(gate.w_tiled, up.w_tiled, a, out_dtype=torch.float32, kernel=getattr(rt, kernel),
                            workspace=ws)
            check_close(got.cpu().numpy(), ref, bf16_out=False, label="split mlp")
        else:
            got = rt.gemm(gate.w_tiled, a, out_dtype=torch.float32, kernel=getattr(rt, kernel), workspace=ws)
            check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=absref, label="split")
        outs.append(got.cpu().numpy())
    assert np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("kernel", ["STREAM", "DEQUANT", "TILE"])
def test_stream_gemm_odd_columns_and_strides(rt, kernel):
    """Row-major weight with N not a multiple of 16, padded activation rows, output written into a
    wider buffer whose other columns and rows must stay untouched."""
    n, k, rows = 200, 448, 7
    case = Q4Case(n, k, seed=21)
    a_full = oracle.bf16_normal((rows, k + 64), seed=22)
    ref = oracle.gemm_a_bf16_w_f32(np.ascontiguousarray(a_full[:, :k]), case.dense)
    a = bf16_tensor(a_full)
    out = torch.full((rows + 2, n + 40), 7.0, dtype=torch.float32, device="cuda")
    rt.gemm(case.w_rm, a, out=out[:, :], rows=rows, kernel=getattr(rt, kernel))
    o = out.cpu().numpy()
    check_close(o[:rows, :n], ref, bf16_out=False, tight=True,
                absref=abs_gemm(np.ascontiguousarray(a_full[:, :k]), case.dense))
    assert np.all(o[:rows, n:] == 7.0) and np.all(o[rows:] == 7.0)


def test_residual_in_place(rt):
    case = Q4Case(256, 512, seed=23)
    rows = 5
    a_bits = oracle.bf16_normal((rows, case.k), seed=24)
    base = np.random.default_rng(25).normal(size=(rows, case.n)).astype(np.float32)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense) + base
    out = torch.from_numpy(base.copy()).cuda()
    rt.Engine(kernel=rt.STREAM).gemm(case.w_tiled, bf16_tensor(a_bits), out, residual=True)
    check_close(out.cpu().numpy(), ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, case.dense))


def test_scalar_kernel_any_shape(rt):
    """K not a multiple of 64 goes to the generic kernel under AUTO."""
    case = Q4Case(96, 200, seed=26)
    a_bits = oracle.bf16_normal((3, case.k), seed=27)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    got = rt.gemm(case.w_rm, bf16_tensor(a_bits), out_dtype=torch.float32)
    assert np.allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    with pytest.raises(rt.SploshError) as e:
        rt.gemm(case.w_rm, bf16_tensor(a_bits), kernel=rt.STREAM)
    assert e.value.case == "unsupported"


@pytest.mark.parametrize("kernel", ["AUTO", "STREAM", "TILE"])
@pytest.mark.parametrize("rows", [1, 2, 8, 64, 130])
def test_mlp_in_fused(rt, kernel, rows):
    k, n = 512, 384
    gate, up = Q4Case(n, k, seed=30), Q4Case(n, k, seed=31)
    a_bits = oracle.bf16_normal((rows, k), seed=32)
    g = oracle.gemm_a_bf16_w_f32(a_bits, gate.dense)
    u = oracle.gemm_a_bf16_w_f32(a_bits, up.dense)
    ref = oracle.silu_mul(g, u)
    for w_g, w_u in ((gate.w_tiled, up.w_tiled), (gate.w_rm, up.w_rm)):
        got = rt.mlp_in(w_g, w_u, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=getattr(rt, kernel))
        check_close(got.cpu().numpy(), ref, bf16_out=False, label=f"mlp rows={rows}")
        got = rt.mlp_in(w_g, w_u, bf16_tensor(a_bits), kernel=getattr(rt, kernel))
        check_close(to_f32(got), ref, bf16_out=True, label=f"mlp bf16 rows={rows}")


@pytest.mark.parametrize("rows,n,k", [(65, 384, 576), (300, 256, 640), (513, 128, 64)])
@pytest.mark.parametrize("split", [True, False])
def test_mlp_in_prefill(rt, rows, n, k, split):
    """Fused gate+up through the prefill kernel (AUTO above 128 rows for tiled weights; 65..128 rows
    run as two calls of the M <= 64 kernel): tiles of 128 columns of each weight, silu(g) * u in the
    epilogue and in the stream-K finish pass, ragged rows."""
    gate, up = Q4Case(n, k, seed=60 + rows), Q4Case(n, k, seed=61 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=62 + rows)
    g = oracle.gemm_a_bf16_w_f32(a_bits, gate.dense)
    u = oracle.gemm_a_bf16_w_f32(a_bits, up.dense)
    ref = oracle.silu_mul(g, u)
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    for out_dtype in (torch.float32, torch.bfloat16):
        got = rt.mlp_in(gate.w_tiled, up.w_tiled, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.PREFILL,
                        workspace=ws)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16,
                    label=f"mlp prefill {rows}x{n}x{k} split={split} {out_dtype}")
        auto = rt.mlp_in(gate.w_tiled, up.w_tiled, bf16_tensor(a_bits), out_dtype=out_dtype, workspace=ws)
        if rows > 128:
            assert torch.equal(auto, got), "AUTO takes the prefill kernel above 128 rows"
        else:
            check_close(to_f32(auto), ref, bf16_out=out_dtype == torch.bfloat16,
                        label=f"mlp auto (two M <= 64 calls) {rows}x{n}x{k} split={split} {out_dtype}")


def test_workspace_shared_by_prefill_and_split_k(rt):
    """One workspace for a split prefill call and then split M <= 64 calls (gemm and mlp_in): the
    prefill's partial tiles must not touch the arrival counters at the workspace's start."""
    n, k = 512, 2048
    gate, up = Q4Case(n, k, seed=70), Q4Case(n, k, seed=71)
    ws = torch.zeros(max(rt.workspace_bytes(300, n, k), rt.workspace_bytes(64, n, k)), dtype=torch.uint8,
                     device="cuda")
    for rows in (300, 64, 33, 300, 64):
        a_bits = oracle.bf16_normal((rows, k), seed=72 + rows)
        g = oracle.gemm_a_bf16_w_f32(a_bits, gate.dense)
        got = rt.gemm(gate.w_tiled, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=ws)
        check_close(got.cpu().numpy(), g, bf16_out=False, tight=True, absref=abs_gemm(a_bits, gate.dense),
                    label=f"shared workspace gemm rows={rows}")
        got = rt.mlp_in(gate.w_tiled, up.w_tiled, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=ws)
        check_close(got.cpu().numpy(), oracle.silu_mul(g, oracle.gemm_a_bf16_w_f32(a_bits, up.dense)),
                    bf16_out=False, label=f"shared workspace mlp rows={rows}")
        assert not ws[:16384].any(), f"arrival counters left nonzero after rows={rows}"


def _full_size_weight(rt, n, k, seed):
    """A BASELINE-size tiled q4 weight generated on the device (uniform code words,
    scale = bf16(|N(0, 0.02)|), bias = bf16(N(0, 0.01)))."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    groups = k // 64
    packed = torch.randint(-2**31, 2**31, (n * groups * 8,), dtype=torch.int64, device="cuda", generator=gen).to(torch.int32)
    scales = (torch.randn(n * groups, device="cuda", generator=gen) * 0.02).abs().to(torch.bfloat16).view(torch.int16)
    biases = (torch.randn(n * groups, device="cuda", generator=gen) * 0.01).to(torch.bfloat16).view(torch.int16)
    return rt.Q4Weight(packed, scales, biases, n, k, rt.TILED128)


def _sampled_reference(w, a_bits, cols):
    """The oracle on a sample of output columns of a device tiled weight (untiled on the host)."""
    n, k = w.rows, w.inner
    g = k // 64
    tw = w.packed.cpu().numpy().view(np.uint32)
    ts = w.scales.cpu().numpy().view(np.uint16)
    tb = w.biases.cpu().numpy().view(np.uint16)
    words = oracle.untile128(tw.view(np.uint8), n, g, 32).view(np.uint32).reshape(n, k // 8)
    sc = oracle.untile128(ts.view(np.uint8), n, g, 2).view(np.uint16).reshape(n, g)
    bi = oracle.untile128(tb.view(np.uint8), n, g, 2).view(np.uint16).reshape(n, g)
    dense = oracle.q4_dequant_rowmajor(words[cols], k // 8, sc[cols], bi[cols], len(cols), k)
    return oracle.gemm_a_bf16_w_f32(a_bits, dense), abs_gemm(a_bits, dense)


@pytest.mark.parametrize("rows", [1, 64])
def test_baseline_shapes_sampled(rt, rows):
    """Config 0/1 shapes (K=5120 -> N=17408, K=17408 -> N=5120) at full size, 512 sampled output
    columns checked against the oracle."""
    for n, k in ((17408, 5120), (5120, 17408)):
        w = _full_size_weight(rt, n, k, seed=n + k + rows)
        a_bits = oracle.bf16_normal((rows, k), seed=rows)
        got = rt.gemm(w, bf16_tensor(a_bits))
        cols = np.sort(np.random.default_rng(rows).choice(n, 512, replace=False))
        ref, absref = _sampled_reference(w, a_bits, cols)
        check_close(to_f32(got)[:, cols], ref, bf16_out=True, tight=True, absref=absref, label=f"{n}x{k} rows={rows}")


def test_prefill_shape_sampled(rt):
    """Config 2 (M=2048 prefill, K=5120 -> N=17408) at full size through the tiled kernel:
    256 sampled output columns of 512 sampled rows against the oracle."""
    n, k, rows = 17408, 5120, 2048
    w = _full_size_weight(rt, n, k, seed=7)
    a_bits = oracle.bf16_normal((rows, k), seed=8)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    rng = np.random.default_rng(9)
    cols = np.sort(rng.choice(n, 256, replace=False))
    sel = np.sort(rng.choice(rows, 512, replace=False))
    ref, absref = _sampled_reference(w, np.ascontiguousarray(a_bits[sel]), cols)
    check_close(got[sel][:, cols], ref, bf16_out=True, tight=True, absref=absref, label="prefill")


@pytest.mark.parametrize("rows,n,k", [(256, 256, 640), (300, 384, 576), (513, 128, 64)])
@pytest.mark.parametrize("split", [True, False])
def test_prefill_kernel(rt, rows, n, k, split):
    """The prefill kernel (two waves a SIMD): whole and partial 256 x 256 tiles, with the last round
    of tiles split over all workgroups (stream-K, a workspace) and without (every tile whole)."""
    case = Q4Case(n, k, seed=rows + n)
    a_bits = oracle.bf16_normal((rows, k), seed=k)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    absref = abs_gemm(a_bits, case.dense)
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(case.w_tiled, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.PREFILL, workspace=ws)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"prefill {rows}x{n}x{k} split={split} {out_dtype}")
    base = np.random.default_rng(3).normal(size=(rows, n)).astype(np.float32)
    out = torch.from_numpy(base.copy()).cuda()
    rt.gemm(case.w_tiled, bf16_tensor(a_bits), out=out, residual=out, kernel=rt.PREFILL, workspace=ws)
    check_close(out.cpu().numpy(), ref + base, bf16_out=False, tight=True, absref=absref,
                label=f"prefill residual {rows}x{n}x{k} split={split}")


@pytest.mark.parametrize("split", [True, False])
def test_prefill_strides_and_bounds(rt, split):
    """The prefill kernel on padded activation rows (lda > K), into a wider output buffer (ldc > N)
    whose other columns and rows must stay untouched, with a bf16 residual of that stride: ragged
    rows (300) and N (384) a multiple of 128 but not of the 256-column tile."""
    n, k, rows = 384, 576, 300
    case = Q4Case(n, k, seed=31)
    a_full = oracle.bf16_normal((rows, k + 64), seed=32)
    a_bits = np.ascontiguousarray(a_full[:, :k])
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense)
    absref = abs_gemm(a_bits, case.dense)
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    out = torch.full((rows + 3, n + 72), 7.0, dtype=torch.float32, device="cuda")
    rt.gemm(case.w_tiled, bf16_tensor(a_full), out=out, rows=rows, kernel=rt.PREFILL, workspace=ws)
    o = out.cpu().numpy()
    check_close(o[:rows, :n], ref, bf16_out=False, tight=True, absref=absref, label=f"prefill strided split={split}")
    assert np.all(o[:rows, n:] == 7.0) and np.all(o[rows:] == 7.0)
    base = np.random.default_rng(33).normal(size=(rows + 3, n + 72)).astype(np.float32)
    res = torch.from_numpy(base).cuda().to(torch.bfloat16)
    got = res.clone()
    rt.gemm(case.w_tiled, bf16_tensor(a_full), out=got, residual=got, rows=rows, kernel=rt.PREFILL, workspace=ws)
    g = got.float().cpu().numpy()
    check_close(g[:rows, :n], ref + res.float().cpu().numpy()[:rows, :n], bf16_out=True, tight=True,
                absref=absref + np.abs(res.float().cpu().numpy()[:rows, :n]), label=f"prefill strided residual split={split}")
    assert torch.equal(got[:rows, n:], res[:rows, n:]) and torch.equal(got[rows:], res[rows:])


def test_prefill_down_shape_sampled(rt):
    """Config 2's second shape (M=2048, K=17408 -> N=5120: 160 tiles, all split over the CUs) at
    full size, 256 sampled columns of 256 sampled rows."""
    n, k, rows = 5120, 17408, 2048
    w = _full_size_weight(rt, n, k, seed=11)
    a_bits = oracle.bf16_normal((rows, k), seed=12)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    rng = np.random.default_rng(13)
    cols = np.sort(rng.choice(n, 256, replace=False))
    sel = np.sort(rng.choice(rows, 256, replace=False))
    ref, absref = _sampled_reference(w, np.ascontiguousarray(a_bits[sel]), cols)
    check_close(got[sel][:, cols], ref, bf16_out=True, tight=True, absref=absref, label="prefill down")


DECODE_SHAPES = [(4096, 4096), (1024, 17408), (17408, 320), (256, 64), (2048, 5120), (16384, 1024)]


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("mlp", [False, True])
@pytest.mark.parametrize("n,k", DECODE_SHAPES)
def test_decode_kernel(rt, rows, mlp, n, k):
    """The every-CU decode kernel (AUTO for 1..4 rows of tiled weights when the staged activation
    rows fit its LDS; else kernel STREAM falls back to the streaming kernels): a
    workgroup a block of 8, 16 or 32 rows over the whole of K, so two calls give the same bits.
    The shapes cover every block size, a K of one group, K not a multiple of the workgroup's 4
    waves x steps, and long K."""
    g, u = Q4Case(n, k, seed=700 + rows), Q4Case(n, k, seed=710 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=720 + rows)
    ws = torch.empty(0, dtype=torch.uint8, device="cuda")  # the kernel takes no workspace
    if mlp:
        ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, g.dense), oracle.gemm_a_bf16_w_f32(a_bits, u.dense))
        run = lambda dt: rt.mlp_in(g.w_tiled, u.w_tiled, bf16_tensor(a_bits), out_dtype=dt, kernel=rt.STREAM, workspace=ws)
    else:
        ref = oracle.gemm_a_bf16_w_f32(a_bits, g.dense)
        run = lambda dt: rt.gemm(g.w_tiled, bf16_tensor(a_bits), out_dtype=dt, kernel=rt.STREAM, workspace=ws)
    for out_dtype in (torch.bfloat16, torch.float32):
        first = run(out_dtype)
        second = run(out_dtype)
        assert torch.equal(first.view(torch.uint8), second.view(torch.uint8)), "calls differ"
        check_close(to_f32(first), ref, bf16_out=out_dtype == torch.bfloat16, tight=not mlp,
                    label=f"decode {n}x{k} rows={rows} mlp={mlp} {out_dtype}")
    if not mlp:
        base = np.random.default_rng(5).normal(size=(rows, n)).astype(np.float32)
        out = torch.from_numpy(base.copy()).cuda()
        rt.gemm(g.w_tiled, bf16_tensor(a_bits), out=out, residual=out, kernel=rt.STREAM, workspace=ws)
        check_close(out.cpu().numpy(), ref + base, bf16_out=False, tight=True, label="decode residual")


@pytest.mark.parametrize("rows", [1, 2, 3])
@pytest.mark.parametrize("mlp", [False, True])
@pytest.mark.parametrize("n,k", [(17408, 5120), (17408, 320), (16896, 1024), (5120, 1024), (5120, 8192)])
def test_decode_balance_split(rt, rows, mlp, n, k):
    """The decode kernel with a workspace: when the row blocks do not divide evenly over the CUs
    (and every CU holds two whole blocks or more) the last round's blocks are cut into slices of K
    (on 256 CUs: 544 blocks = 512 whole + 32 in 8 slices; K=320, 5 groups: 5 slices; 528 blocks:
    16 slices of one group; 320 blocks of 16 rows: no split; K=8192 -> N=5120: 640 blocks of 8
    rows, 512 whole + 128 in 2 slices). Against the oracle, the same bits on a second call, every
    arrival counter back at zero, and within rounding of the unsplit kernel (an empty
    workspace)."""
    g, u = Q4Case(n, k, seed=730 + rows), Q4Case(n, k, seed=740 + rows)
    a_bits = oracle.bf16_normal((rows, k), seed=750 + rows)
    need = rt.workspace_bytes(rows, n, k)
    ws = torch.zeros(max(need, 16384), dtype=torch.uint8, device="cuda")
    empty = torch.empty(0, dtype=torch.uint8, device="cuda")
    if mlp:
        ref = oracle.silu_mul(oracle.gemm_a_bf16_w_f32(a_bits, g.dense), oracle.gemm_a_bf16_w_f32(a_bits, u.dense))
        run = lambda w: rt.mlp_in(g.w_tiled, u.w_tiled, bf16_tensor(a_bits), out_dtype=torch.float32,
                                  kernel=rt.STREAM, workspace=w)
    else:
        ref = oracle.gemm_a_bf16_w_f32(a_bits, g.dense)
        run = lambda w: rt.gemm(g.w_tiled, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=rt.STREAM,
                                workspace=w)
    first = run(ws).cpu().numpy()
    second = run(ws).cpu().numpy()
    assert np.array_equal(first, second), "calls differ"
    assert int(ws[:16384].view(torch.int32).abs().sum().item()) == 0, "arrival counters left set"
    check_close(first, ref, bf16_out=False, tight=not mlp, label=f"decode split {n}x{k} rows={rows} mlp={mlp}")
    whole = run(empty).cpu().numpy()
    check_close(first, whole, bf16_out=False, tight=True, label=f"split vs whole {n}x{k}")
