"""The operand producers on the GPU against the CPU oracle: bf16 values bit-exact (silu within
one bf16 step where the device exp differs from the host's in its last bit), per-64 sums to fp32
summation order, the row scale to a few ulp."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


SHAPES = [(1, 64), (3, 320), (64, 5120), (7, 17408), (64, 6144)]


@pytest.mark.parametrize("rows,dim", SHAPES)
def test_prepare_operand(rt, rows, dim):
    x = (np.random.default_rng(rows + dim).normal(size=(rows, dim)) * 2).astype(np.float32)
    out, sums = rt.prepare_operand(torch.from_numpy(x).cuda())
    want, want_sums = oracle.prepare_operand(x)
    assert np.array_equal(_bits(out), want)
    np.testing.assert_allclose(sums.cpu().numpy(), want_sums, rtol=1e-5, atol=1e-4)


def test_prepare_operand_strided(rt):
    """Row strides wider than dim, on both sides."""
    rows, dim = 5, 256
    x = (np.random.default_rng(9).normal(size=(rows, dim + 64))).astype(np.float32)
    out = torch.zeros((rows, dim + 128), dtype=torch.bfloat16, device="cuda")
    xs = torch.from_numpy(x).cuda()[:, :dim]
    o, sums = rt.prepare_operand(xs, out=out[:, :dim])
    want, want_sums = oracle.prepare_operand(x[:, :dim])
    assert np.array_equal(_bits(o), want)
    assert torch.all(out[:, dim:] == 0)
    np.testing.assert_allclose(sums.cpu().numpy(), want_sums, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("rows,dim", SHAPES)
@pytest.mark.parametrize("scaled", [False, True])
def test_silu_mul_operand(rt, rows, dim, scaled):
    rng = np.random.default_rng(100 + rows)
    g = (rng.normal(size=(rows, dim)) * 3).astype(np.float32)
    u = rng.normal(size=(rows, dim)).astype(np.float32)
    s = rng.uniform(0.5, 2.0, size=rows).astype(np.float32) if scaled else None
    out, sums = rt.silu_mul_operand(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(),
                                    None if s is None else torch.from_numpy(s).cuda())
    want, want_sums = oracle.silu_mul_operand(g, u, s)
    got = _bits(out)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1 and np.mean(diff == 0) > 0.995, (diff.max(), np.mean(diff == 0))
    vals = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    np.testing.assert_allclose(sums.cpu().numpy(), vals.reshape(rows, dim // 64, 64).sum(-1), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("rows,dim", SHAPES)
def test_emit_operand_and_row_inv(rt, rows, dim):
    rng = np.random.default_rng(200 + rows)
    h = rng.normal(size=(rows, dim)).astype(np.float32)
    w = rng.normal(1.0, 0.1, size=dim).astype(np.float32)
    wt = torch.from_numpy(w).to(torch.bfloat16).cuda()
    values, sums, squares = rt.emit_operand(torch.from_numpy(h).cuda(), wt)
    want_v, want_s, want_q = oracle.emit_operand(h, _bits(wt))
    assert np.array_equal(_bits(values), want_v)
    np.testing.assert_allclose(sums.cpu().numpy(), want_s, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(squares.cpu().numpy(), want_q, rtol=1e-5)
    inv = rt.row_inv(squares, dim, 1e-6).cpu().numpy()
    np.testing.assert_allclose(inv, oracle.row_inv(want_q, dim, 1e-6), rtol=3e-7 * 8)


def test_operand_rejects_bad_arguments(rt):
    x = torch.zeros((2, 100), device="cuda")
    with pytest.raises(rt.SploshError):
        rt.prepare_operand(x)  # dim not a multiple of 64


@pytest.mark.parametrize("kernel", ["auto", "dequant"])
@pytest.mark.parametrize("rows", [1, 5, 33, 64, 100])
@pytest.mark.parametrize("n,k", [(640, 4352), (5120, 1280)])
def test_gemm_emit(rt, rows, n, k, kernel):
    """Engine.gemm with emit (engine_na.metal:322-473): the residual projection's fp32 output, and
    the next norm's operand computed from that output -- fused into the M <= 64 kernel's epilogue
    (kernel DEQUANT, rows <= 64, with and without split bands), a separate pass after the GEMM
    (AUTO). The values are bit-exact against the oracle's operand of the kernel's own output; sums
    and squares agree to fp32 summation order."""
    if kernel == "dequant" and rows > 64:
        pytest.skip("the M <= 64 kernel takes at most 64 rows")
    kcode = rt.DEQUANT if kernel == "dequant" else rt.AUTO
    from qcheck import Q4Case, abs_gemm, bf16_tensor, check_close
    case = Q4Case(n, k, seed=rows + n)
    a_bits = oracle.bf16_normal((rows, k), seed=rows)
    res = np.random.default_rng(rows).normal(size=(rows, n)).astype(np.float32)
    wn = torch.from_numpy(np.random.default_rng(7).normal(1.0, 0.1, size=n).astype(np.float32)).to(torch.bfloat16).cuda()
    out = torch.from_numpy(res.copy()).cuda()
    got, values, sums, squares = rt.gemm_emit(case.w_tiled, bf16_tensor(a_bits), wn, out=out, residual=out,
                                              kernel=kcode)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense) + res
    h = got.cpu().numpy()
    check_close(h, ref, bf16_out=False, label=f"emit out rows={rows}")
    want_v, want_s, want_q = oracle.emit_operand(h, _bits(wn))
    assert np.array_equal(_bits(values), want_v)
    np.testing.assert_allclose(sums.cpu().numpy(), want_s, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(squares.cpu().numpy(), want_q, rtol=1e-5)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("rows", [256, 300, 600])
@pytest.mark.parametrize("n,k", [(640, 4352), (5120, 1280)])
def test_gemm_emit_prefill(rt, rows, n, k, split):
    """The emit from the prefill kernel's epilogue (AUTO from 256 rows): whole tiles write it from
    the accumulators, tiles split over workgroups from prefill_finish (split=True: the default
    workspace; False: an empty one, every tile whole). Same bar as test_gemm_emit."""
    from qcheck import Q4Case, bf16_tensor, check_close
    case = Q4Case(n, k, seed=rows + 2 * n)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 1)
    res = np.random.default_rng(rows + 1).normal(size=(rows, n)).astype(np.float32)
    wn = torch.from_numpy(np.random.default_rng(8).normal(1.0, 0.1, size=n).astype(np.float32)).to(torch.bfloat16).cuda()
    out = torch.from_numpy(res.copy()).cuda()
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    got, values, sums, squares = rt.gemm_emit(case.w_tiled, bf16_tensor(a_bits), wn, out=out, residual=out,
                                              workspace=ws)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, case.dense) + res
    h = got.cpu().numpy()
    check_close(h, ref, bf16_out=False, label=f"emit prefill out rows={rows} split={split}")
    want_v, want_s, want_q = oracle.emit_operand(h, _bits(wn))
    assert np.array_equal(_bits(values), want_v)
    np.testing.assert_allclose(sums.cpu().numpy(), want_s, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(squares.cpu().numpy(), want_q, rtol=1e-5)
