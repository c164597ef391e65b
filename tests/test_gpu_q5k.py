"""GGUF Q5_K on the GPU against the CPU oracle: plane repack/unpack and decode bit-exact, GEMM to
the path's tolerance. Weights follow the reference's kernel-test generator
(GgufKernelTests.swift:49-82)."""
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


def test_repack_matches_oracle_and_unpacks(rt):
    n, k = 256, 1024
    native = oracle.q45k_random_native(n, k, seed=1)
    w = rt.q5k_repack(dev_u8(native), n, k)
    p0, p1, meta = oracle.q45k_repack(native, n, k)
    assert np.array_equal(w.plane0.cpu().numpy(), p0)
    assert np.array_equal(w.plane1.cpu().numpy(), p1)
    assert np.array_equal(w.meta.cpu().numpy(), meta)
    assert np.array_equal(rt.q5k_unpack(w).cpu().numpy(), native)


def test_dequant_bit_exact_including_golden_block(rt):
    n, k = 128, 512
    native = oracle.q45k_random_native(n, k, seed=2).reshape(n, -1)
    # Put the real golden block (GgufGoldenBlocks.swift:73-122) at row 5, block 1.
    golden = json.loads(GOLDEN.read_text())["q5K"]
    native[5, 176:352] = np.array(golden["bytes"], np.uint8)
    native = native.reshape(-1)
    w = rt.q5k_repack(dev_u8(native), n, k)
    got = rt.dequant(w).cpu().numpy()
    want = oracle.q45k_decode(native).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    values = np.array([np.float32(v) for v in golden["values"]], np.float32)
    assert np.array_equal(got[5, 256:512].view(np.uint32), values.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 2, 3, 16, 17, 64, 100])
def test_stream_gemm(rt, rows):
    n, k = 256, 1280
    native = oracle.q45k_random_native_splitmix(n, k, seed=0x6600 + 13) if rows == 16 else \
        oracle.q45k_random_native(n, k, seed=rows)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=50 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.STREAM)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True,
                    label=f"q5k rows={rows} {out_dtype}")
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=rt.SCALAR)
    check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, label=f"q5k scalar rows={rows}")


def test_residual(rt):
    n, k, rows = 128, 512, 3
    native = oracle.q45k_random_native(n, k, seed=9)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=10)
    base = np.random.default_rng(11).normal(size=(rows, n)).astype(np.float32)
    dense = oracle.q45k_decode(native).reshape(n, k)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense) + base
    out = torch.from_numpy(base.copy()).cuda()
    rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out)
    check_close(out.cpu().numpy(), ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, dense))


@pytest.mark.parametrize("rows", [1, 16, 64, 200])
def test_baseline_shape_sampled(rt, rows):
    """Config 3: Q5_K down projection K=17408 -> N=5120 at full size, 256 sampled columns."""
    n, k = 5120, 17408
    native = oracle.q45k_random_native(n, k, seed=77)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=rows)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    cols = np.sort(np.random.default_rng(rows).choice(n, 256, replace=False))
    blk = k // 256 * 176
    sub = native.reshape(n, blk)[cols].reshape(-1)
    dense = oracle.q45k_decode(sub).reshape(len(cols), k)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    check_close(got[:, cols], ref, bf16_out=True, tight=True, absref=abs_gemm(a_bits, dense),
                label=f"q5k full rows={rows}")


def test_baseline_shape_prefill_sampled(rt):
    """Config 3's weight at prefill size (M=2048, the LDS-tiled MFMA kernel): 256 sampled rows x
    256 sampled columns against the oracle."""
    n, k, rows = 5120, 17408, 2048
    native = oracle.q45k_random_native(n, k, seed=78)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=79)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits)))
    rng = np.random.default_rng(80)
    cols = np.sort(rng.choice(n, 256, replace=False))
    sel = np.sort(rng.choice(rows, 256, replace=False))
    blk = k // 256 * 176
    dense = oracle.q45k_decode(native.reshape(n, blk)[cols].reshape(-1)).reshape(len(cols), k)
    a_sel = np.ascontiguousarray(a_bits[sel])
    ref = oracle.gemm_a_bf16_w_f32(a_sel, dense)
    check_close(got[sel][:, cols], ref, bf16_out=True, tight=True, absref=abs_gemm(a_sel, dense),
                label="q5k full rows=2048")


@pytest.mark.parametrize("rows", [1, 2, 3, 16, 33, 64])
@pytest.mark.parametrize("split", [True, False])
def test_dequant_kernel(rt, rows, split):
    """The MFMA kernel for up to 64 rows, with K split over workgroups (stream-K, a workspace) and
    without (every band whole)."""
    n, k = 256, 1280
    native = oracle.q45k_random_native(n, k, seed=300 + rows)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=400 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)  # the kernel rounds each dequantized weight to bf16
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.DEQUANT, workspace=ws)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"q5k dequant rows={rows} split={split} {out_dtype}")


@pytest.mark.parametrize("rows", [1, 65, 130, 300])
def test_tile_kernel(rt, rows):
    """The LDS-tiled kernel (explicit for planes; AUTO for the native formats): both tile shapes, ragged row and column blocks,
    the residual."""
    n, k = 384, 1280
    native = oracle.q45k_random_native(n, k, seed=600 + rows)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=700 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.TILE)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"q5k tile rows={rows} {out_dtype}")
    base = torch.from_numpy(oracle.bf16_normal((rows, n), seed=7).astype(np.float32)).cuda()
    out = base.clone()
    rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out, kernel=rt.TILE)
    check_close(out.cpu().numpy(), ref + base.cpu().numpy(), bf16_out=False, tight=True, absref=absref,
                label=f"q5k tile residual rows={rows}")


@pytest.mark.parametrize("rows,n,k", [(65, 384, 1280), (300, 256, 512), (513, 128, 256)])
@pytest.mark.parametrize("split", [True, False])
def test_prefill_kernel(rt, rows, n, k, split):
    """The 256 x 256 prefill kernel over planes (AUTO above 64 rows): whole and partial tiles, the
    last round split over all workgroups (stream-K) and not, K of one block, both output types,
    the residual."""
    native = oracle.q45k_random_native(n, k, seed=900 + rows)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=950 + rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype, kernel=rt.PREFILL, workspace=ws)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"q5k prefill {rows}x{n}x{k} split={split} {out_dtype}")
    base = torch.from_numpy(oracle.bf16_normal((rows, n), seed=8).astype(np.float32)).cuda()
    out = base.clone()
    rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out, kernel=rt.PREFILL, workspace=ws)
    check_close(out.cpu().numpy(), ref + base.cpu().numpy(), bf16_out=False, tight=True, absref=absref,
                label=f"q5k prefill residual {rows}x{n}x{k} split={split}")


def test_tile_kernel_large_grid(rt):
    """Enough 128 x 128 blocks for the large tile shape (512 rows), sampled rows."""
    n, k, rows = 2048, 512, 512
    native = oracle.q45k_random_native(n, k, seed=801)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=802)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, kernel=rt.TILE).cpu().numpy()
    pick = np.sort(np.random.default_rng(803).choice(rows, 48, replace=False))
    check_close(got[pick], oracle.gemm_a_bf16_w_f32(a_bits[pick], dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits[pick], dense), label="q5k tile large")


def test_dequant_kernel_remainder_bands_and_residual(rt):
    """More column bands than compute units with a remainder (whole bands and stream-K ranges in one
    launch), fp32 residual in place."""
    n, k, rows = 256 * 64 + 128, 768, 40
    native = oracle.q45k_random_native(n, k, seed=501)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=502)
    base = np.random.default_rng(503).normal(size=(rows, n)).astype(np.float32)
    dense = oracle.q45k_decode(native).reshape(n, k)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense) + base
    out = torch.from_numpy(base.copy()).cuda()
    rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out, kernel=rt.DEQUANT)
    check_close(out.cpu().numpy(), ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, dense),
                label="q5k dequant remainder")


@pytest.mark.parametrize("n,k", [(128, 256), (384, 1280), (1024, 4096), (5120, 2048), (256, 17408)])
def test_decode_kernel(rt, n, k):
    """The one-row Q5_K decode kernel (AUTO for rows == 1): all three row-block sizes (8, 16, 32 by
    the column count), K of one block, K past the first staging pass (17408), the golden block in
    place, a residual, and the same bits from two calls."""
    native = oracle.q45k_random_native(n, k, seed=900 + n).reshape(n, -1)
    golden = json.loads(GOLDEN.read_text())["q5K"]
    native[min(5, n - 1), :176] = np.array(golden["bytes"], np.uint8)
    native = native.reshape(-1)
    w = rt.q5k_repack(dev_u8(native), n, k)
    dense = oracle.q45k_decode(native).reshape(n, k)
    a_bits = oracle.bf16_normal((1, k), seed=901)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    for out_dtype in (torch.bfloat16, torch.float32):
        first = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype)
        second = rt.gemm(w, bf16_tensor(a_bits), out_dtype=out_dtype)
        assert torch.equal(first.view(torch.uint8), second.view(torch.uint8)), "calls differ"
        check_close(to_f32(first), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"q5k decode {n}x{k} {out_dtype}")
    base = np.random.default_rng(7).normal(size=(1, n)).astype(np.float32)
    out = torch.from_numpy(base.copy()).cuda()
    rt.gemm(w, bf16_tensor(a_bits), out=out, residual=out)
    check_close(out.cpu().numpy(), ref + base, bf16_out=False, tight=True, absref=absref, label="q5k decode residual")


@pytest.mark.parametrize("n,k", [(5120, 2048), (5120, 17408), (5248, 1024)])
def test_decode_balance_split(rt, n, k):
    """The Q5_K decode kernel with a workspace: on 256 CUs 640 blocks of 8 rows are 512 whole + 128
    in 2 slices of K, 656 blocks 512 + 144 unsplit (one slice each does not fit the CUs: no
    split), the partials summed by the last slice in slice order. Against the oracle (K=2048), the same bits on a second call, every
    arrival counter back at zero, and within rounding of the unsplit kernel (no workspace)."""
    native = oracle.q45k_random_native(n, k, seed=950 + n + k)
    w = rt.q5k_repack(dev_u8(native), n, k)
    a_bits = oracle.bf16_normal((1, k), seed=951)
    ws = torch.zeros(max(rt.workspace_bytes(1, n, k), 16384), dtype=torch.uint8, device="cuda")
    empty = torch.empty(0, dtype=torch.uint8, device="cuda")
    first = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=ws).cpu().numpy()
    second = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=ws).cpu().numpy()
    assert np.array_equal(first, second), "calls differ"
    assert int(ws[:16384].view(torch.int32).abs().sum().item()) == 0, "arrival counters left set"
    whole = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=empty).cpu().numpy()
    check_close(first, whole, bf16_out=False, tight=True, label=f"q5k split vs whole {n}x{k}")
    if k <= 2048:
        dense = oracle.q45k_decode(native).reshape(n, k)
        check_close(first, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                    absref=abs_gemm(a_bits, dense), label=f"q5k split {n}x{k}")
