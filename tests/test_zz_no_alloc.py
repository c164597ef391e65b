"""splosh_q4_gemm_noalloc (the entry point that allocates nothing) against splosh_q4_gemm with a
zero-filled caller workspace: the same kernels and plan, so the same bits. Two calls in a row,
the second on a smaller input, both through the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from qcheck import Q4Case, bf16_tensor, check_close

pytestmark = pytest.mark.gpu


def _noalloc(lib, w, a, out, residual=None):
    wc = w.c()
    return lib.splosh_q4_gemm_noalloc(ctypes.byref(wc), ctypes.c_void_p(a.data_ptr()), a.stride(0),
                                      ctypes.c_void_p(out.data_ptr()), out.stride(0), 0,
                                      ctypes.c_void_p(residual.data_ptr()) if residual is not None else None,
                                      a.shape[0], 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_workspace_entry_point():
    from splosh_amd import _lib
    from splosh_amd import runtime as rt
    lib = _lib.lib()
    # First: 64 rows on a shape whose bands split K over the workgroups (stream-K partials in the
    # scratch); second: 8 rows on a smaller weight.
    for rows, n, k, seed in ((64, 640, 4352, 1), (8, 384, 1280, 2)):
        case = Q4Case(n, k, seed=seed)
        a_bits = oracle.bf16_normal((rows, k), seed=seed + 10)
        a = bf16_tensor(a_bits)
        need = rt.workspace_bytes(rows, n, k)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
        want = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, workspace=ws)
        got = torch.full((rows, n), float("nan"), device="cuda")
        st = _noalloc(lib, case.w_tiled, a, got)
        assert st == 0, lib.splosh_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows={rows}: differs from splosh_q4_gemm"
        check_close(got.cpu().numpy(), oracle.gemm_a_bf16_w_f32(a_bits, case.dense), bf16_out=False,
                    label=f"noalloc rows={rows}")
        # Residual in place, as Engine.gemm's residual projections call it.
        res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=3).astype(np.float32)).cuda()
        out = res.clone()
        assert _noalloc(lib, case.w_tiled, a, out, residual=out) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, want + res)


# The scratch the entry point plans against: 16 KiB of counters and 8 MiB of partials.
SCRATCH_BYTES = 16384 + (8 << 20)


@pytest.mark.parametrize("rows,n,k", [(100, 1024, 4352), (300, 640, 2048), (1, 17408, 1024), (2, 16896, 512)])
def test_noalloc_planned_against_scratch(rows, n, k):
    """Every kernel plans against the scratch's size: at 100 rows two calls of the M <= 64 kernel
    (64 + 36 rows, one after the other on the scratch), at 300 the prefill kernel, whose partials
    fit it or run unsplit; at one or two rows
    the decode kernel, whose last round of row blocks is split over K in the scratch (544 and 528
    blocks on 256 CUs). The same call through splosh_q4_gemm with a zero-filled workspace of that
    size gives the same bits; both against the oracle. Run twice, so that the second call sees the
    scratch the first left."""
    from splosh_amd import _lib
    from splosh_amd import runtime as rt
    lib = _lib.lib()
    case = Q4Case(n, k, seed=rows)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 1)
    a = bf16_tensor(a_bits)
    ws = torch.zeros(SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    want = rt.gemm(case.w_tiled, a, out_dtype=torch.float32, workspace=ws)
    check_close(want.cpu().numpy(), oracle.gemm_a_bf16_w_f32(a_bits, case.dense), bf16_out=False,
                label=f"workspace rows={rows}")
    for _ in range(2):
        got = torch.full((rows, n), float("nan"), device="cuda")
        st = _noalloc(lib, case.w_tiled, a, got)
        assert st == 0, lib.splosh_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows={rows}: differs from splosh_q4_gemm"


def test_noalloc_rejects_bad_arguments():
    from splosh_amd import _lib
    lib = _lib.lib()
    case = Q4Case(384, 1280, seed=5)
    a = bf16_tensor(oracle.bf16_normal((4, 1280), seed=6))
    out = torch.empty((4, 384), device="cuda")
    wc = case.w_tiled.c()
    st = lib.splosh_q4_gemm_noalloc(ctypes.byref(wc), None, a.stride(0), ctypes.c_void_p(out.data_ptr()),
                                    out.stride(0), 0, None, 4, 0, None)
    assert st == 12  # nullPointer
