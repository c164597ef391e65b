"""The kernels under HIP graph capture: a captured verify step (fused gate+up, then down, with the
stream-K partial workspace) and a decode GEMV are replayed several times, with unrelated eager work
and synchronisations between replays, and every replay must equal the eager result bit for bit
(the kernels are deterministic). Nothing in these paths records a memset into the graph."""
import numpy as np
import pytest
import torch

import oracle
from qcheck import Q4Case, bf16_tensor

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from splosh_amd import runtime
    return runtime


def test_graph_replays_match_eager(rt):
    rows, h, inter = 64, 512, 1024
    gate, up, down = Q4Case(inter, h, seed=60), Q4Case(inter, h, seed=61), Q4Case(h, inter, seed=62)
    x = bf16_tensor(oracle.bf16_normal((rows, h), seed=63))
    x1 = bf16_tensor(oracle.bf16_normal((1, h), seed=64))
    act = torch.empty(rows, inter, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(rows, h, dtype=torch.bfloat16, device="cuda")
    out1 = torch.empty(1, inter, dtype=torch.bfloat16, device="cuda")
    ws_in = torch.zeros(max(rt.workspace_bytes(rows, inter, h), 1), dtype=torch.uint8, device="cuda")
    ws_down = torch.zeros(max(rt.workspace_bytes(rows, h, inter), 1), dtype=torch.uint8, device="cuda")

    def step():
        rt.mlp_in(gate.w_tiled, up.w_tiled, x, out=act, workspace=ws_in)
        rt.gemm(down.w_tiled, act, out=out, workspace=ws_down)
        rt.gemm(gate.w_tiled, x1, out=out1)

    step()  # eager, also initialises the launchers
    torch.cuda.synchronize()
    ref = (act.clone(), out.clone(), out1.clone())

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for k in range(4):
        act.zero_()
        out.fill_(float("nan"))
        out1.zero_()
        junk = torch.randn(1 << 20, device="cuda").sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, want in zip((act, out, out1), ref):
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {k} differs"
        del junk


def test_prefill_graph_replays_match_eager(rt):
    """The prefill kernel and its stream-K finish pass under capture: q4 (single weight and fused
    gate+up) and Q5_K planes at 300 rows, replayed with eager work between replays."""
    rows, h, inter = 300, 512, 1024
    gate, up = Q4Case(inter, h, seed=70), Q4Case(inter, h, seed=71)
    native = oracle.q45k_random_native(h, inter, seed=72)
    wq5 = rt.q5k_repack(torch.from_numpy(native).cuda(), h, inter)
    x = bf16_tensor(oracle.bf16_normal((rows, h), seed=73))
    xi = bf16_tensor(oracle.bf16_normal((rows, inter), seed=74))
    act = torch.empty(rows, inter, dtype=torch.bfloat16, device="cuda")
    g1 = torch.empty(rows, inter, dtype=torch.float32, device="cuda")
    o5 = torch.empty(rows, h, dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(max(rt.workspace_bytes(rows, inter, h), rt.workspace_bytes(rows, h, inter)), dtype=torch.uint8,
                     device="cuda")

    def step():
        rt.mlp_in(gate.w_tiled, up.w_tiled, x, out=act, workspace=ws)
        rt.gemm(gate.w_tiled, x, out=g1, workspace=ws)
        rt.gemm(wq5, xi, out=o5, workspace=ws)

    step()
    torch.cuda.synchronize()
    ref = (act.clone(), g1.clone(), o5.clone())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for k in range(4):
        act.zero_()
        g1.fill_(float("nan"))
        o5.zero_()
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, want in zip((act, g1, o5), ref):
            assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got.view(torch.int32),
                               want.view(torch.int16) if want.dtype == torch.bfloat16 else want.view(torch.int32)), \
                f"replay {k} differs"
        del junk
