"""Benchmark of the quantized-matmul hot path on one MI355X.

Default workload (the draft-verify step the metric is quoted on): M = 64
activation rows (8 sessions x 8 drafted tokens), 4-bit g64 affine weights, the fused gate+up
projection (two K=5120 -> N=17408 weights sharing one activation read, out = silu(g) * u) followed
by the down projection (K=17408 -> N=5120) on that output. One "step" is that pair of launches.

    python bench.py [--steps K] [--warmup W]
                    [--workload verify64|decode1|q5k1|q5k16|q5k64|q4k1|q4k64|q6k1|q80_1|iq4nl1|iq4xs1|q3k1|iq3s1|prefill2048|layerset|lmhead1|lmhead64|operand64|emit64|emit2048|stream50|stream715|gemm2048]

Inputs are synthetic (seeded, on the device): code words uniform random, scale = bf16(|N(0,0.02)|),
bias = bf16(N(0,0.01)), activations bf16(N(0,1)). Several copies of the weight set are rotated so
that the working set (>= 1.5 GB) is far larger than the 256 MB Infinity Cache and every step
streams its weights from HBM. `value` is algorithmic bytes per step / step time (TB/s, effective):
each operand counted once, weights N K / 2 + N (K / 64) * 4 bytes.

Prints ONE JSON line. --gpus N > 1 is refused: the path is measured on one GPU.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA

# HBM bytes per launch of the dominant kernel measured with rocprofv3 --pmc, keyed by (workload,
# call): FETCH_SIZE x 2 + WRITE_SIZE (KiB x 1024), the factors being what the two counters read for
# a plain 256 MiB device copy (FETCH_SIZE reads half the bytes moved, WRITE_SIZE all of them).
# The readings and commands are in profiles/; calls not listed are unmeasured (None).
MEASURED_TRAFFIC = {
    ("verify64", "mlp_in"): 55922.4 * 2 * 1024 + 9871.0 * 1024,  # mma_kernel<Q4Format<2, true, 2, 4, 3, false, false>, 2, 2, 4, 3>
    ("verify64", "down"): 35307.0 * 2 * 1024 + 4460.6 * 1024,  # mma_kernel<Q4Format<1, true, 2, 4, 3, false, false>, 2, 2, 4, 3>
    ("decode1", "gemv"): 24607.9 * 2 * 1024 + 75.0 * 1024,  # q4_decode_kernel<1, 1, 32, 3>
    ("lmhead1", "lm_head"): 349321.9 * 2 * 1024 + 526.2 * 1024,  # q4_decode_kernel<1, 1, 32, 2>
    ("q5k1", "q5k"): 30124.4 * 2 * 1024 + 30.0 * 1024,  # q5k_decode_kernel<8, 2, true>
    ("q5k64", "q5k"): 41299.7 * 2 * 1024 + 4303.0 * 1024,  # mma_kernel<Q5Format<2, 4, 3, true>, 2, 2, 4, 3>
    ("q5k16", "q5k"): 32869.4 * 2 * 1024 + 1050.0 * 1024,  # mma_kernel<Q5Format<2, 4, 3, true>, 1, 2, 4, 3>
    ("prefill2048", "prefill_up"): 264791.5 * 2 * 1024 + 114688.0 * 1024,  # prefill_kernel<Q4Stage>
    ("q5k2048", "q5k"): 347729.4 * 2 * 1024 + 98304.0 * 1024,  # prefill_kernel<Q5Stage<true>>
    ("q6k2048", "gguf"): 366940.1 * 2 * 1024 + 110080.0 * 1024,  # prefill_kernel<GgufStage<14>>
    ("q6k64", "gguf"): 47875.7 * 2 * 1024 + 4212.1 * 1024,  # mma_kernel<GgufFormat<14, 2, 4, 3>, 2, 2, 4, 3>
    ("iq3s64", "gguf"): 30858.2 * 2 * 1024 + 4174.7 * 1024,  # mma_kernel<GgufFormat<21, 2, 4, 3>, 2, 2, 4, 3>
    ("q6k64r", "gguf"): 47010.9 * 2 * 1024 + 4340.4 * 1024,  # the same, Q6_K in the ROWS32 order
    ("q80_64r", "gguf"): 57538.1 * 2 * 1024 + 4337.7 * 1024,  # mma_kernel<GgufFormat<8, 2, 4, 3>, 2, 2, 4, 3>, ROWS32
    ("q6k1", "gguf"): 36194.4 * 2 * 1024 + 10.0 * 1024,  # gguf_pairs_kernel<14, 4, 2, 0>
    ("q3k1", "gguf"): 19023.7 * 2 * 1024 + 10.0 * 1024,  # gguf_pairs_kernel<11, 4, 2, 0>
    ("iq3s1", "gguf"): 19064.2 * 2 * 1024 + 10.0 * 1024,  # gguf_pairs_kernel<21, 4, 2, 0>
    ("q80_1", "gguf"): 46754.4 * 2 * 1024 + 10.0 * 1024,  # gguf_pairs_kernel<8, 4, 2, 2>
    ("q80_4", "gguf"): 47196.6 * 2 * 1024 + 40.0 * 1024,  # gguf_pairs_kernel<8, 4, 2, 1>
    ("q6k4", "gguf"): 36625.1 * 2 * 1024 + 40.0 * 1024,  # gguf_pairs_kernel<14, 4, 2, 1>
    ("stream50", "read"): 24684.0 * 2 * 1024 + 64.0 * 1024,  # stream_read_kernel (shape 0, the default)
    ("layerset", "mlp_in"): 55918.2 * 2 * 1024 + 9871.0 * 1024,  # mma_kernel<Q4Format<2, true, 2, 4, 3, false, false>, 2, 2, 4, 3>
    ("lmhead64", "lm_head"): 358246.9 * 2 * 1024 + 39119.8 * 1024,  # mma_kernel<Q4Format<2, true, 2, 4, 3, false, false, true>, 2, 2, 4, 3> (the split pair)
    ("emit64", "fused"): 35993.7 * 2 * 1024 + 5883.2 * 1024,  # mma_kernel<Q4Format<1, true, 2, 4, 3, false, true>, 2, 2, 4, 3>
}


def q4_bytes(n, k):
    return n * k // 2 + n * (k // 64) * 4


def make_q4(rt, n, k, gen):
    import torch
    groups = k // 64
    packed = torch.randint(-2**31, 2**31, (n * groups * 8,), dtype=torch.int64, device="cuda",
                           generator=gen).to(torch.int32)
    scales = (torch.randn(n * groups, device="cuda", generator=gen) * 0.02).abs().to(torch.bfloat16).view(torch.int16)
    biases = (torch.randn(n * groups, device="cuda", generator=gen) * 0.01).to(torch.bfloat16).view(torch.int16)
    return rt.Q4Weight(packed, scales, biases, n, k, rt.TILED128)


def make_q5k(rt, n, k, gen, fifth=True):
    """Q5_K (or Q4_K) planes with every bit random except the fp16 d / dmin fields, drawn like the
    reference's kernel test (GgufKernelTests.swift:49-82): d ~ 1e-4 (2e-4 for Q4_K) (1 +- 0.25),
    dmin ~ 1.5e-3, 1 in 4 negative."""
    import torch
    blocks = n * (k // 256)
    native = torch.randint(0, 256, (blocks, 176 if fifth else 144), dtype=torch.uint8, device="cuda", generator=gen)
    for field, mag in ((0, 1e-4 if fifth else 2e-4), (2, 1.5e-3)):
        v = mag * (1 + 0.25 * (torch.rand(blocks, device="cuda", generator=gen) * 2 - 1))
        neg = torch.randint(0, 4, (blocks,), device="cuda", generator=gen) == 0
        v = torch.where(neg, -v, v).to(torch.float16).view(torch.uint8).view(blocks, 2)
        native[:, field:field + 2] = v
    w = rt.q5k_repack(native.view(-1), n, k) if fifth else rt.q4k_repack(native.view(-1), n, k)
    return w, native


def copies_for(bytes_per_set, minimum=1.5e9, cap=16):
    return max(2, min(cap, int(-(-minimum // bytes_per_set))))


class Timer:
    """HIP events on the stream the library launches on (torch's current stream)."""

    def __init__(self):
        import torch
        self.torch = torch

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        return e


def build_workload(name, rt, torch, gen, kernel):
    """Returns (steps: list of callables over copies, bytes_per_step, flops_per_step, kernels, config)."""
    def workspace(rows, n, k):
        need = rt.workspace_bytes(rows, n, k)
        return torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")  # zero-filled before first use

    if name == "prefill2048":
        # Config 2: both prefill shapes, K=5120 -> N=17408 (up) and K=17408 -> N=5120 (down).
        m = 2048
        shapes = (("prefill_up", 17408, 5120), ("prefill_down", 5120, 17408))
        mats, xs, outs, scratch = {}, {}, {}, {}
        for nm, n, k in shapes:
            ncopy = copies_for(q4_bytes(n, k), minimum=0.5e9)
            mats[nm] = [make_q4(rt, n, k, gen) for _ in range(ncopy)]
            xs[nm] = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
            outs[nm] = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
            scratch[nm] = workspace(m, n, k)

        def launches(i):
            calls = []
            for nm, _, _ in shapes:
                w = mats[nm][i % len(mats[nm])]
                calls.append((nm, lambda w=w, nm=nm: rt.gemm(w, xs[nm], out=outs[nm], kernel=kernel,
                                                             workspace=scratch[nm])))
            return calls

        kb = {nm: q4_bytes(n, k) + m * k * 2 + m * n * 2 for nm, n, k in shapes}
        kf = {nm: 2 * m * n * k for nm, n, k in shapes}
        cfg = {"workload": "prefill M=2048: K5120->N17408 and K17408->N5120", "rows": m,
               "format": "mlx affine q4 g64, tiled128", "weight_copies": {nm: len(v) for nm, v in mats.items()}}
        return launches, sum(kb.values()), sum(kf.values()), kb, cfg, kf
    if name == "verify64":
        m, h, inter = 64, 5120, 17408
        one = 2 * q4_bytes(inter, h) + q4_bytes(h, inter)
        ncopy = copies_for(one)
        sets = [(make_q4(rt, inter, h, gen), make_q4(rt, inter, h, gen), make_q4(rt, h, inter, gen))
                for _ in range(ncopy)]
        x = (torch.randn(m, h, device="cuda", generator=gen)).to(torch.bfloat16)
        ws_in, ws_down = workspace(m, inter, h), workspace(m, h, inter)
        act = torch.empty(m, inter, dtype=torch.bfloat16, device="cuda")
        out = torch.empty(m, h, dtype=torch.bfloat16, device="cuda")
        gate_up_bytes = 2 * q4_bytes(inter, h) + m * h * 2 + m * inter * 2
        down_bytes = q4_bytes(h, inter) + m * inter * 2 + m * h * 2

        def launches(i):
            g, u, d = sets[i % ncopy]
            return [("mlp_in", lambda: rt.mlp_in(g, u, x, out=act, kernel=kernel, workspace=ws_in)),
                    ("down", lambda: rt.gemm(d, act, out=out, kernel=kernel, workspace=ws_down))]

        cfg = {"workload": "draft-verify step: fused gate+up (2x K5120->N17408) + down (K17408->N5120)",
               "rows": m, "format": "mlx affine q4 g64, tiled128", "weight_copies": ncopy}
        return launches, gate_up_bytes + down_bytes, 2 * m * (2 * inter * h + h * inter), \
            {"mlp_in": gate_up_bytes, "down": down_bytes}, cfg, {"mlp_in": 4 * m * inter * h, "down": 2 * m * h * inter}
    if name == "decode1":
        m, k, n = 1, 5120, 17408
        ncopy = copies_for(q4_bytes(n, k))
        ws = [make_q4(rt, n, k, gen) for _ in range(ncopy)]
        x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        b = q4_bytes(n, k) + m * k * 2 + m * n * 2
        ws_dec = workspace(m, n, k)

        def launches(i):
            w = ws[i % ncopy]
            return [("gemv", lambda: rt.gemm(w, x, out=out, kernel=kernel, workspace=ws_dec))]

        cfg = {"workload": "decode GEMV K5120->N17408", "rows": 1, "format": "mlx affine q4 g64, tiled128",
               "weight_copies": ncopy}
        return launches, b, 2 * m * n * k, {"gemv": b}, cfg, {"gemv": 2 * m * n * k}
    if name == "layerset":
        # Config 4: every linear projection of one hybrid layer set at M=64 (shapes as BASELINE.json
        # states them): attention q, k, v, o; gated-delta input (qkv+z+b/a, 12288 outputs) and
        # output (6144 -> 5120); the MLP's fused gate+up and down. The attention layer's q, k and v
        # read one activation and go as one grouped launch (splosh_q4_gemm_group, the reference's
        # concurrent encoder); one step is six launches over the nine weights.
        m, h = 64, 5120
        shapes = [("attn_q", 5120, h), ("attn_k", 1024, h), ("attn_v", 1024, h), ("attn_o", 5120, h),
                  ("gdn_in", 12288, h), ("gdn_out", 5120, 6144), ("mlp_gate", 17408, h), ("mlp_up", 17408, h),
                  ("mlp_down", 5120, 17408)]
        one = sum(q4_bytes(n, k) for _, n, k in shapes)
        ncopy = copies_for(one)
        sets = [{nm: make_q4(rt, n, k, gen) for nm, n, k in shapes} for _ in range(ncopy)]
        xs = {k: torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16) for k in (h, 6144, 17408)}
        outs = {nm: torch.empty(m, n, dtype=torch.bfloat16, device="cuda") for nm, n, _ in shapes}
        scratch = {nm: workspace(m, n, k) for nm, n, k in shapes}
        scratch["attn_qkv"] = workspace(m, 7168, h)
        qkv = ("attn_q", "attn_k", "attn_v")
        calls = [(nm, n, k) for nm, n, k in shapes if nm not in ("mlp_gate", "mlp_up") + qkv]

        def launches(i):
            ws_ = sets[i % ncopy]
            out = [("attn_qkv", lambda: rt.gemm_group([ws_[nm] for nm in qkv], xs[h], outs=[outs[nm] for nm in qkv],
                                                      kernel=kernel, workspace=scratch["attn_qkv"]))]
            out += [(nm, lambda nm=nm, k=k: rt.gemm(ws_[nm], xs[k], out=outs[nm], kernel=kernel, workspace=scratch[nm]))
                    for nm, n, k in calls]
            out.append(("mlp_in", lambda: rt.mlp_in(ws_["mlp_gate"], ws_["mlp_up"], xs[h], out=outs["mlp_gate"],
                                                    kernel=kernel, workspace=scratch["mlp_gate"])))
            return out

        kb = {nm: q4_bytes(n, k) + m * k * 2 + m * n * 2 for nm, n, k in calls}
        kb["attn_qkv"] = q4_bytes(7168, h) + m * h * 2 + m * 7168 * 2
        kb["mlp_in"] = 2 * q4_bytes(17408, h) + m * h * 2 + m * 17408 * 2
        kf = {nm: 2 * m * n * k for nm, n, k in calls}
        kf["attn_qkv"] = 2 * m * 7168 * h
        kf["mlp_in"] = 4 * m * 17408 * h
        cfg = {"workload": "layer set at M=64: attention q/k/v (grouped) and o, gated-delta in/out, MLP gate+up and down",
               "rows": m, "format": "mlx affine q4 g64, tiled128", "weight_copies": ncopy}
        return launches, sum(kb.values()), sum(kf.values()), kb, cfg, kf
    if name.startswith("stream"):
        # The practical ceiling of one launch: a plain streaming read of as many bytes as the named
        # decode weight (stream50: config 0's 50,180,096 bytes; stream715: the lm_head's), rotated
        # over copies. Not part of the path: the probes live in libsplosh_probe.so, built beside the
        # product library and loaded only here. SPLOSH_PROBE_SHAPE picks the probe: 0 = contiguous
        # slices on SPLOSH_PROBE_GRID workgroups of 256 (default 2048, the best of 256..4096), 1 / 2 =
        # persistent workgroups of 1024 (default two a CU) with 8 / 16 loads in flight a thread,
        # 3 = a device-to-device copy of the buffer (hipMemcpyAsync through torch; reads and writes).
        import ctypes
        from splosh_amd import _lib
        lib = ctypes.CDLL(str(Path(_lib.PKG) / "libsplosh_probe.so"))
        lib.splosh_probe_stream_read.restype = ctypes.c_int
        lib.splosh_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_void_p]
        b = {"stream50": q4_bytes(17408, 5120), "stream715": q4_bytes(248320, 5120)}[name]
        ncopy = copies_for(b)
        bufs = [torch.randint(0, 255, (b,), dtype=torch.uint8, device="cuda", generator=gen) for _ in range(ncopy)]
        shape = int(os.environ.get("SPLOSH_PROBE_SHAPE", "0"))
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        grid = int(os.environ.get("SPLOSH_PROBE_GRID", "2048" if shape == 0 else str(2 * cus)))
        sink = torch.zeros(16 * grid, dtype=torch.int32, device="cuda")
        dst = torch.empty(b, dtype=torch.uint8, device="cuda") if shape == 3 else None

        def launches(i):
            buf = bufs[i % ncopy]
            if shape == 3:
                return [("read", lambda: dst.copy_(buf))]
            return [("read", lambda: _lib.check(lib.splosh_probe_stream_read(
                buf.data_ptr(), b, sink.data_ptr(), grid, shape, torch.cuda.current_stream().cuda_stream)))]

        cfg = {"workload": f"streaming read of {b} bytes a launch (probe {shape}, grid {grid}, not the path)",
               "rows": 0, "format": "bytes", "weight_copies": ncopy}
        return launches, b, 0, {"read": b}, cfg, {"read": 0}
    if name == "gemm2048":
        # The practical ceiling of the matrix cores on config 2's two shapes: the vendor bf16 GEMM
        # (torch.matmul, hipBLASLt) with the weights already dequantized to bf16 row-major. Not part
        # of the path: a reference point for prefill2048, which also dequantizes q4.
        m = 2048
        shapes = (("gemm_up", 17408, 5120), ("gemm_down", 5120, 17408))
        wb = {nm: torch.randn(n, k, device="cuda", generator=gen).to(torch.bfloat16) for nm, n, k in shapes}
        xs = {nm: torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16) for nm, n, k in shapes}
        outs = {nm: torch.empty(m, n, dtype=torch.bfloat16, device="cuda") for nm, n, k in shapes}

        def launches(i):
            return [(nm, lambda nm=nm: torch.matmul(xs[nm], wb[nm].t(), out=outs[nm])) for nm, _, _ in shapes]

        kb = {nm: 2 * n * k + m * k * 2 + m * n * 2 for nm, n, k in shapes}
        kf = {nm: 2 * m * n * k for nm, n, k in shapes}
        cfg = {"workload": "bf16 GEMM (torch.matmul) on the prefill shapes (reference point, not the path)",
               "rows": m, "format": "bf16", "weight_copies": 1}
        return launches, sum(kb.values()), sum(kf.values()), kb, cfg, kf
    if name.startswith("emit"):
        # The MLP's down projection at M rows (emit64, emit2048) as the residual projection that
        # feeds the next RMSNorm: fp32 hidden state += a w^T, and the next GEMM's operand (bf16
        # h * norm weight, per-64 sums and sums of squares). "fused": the emit in the GEMM's
        # epilogue (splosh_q4_gemm_emit); "separate": the GEMM, then the operand pass over the
        # hidden state.
        m, h, inter = int(name[4:] or 64), 5120, 17408
        ncopy = copies_for(q4_bytes(h, inter))
        ws = [make_q4(rt, h, inter, gen) for _ in range(ncopy)]
        x = torch.randn(m, inter, device="cuda", generator=gen).to(torch.bfloat16)
        hid = torch.randn(m, h, device="cuda", generator=gen)
        wn = (1 + 0.1 * torch.randn(h, device="cuda", generator=gen)).to(torch.bfloat16)
        scr = workspace(m, h, inter)
        be = torch.empty(m, h, dtype=torch.bfloat16, device="cuda")
        se = torch.empty(m, h // 64, device="cuda")
        qe = torch.empty_like(se)
        b = q4_bytes(h, inter) + m * inter * 2 + 2 * m * h * 4 + m * h * 2 + 2 * m * (h // 64) * 4

        def launches(i):
            w = ws[i % ncopy]
            # At most 64 rows the fused epilogue is the M <= 64 kernel's, asked for by name (AUTO takes
            # the separate pass there); above that AUTO's prefill or tile kernel.
            fk = rt.DEQUANT if m <= 64 else rt.AUTO
            return [("fused", lambda: rt.gemm_emit(w, x, wn, out=hid, residual=hid, kernel=fk, workspace=scr)),
                    ("separate", lambda: (rt.gemm(w, x, out=hid, residual=hid, out_dtype=torch.float32, workspace=scr),
                                          rt.emit_operand(hid, wn, values=be, sums=se, squares=qe)))]

        cfg = {"workload": f"down projection K17408->N5120 at M={m} with the next norm's operand emitted", "rows": m,
               "format": "mlx affine q4 g64, tiled128", "weight_copies": ncopy}
        return launches, 2 * b, 4 * m * h * inter, {"fused": b, "separate": b}, cfg, \
            {"fused": 2 * m * h * inter, "separate": 2 * m * h * inter}
    if name.startswith("operand"):
        # The operand producers around the draft-verify MLP at M rows (default 64): the input
        # operand (fp32 -> bf16 + sums, 5120), the down projection's operand (silu(g) u, 17408) and
        # the emitted next-norm operand of the hidden state (5120). HBM bound.
        m = int(name[7:] or 64)
        h, inter = 5120, 17408
        x = torch.randn(m, h, device="cuda", generator=gen)
        g = torch.randn(m, inter, device="cuda", generator=gen)
        u = torch.randn(m, inter, device="cuda", generator=gen)
        wn = (1 + 0.1 * torch.randn(h, device="cuda", generator=gen)).to(torch.bfloat16)
        bx, sx = torch.empty(m, h, dtype=torch.bfloat16, device="cuda"), torch.empty(m, h // 64, device="cuda")
        bd, sd = torch.empty(m, inter, dtype=torch.bfloat16, device="cuda"), torch.empty(m, inter // 64, device="cuda")
        be, se, qe = torch.empty_like(bx), torch.empty_like(sx), torch.empty_like(sx)

        def launches(i):
            return [("prepare", lambda: rt.prepare_operand(x, out=bx, sums=sx)),
                    ("silu_mul", lambda: rt.silu_mul_operand(g, u, out=bd, sums=sd)),
                    ("emit", lambda: rt.emit_operand(x, wn, values=be, sums=se, squares=qe))]

        kb = {"prepare": m * h * 6 + m * (h // 64) * 4, "silu_mul": m * inter * 10 + m * (inter // 64) * 4,
              "emit": m * h * 6 + h * 2 + 2 * m * (h // 64) * 4}
        cfg = {"workload": f"operand producers at M={m}: prepare (5120), silu*mul (17408), emit (5120)", "rows": m,
               "format": "fp32 in, bf16 operand + per-64 sums out"}
        return launches, sum(kb.values()), 0, kb, cfg, {k: 0 for k in kb}
    if name.startswith("lmhead"):
        # Config 4's lm_head, 5120 -> 248320, at M=1 or M=64.
        m, k, n = int(name[6:]), 5120, 248320
        ncopy = copies_for(q4_bytes(n, k))
        ws = [make_q4(rt, n, k, gen) for _ in range(ncopy)]
        x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        ws_lm = workspace(m, n, k)
        b = q4_bytes(n, k) + m * k * 2 + m * n * 2

        def launches(i):
            w = ws[i % ncopy]
            return [("lm_head", lambda: rt.gemm(w, x, out=out, kernel=kernel, workspace=ws_lm))]

        cfg = {"workload": f"lm_head K5120->N248320 at M={m}", "rows": m, "format": "mlx affine q4 g64, tiled128",
               "weight_copies": ncopy}
        return launches, b, 2 * m * n * k, {"lm_head": b}, cfg, {"lm_head": 2 * m * n * k}
    if name.startswith("q5k") or name.startswith("q4k"):
        # Config 3's shape (down projection K=17408 -> N=5120) in GGUF Q5_K, or Q4_K (the same
        # blocks without fifth bits: 144 bytes).
        fifth = name.startswith("q5k")
        m = int(name[3:] or 64)
        k, n = 17408, 5120
        one = n * (k // 256) * (176 if fifth else 144)
        ncopy = copies_for(one)
        ws = [make_q5k(rt, n, k, gen, fifth)[0] for _ in range(ncopy)]
        x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        b = one + m * k * 2 + m * n * 2
        ws_q5 = workspace(m, n, k)

        def launches(i):
            w = ws[i % ncopy]
            return [("q5k", lambda: rt.gemm(w, x, out=out, kernel=kernel, workspace=ws_q5))]

        cfg = {"workload": f"{'Q5_K' if fifth else 'Q4_K'} down K17408->N5120", "rows": m,
               "format": f"gguf {'q5_k' if fifth else 'q4_k'} planes",
               "weight_copies": ncopy}
        return launches, b, 2 * m * n * k, {"q5k": b}, cfg, {"q5k": 2 * m * n * k}
    native_types = {"q80_": (8, "Q8_0"), "q6k": (14, "Q6_K"), "iq4nl": (20, "IQ4_NL"), "iq4xs": (23, "IQ4_XS"),
                    "q3k": (11, "Q3_K"), "iq3s": (21, "IQ3_S")}
    for prefix, (gtype, label) in native_types.items():
        if not name.startswith(prefix):
            continue
        # Config 3's shape (K=17408 -> N=5120) with the weight in the native blocks of another GGUF
        # format (random bytes, fp16 scale fields of about 1e-3); a trailing "r": in the ROWS32
        # order (splosh_gguf_repack_rows32).
        rows32 = name.endswith("r")
        m = int(name[len(prefix):len(name) - (1 if rows32 else 0)] or 1)
        k, n = 17408, 5120
        elems, size = rt.GGUF_NATIVE[gtype]
        one = n * (k // elems) * size
        ncopy = copies_for(one)
        at = {14: 208, 11: 108}.get(gtype, 0)
        ws = []
        for _ in range(ncopy):
            blocks = n * (k // elems)
            native = torch.randint(0, 256, (blocks, size), dtype=torch.uint8, device="cuda", generator=gen)
            d = (1e-3 * (1 + 0.25 * (torch.rand(blocks, device="cuda", generator=gen) * 2 - 1))).to(torch.float16)
            native[:, at:at + 2] = d.view(torch.uint8).view(blocks, 2)
            w = rt.GgufWeight(native.view(-1), gtype, n, k)
            ws.append(rt.gguf_repack_rows32(w) if rows32 else w)
            del native
        x = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)
        out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        b = one + m * k * 2 + m * n * 2
        ws_g = workspace(m, n, k)

        def launches(i):
            w = ws[i % ncopy]
            return [("gguf", lambda: rt.gemm(w, x, out=out, workspace=ws_g))]

        order = "ROWS32 order" if rows32 else "native blocks"
        cfg = {"workload": f"{label} K17408->N5120 ({order})", "rows": m, "format": f"gguf {label.lower()}",
               "weight_copies": ncopy}
        return launches, b, 2 * m * n * k, {"gguf": b}, cfg, {"gguf": 2 * m * n * k}
    raise SystemExit(f"unknown workload {name}")


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(workload, step_bytes, step_flops, seconds=3.0):
    """The CPU oracle (oracle/: dequantize each weight row to fp32, sequential fp32 dot per
    activation row -- DequantOracle.dequantize + the fp32 GEMM loop) timed on a bounded sample of
    output columns of the same workload, on one core and on every core of the host, and
    extrapolated to the whole step. The rate counts the same bytes (or flops) as the GPU's."""
    import numpy as np
    import oracle
    nproc = os.cpu_count() or 1
    if workload == "verify64":
        mats = [(17408, 5120), (17408, 5120), (5120, 17408)]
        m = 64
    elif workload == "decode1":
        mats = [(17408, 5120)]
        m = 1
    elif workload == "prefill2048":
        mats = [(17408, 5120), (5120, 17408)]
        m = 2048
    else:
        return None

    def step_seconds(threads):
        # A seeded sample weight per shape; a column's cost does not depend on its values. The
        # sample grows until it has run for `seconds` or covers every column.
        frac = 1 / 256 if m <= 64 else 1 / 8192
        while True:
            t_total, elapsed = 0.0, 0.0
            for idx, (n, k) in enumerate(mats):
                cols = max(threads, int(n * frac))
                words, stride, sc, bi = oracle.q4_random_weight(cols, k, seed=idx)
                a = oracle.bf16_normal((m, k), seed=99)
                t0 = time.perf_counter()
                oracle.q4_gemm_rowmajor(a, words, stride, sc, bi, cols, k, threads=threads)
                dt = time.perf_counter() - t0
                t_total += dt * n / cols
                elapsed += dt
            if elapsed >= seconds or frac >= 1.0:
                return t_total, frac
            frac = min(1.0, frac * max(2.0, seconds / max(elapsed, 1e-3)))

    t1, f1 = step_seconds(1)
    tn, fn = step_seconds(nproc)
    work, unit = (step_flops, "TFLOP/s") if workload == "prefill2048" else (step_bytes, "TB/s")
    v1, vn = work / t1 / 1e12, work / tn / 1e12
    return {"value": vn, "unit": unit, "cores": nproc, "kind": "port",
            "sample": f"{fn * 100:.2f}% (all cores) and {f1 * 100:.2f}% (one core) of each weight's output "
                      f"columns at M={m}, extrapolated to the full step; same work count as the GPU line",
            "single_core": v1, "all_cores": vn, "nproc": nproc, "cpu_model": _cpu_model(),
            "step_seconds": {"single_core": t1, "all_cores": tn}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="verify64")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch from the host every step (no HIP graph)")
    ap.add_argument("--kernel", default="AUTO", choices=["AUTO", "STREAM", "DEQUANT", "TILE", "SCALAR", "PREFILL"])
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB ten times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "launches": 10}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the path; --gpus {args.gpus} is not supported "
              "(the multi-GPU design shards the weights along N: every GPU streams N / G columns of each "
              "projection and the outputs are gathered)", file=sys.stderr)
        sys.exit(2)

    import torch
    from splosh_amd import runtime as rt

    gen = torch.Generator(device="cuda").manual_seed(0x5EED0001)
    launches, step_bytes, step_flops, kernel_bytes, cfg, kernel_flops = build_workload(args.workload, rt, torch, gen,
                                                                               getattr(rt, args.kernel))
    timer = Timer()
    names = [nm for nm, _ in launches(0)]
    torch.cuda.synchronize()
    for i in range(args.warmup):
        for _, fn in launches(i):
            fn()
    torch.cuda.synchronize()

    if args.eager:
        # Host-launched: includes the Python/ctypes call overhead between launches.
        events = []
        start = timer.event()
        for i in range(args.steps):
            evs = [timer.event()]
            for _, fn in launches(args.warmup + i):
                fn()
                evs.append(timer.event())
            events.append(evs)
        end = timer.event()
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(end)
        per_kernel = {nm: sum(evs[j].elapsed_time(evs[j + 1]) for evs in events) / args.steps
                      for j, nm in enumerate(names)}
    else:
        # The K steps are captured once into a HIP graph (as a serving loop replays a layer) and the
        # timed region is one replay of it: GPU time without host launch gaps. Each kernel's own
        # time comes from a graph of its K launches alone, replayed the same way.
        def capture(kinds):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(args.steps):
                    for nm, fn in launches(args.warmup + i):
                        if nm in kinds:
                            fn()
            return g

        def replay_ms(kinds):
            # Two captures of the same K steps: the warm one and the timed one are enqueued back to
            # back with no host sync between them, so the timed graph is submitted while the GPU
            # still runs the warm one (a second launch of the same graph would wait on the host for
            # the first to finish, and its submission would land in the timed region), and the start
            # event is reached only when the GPU is done with the warm steps: the timed region holds
            # the K steps' GPU time, whatever K is.
            # The warm replays also cover about 30 ms, so that the timed steps run at the clock the
            # part settles at under this load, not during its ramp after the idle capture.
            g_warm, g_timed = capture(kinds), capture(kinds)
            torch.cuda.synchronize()
            t0 = timer.event()
            g_warm.replay()
            t1 = timer.event()
            torch.cuda.synchronize()
            reps = max(1, min(1000, int(30.0 / max(t0.elapsed_time(t1), 1e-3)) + 1))
            for _ in range(reps):
                g_warm.replay()
            start = timer.event()
            g_timed.replay()
            end = timer.event()
            torch.cuda.synchronize()
            return start.elapsed_time(end)

        total_ms = replay_ms(set(names))
        per_kernel = {nm: replay_ms({nm}) / args.steps for nm in names}
    ms_per_step = total_ms / args.steps

    dominant = max(per_kernel, key=per_kernel.get)
    dom_ms = per_kernel[dominant]
    # Prefill-sized workloads (512 rows or more) are bound by the matrix cores, the others by HBM.
    compute_bound = cfg.get("rows", 0) >= 512 and kernel_flops.get(dominant, 0) > 0
    traffic = MEASURED_TRAFFIC.get((args.workload, dominant))
    traffic = int(traffic) if traffic is not None else None
    if compute_bound:
        achieved = kernel_flops[dominant] / (dom_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                    "traffic": traffic, "kernel": dominant,
                    "kernel_us": round(dom_ms * 1e3, 2), "algorithmic_flops": kernel_flops[dominant]}
        value, unit = step_flops / (ms_per_step * 1e-3) / 1e12, "TFLOP/s"
    else:
        achieved = kernel_bytes[dominant] / (dom_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": traffic,
                    "kernel": dominant, "kernel_us": round(dom_ms * 1e3, 2),
                    "algorithmic_bytes": kernel_bytes[dominant]}
        value, unit = step_bytes / (ms_per_step * 1e-3) / 1e12, "TB/s"
    cpu = None if args.no_cpu else cpu_baseline(args.workload, step_bytes, step_flops)
    result = {
        "metric": "quant GEMM effective HBM TB/s at M=1/64; TFLOP/s at M=2048 prefill",
        "value": round(value, 4), "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x q4 -> fp32 acc, bf16 out", "data": "synthetic (seeded, on device)",
        "config": cfg,
        "kernels_us": {k: round(v * 1e3, 2) for k, v in per_kernel.items()},
        "tflops": round(step_flops / (ms_per_step * 1e-3) / 1e12, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "launch": "eager" if args.eager else "hip graph of the K steps, one replay timed",
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
