"""Shared helpers of the GPU parity tests: seeded inputs on the device, and the tolerance checks."""
import numpy as np
import torch

import oracle
from splosh_amd import runtime as rt


def abs_gemm(a_bits, dense):
    """sum_k |a[m][k]| |w[n][k]| in fp64: the scale of the weight-rounding error of an output."""
    return np.abs(oracle.bf16_to_f32(a_bits).astype(np.float64)) @ np.abs(dense.astype(np.float64)).T


def dev_u32(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).cuda()


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def dev_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def bf16_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def to_f32(t):
    return t.float().cpu().numpy()


class Q4Case:
    """A seeded q4 weight, row-major on the host plus both device layouts."""

    def __init__(self, n, k, seed):
        self.n, self.k = n, k
        self.words, self.stride, self.scales, self.biases = oracle.q4_random_weight(n, k, seed)
        self.w_rm = rt.Q4Weight(dev_u32(self.words), dev_u16(self.scales), dev_u16(self.biases), n, k,
                                rt.ROW_MAJOR, self.stride)
        self.dense = oracle.q4_dequant_rowmajor(self.words, self.stride, self.scales, self.biases, n, k)
        self._tiled = None

    @property
    def w_tiled(self):
        if self._tiled is None:
            g = self.k // 64
            tw = oracle.tile128(self.words[:, : self.k // 8].reshape(-1).view(np.uint8), self.n, g, 32).view(np.uint32)
            ts = oracle.tile128(self.scales.reshape(-1).view(np.uint8), self.n, g, 2).view(np.uint16)
            tb = oracle.tile128(self.biases.reshape(-1).view(np.uint8), self.n, g, 2).view(np.uint16)
            self._tiled = rt.Q4Weight(dev_u32(tw), dev_u16(ts), dev_u16(tb), self.n, self.k, rt.TILED128)
        return self._tiled


def check_close(got, ref, *, bf16_out, tight=False, absref=None, label=""):
    """The path's tolerance: max |err| / max |ref| <= 1e-2 and cosine >=
    0.9999 against the fp32-accumulate reference, plus the reference tests' sum-normalised relErr
    <= 1e-2 (GemmOracleTests.swift:155-158).

    `tight` adds a per-element bound: one bf16 rounding of the output (2^-8 relative, bf16 out)
    plus 1e-5 (bf16) or 2e-5 (fp32) of the largest output, plus -- when `absref` = sum_k |a||w| is
    given -- 2^-8 of it, which covers kernels that round the dequantized weight to bf16 (at most
    2^-9 relative per weight) with room for fp32 summation order."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    diff = np.abs(got - ref)
    scale = max(np.abs(ref).max(), 1e-6)
    max_rel = diff.max() / scale
    rel_sum = diff.sum() / max(np.abs(ref).sum(), 1e-6)
    cos = (got * ref).sum() / max(np.sqrt((got * got).sum() * (ref * ref).sum()), 1e-30)
    assert max_rel <= 1e-2, f"{label}: max rel err {max_rel}"
    assert rel_sum <= 1e-2, f"{label}: relErr {rel_sum}"
    assert cos >= 0.9999, f"{label}: cosine {cos}"
    if tight:
        if bf16_out:
            bound = np.abs(ref) * 2.0 ** -8 + 1e-5 * scale
        else:
            bound = np.full(ref.shape, 2e-5 * scale)
        if absref is not None:
            bound = bound + np.asarray(absref, np.float64) * 2.0 ** -8
        worst = (diff - bound).max()
        assert worst <= 0, f"{label}: beyond the tight bound by {worst} (max rel {max_rel})"
    return max_rel, cos


def rows32_order(native, gguf_type, rows, inner):
    """The ROWS32 order of a native-block weight (numpy, host): the 256-element units of 32
    consecutive rows interleaved, unit u of row n at ((n // 32) * units * 32 + u * 32 + n % 32) unit
    bytes, rows padded with zeros to a multiple of 32."""
    elems, size = oracle.GGUF_BLOCK[gguf_type]
    ub, units = 256 // elems * size, inner // 256
    r32 = (rows + 31) // 32 * 32
    x = np.zeros((r32, units, ub), np.uint8)
    x[:rows] = np.asarray(native, np.uint8).reshape(rows, units, ub)
    return x.reshape(r32 // 32, 32, units, ub).transpose(0, 2, 1, 3).reshape(-1).copy()
