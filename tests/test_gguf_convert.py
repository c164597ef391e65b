"""GgufConvert's treatment of a Qwen GGUF file (GgufConvert.swift, GgufNames.swift): the value-head
order of the gated-delta layers, the float -> Q8_0 requantisation, and the dense tensors. The
product (splosh_amd/gguf.py, numpy) is checked against the C oracle, and the oracle against
closed forms, known answers of the reference's own description and numpy's binary16 rounding."""
import numpy as np

import oracle
from splosh_amd import gguf


def test_mlx_value_head_known_answers():
    """GgufNames.swift:92-104: file head i is the engine's 3 (i % 16) + i / 16 of 48."""
    known = {0: 0, 1: 3, 2: 6, 15: 45, 16: 1, 17: 4, 31: 46, 32: 2, 33: 5, 47: 47}
    for i, want in known.items():
        assert oracle.mlx_value_head(i) == want
        assert gguf.mlx_value_head(i) == want
    heads = [oracle.mlx_value_head(i) for i in range(48)]
    assert sorted(heads) == list(range(48))  # a permutation
    assert heads == [gguf.mlx_value_head(i) for i in range(48)]


def test_head_destination():
    """HeadOrder.destination (GgufConvert.swift:62-69): units before `first` and past the heads stay;
    unit u of head h moves to head mlxValueHead(h) at the same offset."""
    qkv = gguf.WEIGHT_HEAD_ORDER["attn_qkv.weight"]
    assert (qkv.first, qkv.span) == (4096, 128)
    for u in (0, 100, 4095):
        assert qkv.destination(u) == u == oracle.head_destination(u, 4096, 128)
    # file head 17, offset 5 -> engine head 4
    assert qkv.destination(4096 + 17 * 128 + 5) == 4096 + 4 * 128 + 5 == oracle.head_destination(4096 + 17 * 128 + 5, 4096, 128)
    assert qkv.destination(10240) == 10240  # past the 48 heads
    dest = [qkv.destination(u) for u in range(10240)]
    assert sorted(dest) == list(range(10240))
    alpha = gguf.WEIGHT_HEAD_ORDER["ssm_alpha.weight"]
    assert [alpha.destination(i) for i in range(48)] == [oracle.mlx_value_head(i) for i in range(48)]


def test_order_rows_matches_oracle():
    rng = np.random.default_rng(5)
    for tail, rows, row_bytes in (("attn_qkv.weight", 10240, 8), ("attn_gate.weight", 6144, 4),
                                  ("ssm_beta.weight", 48, 34)):
        order = gguf.WEIGHT_HEAD_ORDER[tail]
        native = rng.integers(0, 256, rows * row_bytes, dtype=np.uint8)
        stored = -(-rows // 128) * 128
        got = gguf.order_rows(native, rows, row_bytes, order, stored_rows=stored)
        want = oracle.order_rows(native, rows, row_bytes, order.first, order.span, stored=stored)
        assert np.array_equal(got, want), tail
        assert not got[rows * row_bytes:].any()
        # rows of a head land whole: file row r is at its destination
        r = rows - 1
        d = order.destination(r)
        assert np.array_equal(got[d * row_bytes:(d + 1) * row_bytes], native[r * row_bytes:(r + 1) * row_bytes])
    plain = rng.integers(0, 256, 200 * 6, dtype=np.uint8)
    assert np.array_equal(gguf.order_rows(plain, 200, 6, None, stored_rows=256)[:1200], plain)


def test_f16_rounding_pinned_by_numpy():
    """The oracle's fp32 -> fp16 (Swift's Float16(Float), RNE) against numpy's on normals,
    subnormals, ties, overflow and zeros."""
    rng = np.random.default_rng(6)
    v = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.98023259e-08, 1e-12, 1.00048828125, 1.0009765625 + 2 ** -12], np.float32)])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16_rne(v), want)


def test_q8_0_closed_forms():
    """GgufConvert.q8_0Blocks: largest 127 -> scale 1 (fp16 0x3C00) and codes the values rounded half
    away from zero; a zero block -> scale 0, codes 0; largest 254 -> scale 2."""
    v = np.zeros(96, np.float32)
    v[:32] = np.arange(32, dtype=np.float32) * 4 - 64.5  # -64.5 .. 59.5: halves
    v[31] = 127.0
    v[64:96] = np.linspace(-254, 254, 32, dtype=np.float32)
    for blocks in (oracle.q8_0_blocks(v), gguf.q8_0_blocks(v)):
        b = blocks.reshape(3, 34)
        assert b[0, :2].view(np.uint16)[0] == 0x3C00
        codes = b[0, 2:].view(np.int8).astype(np.int64)
        x = v[:32].astype(np.float64)
        assert np.array_equal(codes, np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5)))
        assert codes[0] == -65 and codes[1] == -61  # -64.5 -> -65, -60.5 -> -61 (away from zero)
        assert not b[1].any()
        assert b[2, :2].view(np.float16)[0] == np.float16(2.0)
        assert b[2, 2:].view(np.int8)[0] == -127 and b[2, 2:].view(np.int8)[31] == 127


def test_q8_0_product_matches_oracle_and_decodes():
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(32 * 500) * rng.choice([1e-4, 1e-2, 1.0, 30.0], 32 * 500)).astype(np.float32)
    got = gguf.q8_0_blocks(v)
    assert np.array_equal(got, oracle.q8_0_blocks(v))
    # the reference decoder (golden-pinned) gives the values back to within half a code step, plus
    # the scale's fp16 rounding
    back = oracle.gguf_decode(8, got)
    step = np.abs(v.reshape(-1, 32)).max(axis=1) / 127
    err = np.abs(back - v).reshape(-1, 32).max(axis=1)
    assert (err <= step * (0.5 + 127 * 2 ** -11) + 1e-30).all()


def test_dense_bf16():
    """GgufConvert.ggufDense: RNE to bf16, the decay back to A_log, units to their engine place."""
    rng = np.random.default_rng(8)
    # A_log: the file holds -exp(A_log)
    a_log = rng.uniform(-2, 2, 48).astype(np.float32)
    unit, order, neg = gguf.DENSE_HEAD_ORDER["ssm_a"]
    got = gguf.dense_bf16(-np.exp(a_log).astype(np.float32), unit, order, neg)
    back = oracle.bf16_to_f32(got)
    want = np.empty(48, np.float32)
    want[[oracle.mlx_value_head(i) for i in range(48)]] = a_log
    assert np.abs(back - want).max() <= 2 ** -7 * np.abs(want).max()
    # the convolution: channels of 4 taps, the value channels (from 4096) by head
    conv = rng.standard_normal(10240 * 4).astype(np.float32)
    unit, order, neg = gguf.DENSE_HEAD_ORDER["ssm_conv1d.weight"]
    got = gguf.dense_bf16(conv, unit, order, neg)
    bits = oracle.f32_to_bf16_rne(conv)
    want = oracle.order_rows(bits.view(np.uint8), 10240, 8, order.first, order.span).view(np.uint16)
    assert np.array_equal(got, want)
    # the RNE tie case rounds to even
    assert gguf.bf16_rne(np.array([1.0 + 2 ** -8], np.float32))[0] == 0x3F80
    assert gguf.bf16_rne(np.array([1.0 + 3 * 2 ** -8], np.float32))[0] == 0x3F82


def test_head_gather_oracle():
    """The activations a head-ordered weight meets: column k of the result is engine column
    mlxValueHead(k / 128) 128 + k % 128."""
    a = np.arange(2 * 6144, dtype=np.uint16).reshape(2, 6144)
    g = oracle.head_gather(a)
    for k in (0, 127, 128, 17 * 128 + 9, 6143):
        col = oracle.mlx_value_head(k // 128) * 128 + k % 128
        assert g[1, k] == a[1, col]
    assert sorted(g[0].tolist()) == a[0].tolist()
