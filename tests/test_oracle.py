"""The CPU oracle pinned against the reference's own known answers and against mathematics.

Each check is chosen so that a plausible slip in the restatement (a dropped term, a wrong shift,
a swapped operand) fails it: closed forms from the reference's tests, the real GGUF golden
blocks, fp64 brute force, and structural invariants.
"""
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "gguf_golden_blocks.json"


def f32(x):
    return np.float32(x)


# ---- bf16 helpers (Q4BufferLayout.swift:123-129) ---------------------------------------------

def test_bf16_roundings(oracle):
    assert oracle.f32_to_bf16_halfup(1.0) == 0x3F80
    # 1 + 2^-8 is exactly half an ulp of bf16: half-up goes away from zero, RNE to even.
    half = np.float32(1.0 + 2.0 ** -8)
    assert oracle.f32_to_bf16_halfup(half) == 0x3F81
    assert int(oracle.f32_to_bf16_rne(np.array([half]))[0]) == 0x3F80
    assert int(oracle.f32_to_bf16_rne(np.array([np.float32(1.0 + 3 * 2.0 ** -8)]))[0]) == 0x3F82
    assert oracle.bf16_to_f32(np.array([0xC000], np.uint16))[0] == -2.0


# ---- MLX affine q4 --------------------------------------------------------------------------

def _bf16(x):
    import oracle
    return oracle.f32_to_bf16_halfup(x)


def test_mlx_affine_group64_closed_form(oracle):
    """QuantDequantOracleTests.swift:31-48: a 65-column row, scales [2, 3], biases [-1, 10]."""
    columns = 65
    words = np.zeros(32, np.uint32)  # 128-byte padded row
    for c in range(columns):
        words[c // 8] |= np.uint32((c % 16) << ((c % 8) * 4))
    scales = np.array([_bf16(2), _bf16(3)], np.uint16)
    biases = np.array([_bf16(-1), _bf16(10)], np.uint16)
    got = oracle.q4_dequant_rowmajor(words, 32, scales, biases, 1, columns)[0]
    expected = np.array([(2 if c < 64 else 3) * (c % 16) + (-1 if c < 64 else 10) for c in range(columns)],
                        np.float32)
    assert np.array_equal(got, expected)


def test_q4_buffer_layout_padded_rows(oracle):
    """Q4BufferLayoutTests.swift:7-27: K=65 -> 9 words, stride 128 B (23 padding words);
    decode(0,0)=0, decode(0,64)=-1, decode(1,64)=2."""
    rows, K = 2, 65
    stride = 32
    words = np.zeros(rows * stride, np.uint32)
    for r in range(rows):
        for k in range(K):
            words[r * stride + k // 8] |= np.uint32(((k + r) & 15) << (4 * (k % 8)))
    sidecars = rows * 2
    scales = np.array([_bf16(2 + i) for i in range(sidecars)], np.uint16)
    biases = np.array([_bf16(-i) for i in range(sidecars)], np.uint16)
    w = oracle.q4_dequant_rowmajor(words, stride, scales, biases, rows, K)
    assert w[0, 0] == 0 and w[0, 64] == -1 and w[1, 64] == 2
    from splosh_amd.quant import Q4BufferLayout
    layout = Q4BufferLayout(rows=2, logical_k=65)
    assert (layout.packed_words_per_row, layout.row_stride_bytes, layout.padding_words_per_row) == (9, 128, 23)


def test_tile_roundtrip_and_addressing(oracle):
    rows, groups, eb = 256, 3, 32
    src = np.arange(rows * groups * eb, dtype=np.uint32).astype(np.uint8)
    t = oracle.tile128(src, rows, groups, eb)
    assert np.array_equal(oracle.untile128(t, rows, groups, eb), src)
    # Record (row 130, group 2) lands at ((1 * groups + 2) * 128 + 2) (Retile.swift:142-147).
    row, g = 130, 2
    dst_rec = (1 * groups + 2) * 128 + 2
    assert np.array_equal(t[dst_rec * eb:(dst_rec + 1) * eb], src[(row * groups + g) * eb:(row * groups + g + 1) * eb])


def test_tiled_dequant_matches_rowmajor(oracle):
    N, K = 256, 192
    words, stride, scales, biases = oracle.q4_random_weight(N, K, seed=7)
    ref = oracle.q4_dequant_rowmajor(words, stride, scales, biases, N, K)
    groups = K // 64
    tw = oracle.tile128(words[:, :K // 8].reshape(-1).view(np.uint8), N, groups, 32).view(np.uint32)
    ts = oracle.tile128(scales.reshape(-1).view(np.uint8), N, groups, 2).view(np.uint16)
    tb = oracle.tile128(biases.reshape(-1).view(np.uint8), N, groups, 2).view(np.uint16)
    assert np.array_equal(oracle.q4_dequant_tiled(tw, ts, tb, N, K), ref)


def test_dequant_against_float64(oracle):
    """s*q is exact in fp32 (8-bit mantissa times a 4-bit integer), so s*q+b rounded once equals
    the fp64 value rounded to fp32."""
    N, K = 64, 320
    words, stride, scales, biases = oracle.q4_random_weight(N, K, seed=11)
    got = oracle.q4_dequant_rowmajor(words, stride, scales, biases, N, K)
    k = np.arange(K)
    q = (words[:, k // 8] >> (4 * (k % 8)).astype(np.uint32)) & 15
    s = oracle.bf16_to_f32(scales).astype(np.float64)[:, k // 64]
    b = oracle.bf16_to_f32(biases).astype(np.float64)[:, k // 64]
    assert np.array_equal(got, (s * q + b).astype(np.float32))


# ---- GEMM -----------------------------------------------------------------------------------

def test_gemm_bf16_known_answer(oracle):
    """GemmOracleTests.swift:27-28,76-84: [-8, -4.5, 7, 39]."""
    a = np.array([0x3f80, 0xc000, 0x4040, 0x3e80, 0x4120, 0xbf00], np.uint16)
    b = np.array([0x4000, 0xbf80, 0x3f00, 0x4080, 0xc040, 0x3fc0], np.uint16)
    assert oracle.gemm_bf16(a, b, 2, 2, 3).reshape(-1).tolist() == [-8.0, -4.5, 7.0, 39.0]


def named_q4_case(oracle, rows, columns, inner):
    """The inputs of GemmOracleTests.swift:165-191 (codes (n + 3k) & 15, scales 0.25 + 0.125 i,
    biases -0.5 + 0.25 i, A ((i % 11) - 5) * 0.125)."""
    stride = ((inner + 7) // 8 * 4 + 127) // 128 * 32
    groups = (inner + 63) // 64
    words = np.zeros(columns * stride, np.uint32)
    for n in range(columns):
        for k in range(inner):
            words[n * stride + k // 8] |= np.uint32(((n + 3 * k) & 15) << (4 * (k % 8)))
    sc = np.array([_bf16(0.25 + i * 0.125) for i in range(columns * groups)], np.uint16)
    bi = np.array([_bf16(-0.5 + i * 0.25) for i in range(columns * groups)], np.uint16)
    a = np.array([_bf16(((i % 11) - 5) * 0.125) for i in range(rows * inner)], np.uint16).reshape(rows, inner)
    return words, stride, sc, bi, a


@pytest.mark.parametrize("rows,columns,inner", [(2, 3, 65), (3, 2, 128), (1, 1, 64)])
def test_named_q4_cases_against_float64(oracle, rows, columns, inner):
    words, stride, sc, bi, a = named_q4_case(oracle, rows, columns, inner)
    w = oracle.q4_dequant_rowmajor(words, stride, sc, bi, columns, inner)
    got = oracle.gemm_a_bf16_w_f32(a, w)
    exact = oracle.bf16_to_f32(a).astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(got, exact, rtol=1e-6, atol=1e-6)
    fused = oracle.q4_gemm_rowmajor(a, words, stride, sc, bi, columns, inner)
    assert np.array_equal(fused, got)


def test_per_group_identity(oracle):
    """sum_k a (s q + b) = s sum(a q) + b sum(a) per 64-group (MlpFusedTests.swift:200-212)."""
    M, N, K = 3, 8, 256
    words, stride, sc, bi = oracle.q4_random_weight(N, K, seed=3)
    a = oracle.bf16_normal((M, K), seed=4)
    got = oracle.gemm_a_bf16_w_f32(a, oracle.q4_dequant_rowmajor(words, stride, sc, bi, N, K)).astype(np.float64)
    k = np.arange(K)
    q = ((words[:, k // 8] >> (4 * (k % 8)).astype(np.uint32)) & 15).astype(np.float64)
    af = oracle.bf16_to_f32(a).astype(np.float64)
    s = oracle.bf16_to_f32(sc).astype(np.float64)
    b = oracle.bf16_to_f32(bi).astype(np.float64)
    ident = np.zeros((M, N))
    for g in range(K // 64):
        sl = slice(64 * g, 64 * g + 64)
        ident += s[:, g] * (af[:, sl] @ q[:, sl].T) + b[:, g] * af[:, sl].sum(1, keepdims=True)
    assert np.allclose(got, ident, rtol=1e-5, atol=1e-4)


def test_silu_mul(oracle):
    g = np.array([-3.0, -0.5, 0.0, 0.5, 2.0, 20.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -1.0, 0.25, 1.0], np.float32)
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.allclose(oracle.silu_mul(g, u), ref, rtol=2e-7, atol=0)


# ---- GGUF -----------------------------------------------------------------------------------

@pytest.mark.parametrize("name,fifth", [("q5K", True), ("q4K", False)])
def test_gguf_golden_blocks(oracle, name, fifth):
    """GgufTests.swift:237-247 over GgufGoldenBlocks (real blocks of Qwen3.8-27B): bit-exact."""
    block = json.loads(GOLDEN.read_text())[name]
    expected = np.array([np.float32(v) for v in block["values"]], np.float32)
    got = oracle.q45k_decode(np.array(block["bytes"], np.uint8), fifth_bit=fifth)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("name,gguf_type", [("q6K", 14), ("q8_0", 8), ("iq4NL", 20), ("iq4XS", 23), ("q3K", 11),
                                             ("iq3S", 21)])
def test_gguf_golden_blocks_other_formats(oracle, name, gguf_type):
    """The other formats' golden blocks (GgufGoldenBlocks.swift, GgufTests.swift:237-247): the
    oracle's decode is bit-exact against the values the reference holds for each real block."""
    block = json.loads(GOLDEN.read_text())[name]
    expected = np.array([np.float32(v) for v in block["values"]], np.float32)
    got = oracle.gguf_decode(gguf_type, np.array(block["bytes"], np.uint8))
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def _f16(x):
    return list(np.array([x], np.float16).view(np.uint8))


def test_gguf_closed_forms(oracle):
    """Blocks whose values follow from the format alone: a dropped sign, a swapped nibble order or a
    wrong bit position each changes one of them."""
    # Q8_0: d = 0.5, codes -128..127 (bytes 0x80.. wrap): value = code / 2.
    codes = np.arange(-16, 16, dtype=np.int8)
    v = oracle.gguf_decode(8, np.array(_f16(0.5) + list(codes.view(np.uint8)), np.uint8))
    assert np.array_equal(v, codes.astype(np.float32) * 0.5)
    # IQ4_NL: d = 1, byte e = (15 - e) << 4 | e: element e is table[e], element 16 + e table[15 - e].
    table = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    qs = [((15 - e) << 4) | e for e in range(16)]
    v = oracle.gguf_decode(20, np.array(_f16(1.0) + qs, np.uint8))
    assert np.array_equal(v[:16], table) and np.array_equal(v[16:], table[::-1])
    # Q6_K: d = 1, scales 1, ql = 0x21 (low codes 1 / 2), qh = 0b11100100 (high bits 0, 1, 2, 3 for
    # quarters 0..3): group j has code (low | high << 4) - 32 with low = 1 for quarters 0, 1 and 2 for
    # quarters 2, 3, i.e. -31, -15, 2, 18 in both halves.
    block = [0x21] * 128 + [0b11100100] * 64 + [1] * 16 + _f16(1.0)
    v = oracle.gguf_decode(14, np.array(block, np.uint8)).reshape(8, 32)
    assert np.array_equal(v[:, 0], np.array([-31, -15, 2, 18] * 2, np.float32))
    assert np.all(v == v[:, :1])
    # Q6_K scale sign and per-16 split: scale bytes 2j = -1, 2j + 1 = 3.
    block = [0x21] * 128 + [0] * 64 + [0xFF, 3] * 8 + _f16(1.0)
    v = oracle.gguf_decode(14, np.array(block, np.uint8)).reshape(8, 32)
    assert np.all(v[0, :16] == 31) and np.all(v[0, 16:] == -93)
    # IQ4_XS: d = 2, group j's scale 32 + j (low nibbles j, high bits 2 = 0b10 << 2j), codes 8
    # (table value 1): group j is 2 j everywhere.
    high = sum(2 << (2 * j) for j in range(8))
    low = [(j | ((j + 1) << 4)) for j in range(0, 8, 2)]
    block = _f16(2.0) + [high & 0xFF, high >> 8] + low + [0x88] * 128
    v = oracle.gguf_decode(23, np.array(block, np.uint8)).reshape(8, 32)
    assert np.array_equal(v[:, 0], 2.0 * np.arange(8, dtype=np.float32)) and np.all(v == v[:, :1])


def test_iq3s_grid_matches_the_reference_table(oracle):
    """The oracle's IQ3_S codebook equals the 512 entries read from the reference's file."""
    want = np.array(json.loads((GOLDEN.parent / "iq3s_grid.json").read_text())["grid"], np.uint32)
    assert np.array_equal(oracle.iq3s_grid(), want)


def test_q3k_closed_forms(oracle):
    """Q3_K blocks whose values follow from the layout (GgufQuant.swift:232-256): d = 1; scale k
    built from its low nibble (byte k % 4 of word (k / 4) % 2, nibble k / 8) and its top two bits
    (bits 2 (k / 4) of byte 104 + k % 4), applied less 32 to 16 elements; group j's code takes bits
    2 (j % 4) of byte 32 + 32 (j / 4) + e and bit j of byte e, less 4."""
    b = np.zeros(110, np.uint8)
    b[108:110] = _f16(1.0)
    # Every scale = 33 (low nibble 1, top bits 2 = 0b10): byte k%4 of words 0, 1 hold nibbles
    # 1 | 1 << 4; bytes 104..107 hold 0b10 at every 2-bit field.
    b[96:104] = 0x11
    b[104:108] = 0b10101010
    v = oracle.gguf_decode(11, b).reshape(8, 32)
    assert np.all(v == (33 - 32) * (0 - 4))  # all codes 0 - 4
    # Group 5 (half 1, shift 2): low bits 3 at element 7; high bit (bit 5 of byte 7) set -> code
    # 3 | 4 = 7 - 4 = 3.
    b[32 + 32 + 7] = 0b11 << 2
    b[7] = 1 << 5
    v = oracle.gguf_decode(11, b).reshape(8, 32)
    assert v[5, 7] == 3.0 and v[5, 6] == -4.0 and v[1, 7] == -4.0
    # Scale 11 (word 2: high nibble of byte 3 of word 0; top bits at bits 4..5 of byte 107) = 0:
    # group 5's elements 16..31 get scale 1 | 0 << 4 ... set the nibble to 5 and top bits to 1.
    b[96 + 3] = (5 << 4) | 1
    b[104 + 3] = (int(b[104 + 3]) & 0xCF) | (1 << 4)
    v = oracle.gguf_decode(11, b).reshape(8, 32)
    assert np.all(v[5, 16:] == ((5 | 16) - 32) * -4.0) and np.all(v[5, 8:16] == 1 * -4.0)


def test_iq3s_closed_forms(oracle):
    """IQ3_S blocks whose values follow from the layout (GgufQuant.swift:277-300): d = 0.5, scale
    nibble s weighs group j by d (1 + 2 s); grid entry (code byte 8 j + k, ninth bit k of byte 66 + j)
    gives the magnitudes of elements 4 k .. 4 k + 3; sign bit e of bytes 74 + 4 j .. negates."""
    grid = oracle.iq3s_grid()
    b = np.zeros(110, np.uint8)
    b[0:2] = _f16(0.5)
    b[106:110] = [0x21, 0x43, 0x65, 0x87]         # scales 1, 2, ..., 8 for groups 0..7
    b[2:66] = np.arange(64, dtype=np.uint8) * 3   # code bytes
    b[66:74] = [0, 0xFF, 0x0F, 0xF0, 0x55, 0xAA, 0x01, 0x80]  # ninth bits
    b[74:106] = np.arange(32, dtype=np.uint8) * 37  # sign bytes
    v = oracle.gguf_decode(21, b).reshape(8, 32)
    for j in range(8):
        weight = 0.5 * (1 + 2 * (j + 1))
        for e in range(32):
            k, t = e // 4, e % 4
            code = int(b[2 + 8 * j + k]) | (((int(b[66 + j]) >> k) & 1) << 8)
            mag = (int(grid[code]) >> (8 * t)) & 0xFF
            neg = (int(b[74 + 4 * j + e // 8]) >> (e % 8)) & 1
            assert v[j, e] == np.float32(weight * mag * (1 - 2 * neg)), (j, e)


def test_q4k_group_layout_contract(oracle):
    """The inputs of QuantDequantOracleTests.swift:17-29 (d = 1, dmin = 0, 6-bit scales 1 for
    groups 0..3, code bytes 0x10) decoded with GgufQuant's layout (group 2h = low nibbles of run h,
    2h+1 = high nibbles): groups 0 and 2 are 0, 1 and 3 are 1, 4..7 have scale 0.
    DequantOracle.q4_K reads elements 16..31 from the other nibble; llama.cpp and GgufQuant do not."""
    block = np.array([0x00, 0x3c, 0x00, 0x00] + [1] * 8 + [0] * 4 + [0x10] * 128, np.uint8)
    v = oracle.q45k_decode(block, fifth_bit=False)
    assert v[0] == 0 and v[1] == 0 and v[32] == 1
    expected = np.repeat(np.array([0, 1, 0, 1, 0, 0, 0, 0], np.float32), 32)
    assert np.array_equal(v, expected)


def test_q5k_fifth_bit_and_high_scales(oracle):
    """Hand-built Q5_K block: d = 1, dmin = 0.5 (fp16 0x3800). Group 5 takes scale
    (packed[9] & 15) | (packed[1] >> 6) << 4 and min (packed[9] >> 4) | (packed[5] >> 6) << 4
    (GgufQuant.swift:200-202); element 3 of group 5 has its fifth bit set."""
    b = np.zeros(176, np.uint8)
    b[0:2] = [0x00, 0x3c]
    b[2:4] = [0x00, 0x38]
    b[4 + 1] = 0b10_000000   # top bits of scale 5 = 2 -> scale 5 = 2 << 4 | low
    b[4 + 5] = 0b01_000000   # top bits of min 5 = 1
    b[4 + 9] = 0x3_5         # low nibble 5 of scale 5, high nibble 3 of min 5
    b[16 + 3] = 1 << 5       # fifth bit of element 3 of group 5
    b[48 + 32 * 2 + 3] = 0x70  # group 5 = high nibble of run 2: code 7
    v = oracle.q45k_decode(b, fifth_bit=True)
    scale = (2 << 4) | 5
    minimum = (1 << 4) | 3
    assert v[32 * 5 + 3] == np.float32((7 + 16) * scale - 0.5 * minimum)
    assert v[32 * 5 + 0] == np.float32(-0.5 * minimum)


def test_gguf_slot_matches_chunk_order(oracle):
    """gguf_formats.h:17-21: chunk c holds elements 4c..4c+3 and 16+4c..16+4c+3 as four pairs,
    pair p's first element e0 = 16 (p >> 1) + 4c + 2 (p & 1), element e at slot 8c + 2p + (e & 1)."""
    expected = {}
    for c in range(4):
        for p in range(4):
            e0 = 16 * (p >> 1) + 4 * c + 2 * (p & 1)
            for e in (e0, e0 + 1):
                expected[e] = 8 * c + 2 * p + (e & 1)
    assert sorted(expected) == list(range(32))
    assert [oracle.gguf_slot(e) for e in range(32)] == [expected[e] for e in range(32)]


def test_q5k_planes_roundtrip_and_bit_positions(oracle):
    N, K = 128, 512
    native = oracle.q45k_random_native(N, K, seed=5)
    p0, p1, meta = oracle.q45k_repack(native, N, K)
    assert (p0.size, p1.size, meta.size) == oracle.q45k_plane_sizes(N, K)
    assert p0.size + p1.size + meta.size == native.size
    assert np.array_equal(oracle.q45k_unpack(p0, p1, meta, N, K), native)
    # A single set code bit: element 5 of group 1 of row 3 (high nibble of run 0, code 0xF).
    nat = np.zeros_like(native)
    nat[3 * (K // 256) * 176 + 48 + 5] = 0xF0
    q0, q1, qm = oracle.q45k_repack(nat, N, K)
    # slot(5) = 9: word 1, pair index 1 -> bits 16..19; record (row 3, group 1) = 1 * 128 + 3.
    rec = (0 * (K // 32) + 1) * 128 + 3
    word = q0[rec * 16 + 4: rec * 16 + 8].view(np.uint32)[0]
    assert word == 0xF << 16
    assert np.count_nonzero(q0) == 1 and np.count_nonzero(q1) == 0


def test_q5k_splitmix_generator_matches_reference_shape(oracle):
    nat = oracle.q45k_random_native_splitmix(128, 256, seed=0x6600 + 13)
    d = nat.reshape(-1, 176)[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    assert np.all((np.abs(d) >= 0.75e-4 * 0.999) & (np.abs(d) <= 1.25e-4 * 1.001))
    vals = oracle.q45k_decode(nat)
    assert np.all(np.isfinite(vals))


@pytest.mark.parametrize("fifth", [True, False])
def test_q45k_fused_gemm_equals_decode_then_gemm(oracle, fifth):
    """The fused Q4_K/Q5_K GEMM (decode a block row on the fly) against the composition of the two
    separately pinned steps: golden-pinned block decode, then the fp32 sequential-k GEMM. Both sum
    in the same k order, so the results are bit-identical; a wrong block or column index would not be."""
    n, k, rows = 6, 512, 3
    nat = oracle.q45k_random_native_splitmix(n, k, seed=0x6600 + (1 if fifth else 2))
    if not fifth:  # a Q4_K block is the Q5_K block without the 32-byte fifth-bit plane
        nat = np.concatenate([b[:16].tolist() + b[48:].tolist() for b in nat.reshape(-1, 176)]).astype(np.uint8)
    dense = oracle.q45k_decode(nat, fifth_bit=fifth).reshape(n, k)
    a = oracle.bf16_normal((rows, k), seed=5)
    want = oracle.gemm_a_bf16_w_f32(a, dense)
    got = oracle.q45k_gemm_native(a, nat, n, k, fifth_bit=fifth)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    part = oracle.q45k_gemm_native(a, nat, n, k, fifth_bit=fifth, n0=2, n1=5)
    assert np.array_equal(part[:, 2:5], want[:, 2:5]) and np.all(np.isnan(part[:, :2]))


# ---- operand producers (engine_na.metal:38-56, engine.metal:200-233, engine_na.metal:365-411) ----


def _rne_f64(v):
    """Round-to-nearest-even to bf16 of float32 values, via float64 bit arithmetic (independent of
    the oracle's C conversion)."""
    b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_prepare_operand_closed_forms(oracle):
    # A group of equal values sums to 64 x the value; ties round to even.
    x = np.full((2, 128), 1.5, np.float32)
    x[1, :64] = 1.0 + 2.0 ** -8            # tie between 1.0 and 1.0078125: even is 1.0
    x[1, 64:] = 1.0 + 3 * 2.0 ** -8        # tie between 1.0078125 and 1.015625: even is 1.015625
    out, sums = oracle.prepare_operand(x)
    assert np.all(out[0] == 0x3FC0) and np.all(sums[0] == 96.0)
    assert np.all(out[1, :64] == 0x3F80) and sums[1, 0] == 64.0
    assert np.all(out[1, 64:] == 0x3F82) and sums[1, 1] == 64 * 1.015625


def test_prepare_operand_brute_force(oracle):
    x = (np.random.default_rng(1).normal(size=(5, 320)) * 3).astype(np.float32)
    out, sums = oracle.prepare_operand(x)
    assert np.array_equal(out, _rne_f64(x))
    vals = (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(5, 5, 64)
    np.testing.assert_allclose(sums, vals.sum(-1), rtol=1e-6, atol=1e-6)


def test_silu_mul_operand(oracle):
    rng = np.random.default_rng(2)
    g = (rng.normal(size=(3, 192)) * 4).astype(np.float32)
    u = rng.normal(size=(3, 192)).astype(np.float32)
    out, sums = oracle.silu_mul_operand(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    got = (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    # Within one bf16 rounding of the exact product, and equal to its rounding almost everywhere.
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)
    assert np.mean(out == _rne_f64(ref.astype(np.float32))) > 0.99
    np.testing.assert_allclose(sums, got.reshape(3, 3, 64).sum(-1), rtol=1e-6, atol=1e-6)
    # silu(0) = 0; a power-of-two row scale equals scaling the inputs (exact in fp32).
    z, _ = oracle.silu_mul_operand(np.zeros((1, 64), np.float32), np.ones((1, 64), np.float32))
    assert np.all(z == 0)
    s = np.array([0.5, 2.0, 4.0], np.float32)
    a, sa = oracle.silu_mul_operand(g, u, s)
    b, sb = oracle.silu_mul_operand(g * s[:, None], u * s[:, None])
    assert np.array_equal(a, b) and np.array_equal(sa, sb)


def test_emit_operand_and_row_inv(oracle):
    rng = np.random.default_rng(3)
    h = rng.normal(size=(4, 256)).astype(np.float32)
    w = _rne_f64(rng.normal(1.0, 0.1, size=256).astype(np.float32))
    values, sums, squares = oracle.emit_operand(h, w)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(values, _rne_f64(h * wf))   # one fp32 product, then RNE
    got = (values.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    np.testing.assert_allclose(sums, got.reshape(4, 4, 64).sum(-1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(squares, (h.astype(np.float64) ** 2).reshape(4, 4, 64).sum(-1), rtol=1e-6)
    # RMSNorm's row scale: constant mean square c gives 1 / sqrt(c + eps) exactly for c = 4, eps = 0.
    sq = np.full((2, 8), 64 * 4.0, np.float32)
    assert np.all(oracle.row_inv(sq, 512, 0.0) == 0.5)
    inv = oracle.row_inv(squares, 256, 1e-6)
    np.testing.assert_allclose(inv, 1 / np.sqrt((h.astype(np.float64) ** 2).mean(-1) + 1e-6), rtol=1e-6)
