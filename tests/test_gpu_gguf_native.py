"""GGUF Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S and IQ4_XS in native blocks on the GPU against the oracle: the dequant
is bit-exact (the reference's golden blocks included), the GEMM within one bf16 rounding of the
fp32-accumulate reference for every pass count of activation rows, the residual and both output
types, config-0 sizes through sampled columns, and weights read out of a GGUF file."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from qcheck import abs_gemm, bf16_tensor, check_close, to_f32
from splosh_amd import gguf

pytestmark = pytest.mark.gpu
TYPES = {"q8_0": 8, "q6K": 14, "iq4NL": 20, "iq4XS": 23, "q3K": 11, "iq3S": 21}
GOLDEN = Path(__file__).resolve().parent / "golden" / "gguf_golden_blocks.json"


@pytest.fixture(scope="module")
def rt():
    from splosh_amd import runtime
    return runtime


def _weight(rt, t, n, k, seed):
    native = oracle.gguf_random_native(t, n, k, seed)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, n, k)
    return w, oracle.gguf_decode(t, native).reshape(n, k)


@pytest.mark.parametrize("name", list(TYPES))
def test_golden_block_on_device(rt, name):
    block = json.loads(GOLDEN.read_text())[name]
    t = TYPES[name]
    k = len(block["values"])
    w = rt.GgufWeight(torch.tensor(block["bytes"], dtype=torch.uint8).cuda(), t, 1, k)
    expected = np.array([np.float32(v) for v in block["values"]], np.float32)
    assert np.array_equal(rt.dequant(w).cpu().numpy().reshape(-1).view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [1, 3, 4, 9, 65, 200])
def test_native_gemm(rt, name, rows):
    t = TYPES[name]
    n, k = 200, 1536
    w, dense = _weight(rt, t, n, k, seed=rows + t)
    assert np.array_equal(rt.dequant(w).cpu().numpy().view(np.uint32), dense.view(np.uint32))
    a_bits = oracle.bf16_normal((rows, k), seed=rows)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    a = bf16_tensor(a_bits)
    got = rt.gemm(w, a, out_dtype=torch.float32)
    check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=absref, label=f"{name} f32 rows={rows}")
    got = rt.gemm(w, a)
    check_close(to_f32(got), ref, bf16_out=True, tight=True, absref=absref, label=f"{name} bf16 rows={rows}")
    res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=5).astype(np.float32)).cuda()
    got = rt.gemm(w, a, out=res.clone(), out_dtype=torch.float32, residual=res)
    check_close(got.cpu().numpy(), ref + res.cpu().numpy(), bf16_out=False, label=f"{name} residual rows={rows}")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [2, 5, 6, 7, 8])
@pytest.mark.parametrize("n,k", [(200, 1536), (203, 4352)])
def test_two_to_eight_rows_auto(rt, name, rows, n, k):
    """2-8 activation rows through AUTO, with and without a workspace, against the oracle: the
    streaming kernel up to the format's limit (four rows a pass, activations staged in LDS for a
    workgroup's four waves), the stream-K MFMA kernel above it. 203 weight rows leave streaming
    waves past the last row, which still stage their share and meet the barriers, and a partial
    MFMA band; K4352 gives three streaming rounds of 64 groups, the last partial."""
    t = TYPES[name]
    w, dense = _weight(rt, t, n, k, seed=rows + 3 * t + n)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 11)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    a = bf16_tensor(a_bits)
    for ws in (None, torch.empty(0, dtype=torch.uint8, device="cuda")):
        got = rt.gemm(w, a, out_dtype=torch.float32, workspace=ws)
        check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=absref,
                    label=f"{name} rows={rows} n={n} k={k} workspace={'none' if ws is not None else 'fresh'}")


@pytest.mark.parametrize("name,rows", [("q8_0", 5), ("q8_0", 8), ("iq4NL", 4), ("iq4NL", 7), ("q3K", 5), ("q3K", 6)])
def test_streaming_eight_rows(rt, name, rows):
    """The streaming kernel's eight-row pass: Q8_0 and IQ4_NL with K % 256 != 0 (the MFMA kernel
    takes 256 elements a step, so AUTO streams up to eight rows), Q3_K up to its limit of six."""
    t = TYPES[name]
    n, k = 203, 1568 if name != "q3K" else 4352
    w, dense = _weight(rt, t, n, k, seed=rows + 5 * t)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 13)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32)
    check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, dense),
                label=f"{name} streaming rows={rows} k={k}")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [9, 33, 64])
def test_mma_kernel(rt, name, rows):
    """The stream-K MFMA kernel over native blocks (AUTO above the streaming limit, up to 64 rows):
    a partial band (N = 203), 17 steps of K, split over workgroups (workspace) and whole bands (an
    empty one), bf16 and fp32 out, the residual; against the oracle."""
    t = TYPES[name]
    n, k = 203, 4352
    w, dense = _weight(rt, t, n, k, seed=rows + 17 * t)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 19)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    a = bf16_tensor(a_bits)
    for ws in (None, torch.empty(0, dtype=torch.uint8, device="cuda")):
        split = ws is None
        got = rt.gemm(w, a, out_dtype=torch.float32, workspace=ws)
        check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=absref,
                    label=f"{name} mma rows={rows} split={split}")
        got = rt.gemm(w, a, workspace=ws)
        check_close(to_f32(got), ref, bf16_out=True, tight=True, absref=absref, label=f"{name} mma bf16 rows={rows}")
    res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=7).astype(np.float32)).cuda()
    got = rt.gemm(w, a, out=res.clone(), out_dtype=torch.float32, residual=res)
    check_close(got.cpu().numpy(), ref + res.cpu().numpy(), bf16_out=False, label=f"{name} mma residual rows={rows}")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("n,k", [(203, 768), (5, 256)])
def test_rows32_repack_on_device(rt, name, n, k):
    """splosh_gguf_repack_rows32 against the host restatement of the order, byte for byte (the
    padding rows zero); with fewer rows than one group of 32, the GEMM at 1-64 activation rows and
    the dequant against the file order's results, bit for bit."""
    from qcheck import rows32_order
    t = TYPES[name]
    native = oracle.gguf_random_native(t, n, k, seed=81 + t)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, n, k)
    w32 = rt.gguf_repack_rows32(w)
    assert w32.rows32 and w32.native.numel() == (n + 31) // 32 * 32 * native.size // n
    assert np.array_equal(w32.native.cpu().numpy(), rows32_order(native, t, n, k))
    if n < 32:
        dense = oracle.gguf_decode(t, native).reshape(n, k)
        for rows in (1, 3, 9, 64):
            a = bf16_tensor(oracle.bf16_normal((rows, k), seed=rows))
            got = rt.gemm(w, a, out_dtype=torch.float32).cpu().numpy()
            got32 = rt.gemm(w32, a, out_dtype=torch.float32).cpu().numpy()
            assert np.array_equal(got, got32), f"{name} n={n} rows={rows}"
        assert np.array_equal(rt.dequant(w32).cpu().numpy().view(np.uint32), dense.view(np.uint32))


@pytest.mark.parametrize("name", list(TYPES))
def test_rows32_kernels_match_native(rt, name):
    """Every kernel on the ROWS32 order gives what it gives on the file's order, bit for bit (the
    same blocks decoded in the same order): the streaming kernel (1-8 rows), the stream-K MFMA
    kernel (to 64), the tiled kernel (100), the prefill kernel (256), the dequant and the embedding
    lookup; and the native results match the oracle."""
    t = TYPES[name]
    n, k = 256, 768
    native = oracle.gguf_random_native(t, n - 53, k, seed=91 + t)
    rows_w = n - 53  # 203 weight rows: a partial group of 32
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, rows_w, k)
    w32 = rt.gguf_repack_rows32(w)
    dense = oracle.gguf_decode(t, native).reshape(rows_w, k)
    for rows in (1, 2, 4, 6, 8, 33, 64, 100):
        a_bits = oracle.bf16_normal((rows, k), seed=rows + 97)
        a = bf16_tensor(a_bits)
        got = rt.gemm(w, a, out_dtype=torch.float32).cpu().numpy()
        got32 = rt.gemm(w32, a, out_dtype=torch.float32).cpu().numpy()
        assert np.array_equal(got, got32), f"{name} rows={rows}"
        if rows in (2, 33):
            check_close(got, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                        absref=abs_gemm(a_bits, dense), label=f"{name} rows={rows}")
    # The prefill kernel takes whole 128-column tiles: 256 weight rows.
    native_p = oracle.gguf_random_native(t, n, k, seed=93 + t)
    wp = rt.GgufWeight(torch.from_numpy(native_p).cuda(), t, n, k)
    a = bf16_tensor(oracle.bf16_normal((256, k), seed=98))
    assert np.array_equal(rt.gemm(wp, a, out_dtype=torch.float32).cpu().numpy(),
                          rt.gemm(rt.gguf_repack_rows32(wp), a, out_dtype=torch.float32).cpu().numpy())
    assert np.array_equal(rt.dequant(w32).cpu().numpy().view(np.uint32), dense.view(np.uint32))
    tokens = torch.tensor([0, 31, 32, 202, 77, 203], dtype=torch.int32, device="cuda")  # 203: past the table
    assert np.array_equal(rt.embed(w, tokens, out_dtype=torch.float32).cpu().numpy(),
                          rt.embed(w32, tokens, out_dtype=torch.float32).cpu().numpy())


def test_q8_0_one_row_long_k(rt):
    """Q8_0 at one row with K = 33792, past the 32768 whose activation row fits the LDS: the fp32
    decode kernel reading the activations from memory, against the oracle."""
    t = TYPES["q8_0"]
    n, k = 72, 33792
    w, dense = _weight(rt, t, n, k, seed=71)
    a_bits = oracle.bf16_normal((1, k), seed=72)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32).cpu().numpy()
    check_close(got, oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label="q8_0 K33792 one row")


@pytest.mark.parametrize("name", ["q6K", "q8_0"])
def test_config0_size_sampled(rt, name):
    """K=5120 -> N=17408 at one row, 256 sampled output columns against the oracle."""
    t = TYPES[name]
    n, k = 17408, 5120
    elems, size = oracle.GGUF_BLOCK[t]
    native = oracle.gguf_random_native(t, n, k, seed=11)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, n, k)
    a_bits = oracle.bf16_normal((1, k), seed=12)
    got = to_f32(rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32))
    cols = np.sort(np.random.default_rng(13).choice(n, 256, replace=False))
    row_bytes = k // elems * size
    rows = native.reshape(n, row_bytes)[cols]
    dense = oracle.gguf_decode(t, rows.reshape(-1)).reshape(len(cols), k)
    check_close(got[:, cols], oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label=f"{name} config0")


@pytest.mark.parametrize("name", ["q6K", "q3K"])
@pytest.mark.parametrize("rows", [2, 4, 6, 8])
def test_streaming_long_k_sampled(rt, name, rows):
    """Q6_K and Q3_K at K=17408 -> N=5120 through AUTO: the streaming kernel up to the format's
    limit (its pairs form sums the unsigned codes and takes the bias off once a group, so the
    cancellation grows with K), the MFMA kernel above; 256 sampled columns against the oracle at
    the tight tolerance."""
    t = TYPES[name]
    n, k = 5120, 17408
    elems, size = oracle.GGUF_BLOCK[t]
    native = oracle.gguf_random_native(t, n, k, seed=50 + rows)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, n, k)
    a_bits = oracle.bf16_normal((rows, k), seed=51 + rows)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32).cpu().numpy()
    cols = np.sort(np.random.default_rng(52 + rows).choice(n, 256, replace=False))
    dense = oracle.gguf_decode(t, native.reshape(n, k // elems * size)[cols].reshape(-1)).reshape(len(cols), k)
    check_close(got[:, cols], oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label=f"{name} K17408 rows={rows}")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows32", [False, True])
def test_config3_shape_mma_sampled(rt, name, rows32):
    """Config 3's shape (K=17408 -> N=5120) at 64 rows in every native format, through AUTO (the
    stream-K MFMA kernel), in the file's order and the ROWS32 order: 256 sampled columns against
    the oracle at the tight tolerance."""
    t = TYPES[name]
    n, k, rows = 5120, 17408, 64
    elems, size = oracle.GGUF_BLOCK[t]
    native = oracle.gguf_random_native(t, n, k, seed=60 + t)
    w = rt.GgufWeight(torch.from_numpy(native).cuda(), t, n, k)
    if rows32:
        w = rt.gguf_repack_rows32(w)
    a_bits = oracle.bf16_normal((rows, k), seed=61 + t)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32).cpu().numpy()
    cols = np.sort(np.random.default_rng(62 + t).choice(n, 256, replace=False))
    dense = oracle.gguf_decode(t, native.reshape(n, k // elems * size)[cols].reshape(-1)).reshape(len(cols), k)
    check_close(got[:, cols], oracle.gemm_a_bf16_w_f32(a_bits, dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits, dense), label=f"{name} K17408 M=64 rows32={rows32}")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [256, 513])
@pytest.mark.parametrize("split", [True, False])
def test_prefill_kernel(rt, name, rows, split):
    """The 256 x 256 prefill kernel over native blocks (AUTO from 256 rows for N % 128 == 0):
    partial tiles, the last round split over all workgroups (stream-K) and not, both output
    types, the residual."""
    t = TYPES[name]
    n, k = 384, 1536
    w, dense = _weight(rt, t, n, k, seed=rows + 7 * t)
    a_bits = oracle.bf16_normal((rows, k), seed=rows + 1)
    ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
    absref = abs_gemm(a_bits, dense)
    ws = None if split else torch.empty(0, dtype=torch.uint8, device="cuda")
    a = bf16_tensor(a_bits)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = rt.gemm(w, a, out_dtype=out_dtype, workspace=ws)
        check_close(to_f32(got), ref, bf16_out=out_dtype == torch.bfloat16, tight=True, absref=absref,
                    label=f"{name} prefill rows={rows} split={split} {out_dtype}")
    res = torch.from_numpy(oracle.bf16_normal((rows, n), seed=6).astype(np.float32)).cuda()
    got = rt.gemm(w, a, out=res.clone(), out_dtype=torch.float32, residual=res, workspace=ws)
    check_close(got.cpu().numpy(), ref + res.cpu().numpy(), bf16_out=False, tight=True, absref=absref,
                label=f"{name} prefill residual rows={rows} split={split}")


@pytest.mark.parametrize("name", list(TYPES))
def test_tiled_large_grid(rt, name):
    """Enough 128 x 128 blocks for the large tile shape, sampled activation rows."""
    t = TYPES[name]
    n, k, rows = 2048, 512, 512
    w, dense = _weight(rt, t, n, k, seed=40 + t)
    a_bits = oracle.bf16_normal((rows, k), seed=41)
    got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32).cpu().numpy()
    pick = np.sort(np.random.default_rng(42).choice(rows, 48, replace=False))
    check_close(got[pick], oracle.gemm_a_bf16_w_f32(a_bits[pick], dense), bf16_out=False, tight=True,
                absref=abs_gemm(a_bits[pick], dense), label=f"{name} tiled large")


def test_tiled_workspace_reuse_and_no_split(rt):
    """One workspace reused across shapes and formats (the split kernel leaves its counters zeroed),
    and the unsplit kernel (an empty workspace)."""
    k = 2048
    ws = torch.zeros(rt.workspace_bytes(64, 512, k), dtype=torch.uint8, device="cuda")
    for name, n, rows in (("q6K", 512, 64), ("q8_0", 256, 9), ("q6K", 512, 33), ("iq4XS", 384, 64), ("q8_0", 100, 70)):
        t = TYPES[name]
        w, dense = _weight(rt, t, n, k, seed=n + rows)
        a_bits = oracle.bf16_normal((rows, k), seed=rows)
        ref = oracle.gemm_a_bf16_w_f32(a_bits, dense)
        for space in (ws, torch.empty(0, dtype=torch.uint8, device="cuda")):
            got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32, workspace=space)
            check_close(got.cpu().numpy(), ref, bf16_out=False, tight=True, absref=abs_gemm(a_bits, dense),
                        label=f"{name} n={n} rows={rows} split={space.numel() > 0}")
    assert not ws[:16384].any(), "arrival counters left nonzero"


def test_from_gguf_file(rt, tmp_path):
    n, k = 96, 512
    tensors, dense = [], {}
    for name, t in TYPES.items():
        native = oracle.gguf_random_native(t, n, k, seed=t)
        tensors.append((f"blk.0.{name}.weight", t, [k, n], native.tobytes()))
        dense[name] = oracle.gguf_decode(t, native).reshape(n, k)
    f = gguf.GgufFile(gguf.write_gguf(tmp_path / "m.gguf", [], tensors))
    a_bits = oracle.bf16_normal((2, k), seed=3)
    for name in TYPES:
        w = gguf.load_weight(f, f"blk.0.{name}.weight")
        assert isinstance(w, rt.GgufWeight) and (w.rows, w.inner) == (n, k)
        got = rt.gemm(w, bf16_tensor(a_bits), out_dtype=torch.float32)
        check_close(got.cpu().numpy(), oracle.gemm_a_bf16_w_f32(a_bits, dense[name]), bf16_out=False, tight=True,
                    absref=abs_gemm(a_bits, dense[name]), label=f"file {name}")
        w32 = gguf.load_weight(f, f"blk.0.{name}.weight", rows32=True)
        assert w32.rows32 and (w32.rows, w32.inner) == (n, k)
        assert np.array_equal(rt.gemm(w32, bf16_tensor(a_bits), out_dtype=torch.float32).cpu().numpy(),
                              got.cpu().numpy())


def test_rejects_other_types_and_bad_shapes(rt):
    from splosh_amd import _lib
    a = bf16_tensor(oracle.bf16_normal((1, 512), seed=1))
    out = torch.empty((1, 64), dtype=torch.float32, device="cuda")
    native = torch.zeros(64 * 16 * 34, dtype=torch.uint8, device="cuda")
    lib = _lib.lib()
    for t in (0, 2, 12, 13):   # f32, Q4_0; Q4_K and Q5_K take the plane form, not native blocks
        st = lib.splosh_gguf_gemm(t, native.data_ptr(), 64, 512, a.data_ptr(), 512, out.data_ptr(), 64,
                                  _lib.F32, None, 1, None, 0, None)
        assert st != 0
    st = lib.splosh_gguf_gemm(8, native.data_ptr(), 64, 500, a.data_ptr(), 512, out.data_ptr(), 64, _lib.F32,
                              None, 1, None, 0, None)
    assert st != 0
    # A native pointer that is not 4-byte aligned is refused (the kernels read dword windows).
    st = lib.splosh_gguf_gemm(8, native.data_ptr() + 2, 64, 512, a.data_ptr(), 512, out.data_ptr(), 64, _lib.F32,
                              None, 1, None, 0, None)
    assert st == 2  # layoutMismatch
