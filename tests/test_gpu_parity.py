"""GPU parity of the HIP backend against the CPU oracle, through the C ABI.

Bar (as stated for this path): bf16 outputs within 1e-2 * max|y_oracle| of the
oracle (the relOK convention of ggml/ggml_test.go:56-65, fp32 accumulation on
both sides); dequantized weights bit-exact. fp32 outputs are held to 1e-3.
At full model sizes the oracle is run on a random subset of output rows (each
output depends only on its own weight row), and size-independent properties
(one-hot columns, linearity) cover the whole matrix.
"""
import numpy as np
import pytest

from janis_amd import synth
from janis_amd.engine import BF16, F16, F32, I32, U32, JanisHipError
from tests.conftest import hip_runtime, rel_ok, step, upload_quant

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
F32_TOL = 1e-3


def _oracle_rows(oracle, x, q, rows):
    """Oracle QuantMatmul restricted to output rows `rows` (decode or prefill path)."""
    return oracle.quant_matmul(x, q.w[rows], q.s[rows], q.b[rows], q.group_size)


# -- Dequantize ----------------------------------------------------------------

def test_dequantize_known_answer(hip):
    """cpu/cpu_test.go:121-149 through the C ABI."""
    step("jh_dequantize word 0x87654321 gs=4")
    w = hip.FromRaw(U32, np.array([0x87654321], np.uint32), 1, 1)
    s = hip.FromFloats(np.array([2.0, 0.1], np.float32), 1, 2)
    b = hip.FromFloats(np.array([0.5, -1.0], np.float32), 1, 2)
    got = hip.Floats(hip.Dequantize(w, s, b, 4, 4))[0]
    want = np.array([2.5, 4.5, 6.5, 8.5, -0.5, -0.4, -0.3, -0.2], np.float32)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)
    step("jh_quant_matmul ones gs=4 (generic kernel)")
    x = hip.FromFloats(np.ones(8, np.float32), 1, 8)
    y = hip.Floats(hip.QuantMatmul(x, w, s, b, True, 4, 4))
    assert abs(float(y[0, 0]) - 20.6) < 1e-5


@pytest.mark.parametrize("sb", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("n,k,gs", [(64, 4096, 64), (33, 768, 32), (17, 1024, 128), (5, 64, 16)])
def test_dequantize_bit_exact(hip, oracle, sb, n, k, gs):
    q = synth.quant_linear(100 + n, n, k, gs)
    w = hip.FromRaw(U32, q.w, n, k // 8)
    if sb == "bf16":
        s_np, b_np = q.s, q.b
        s, b = hip.FromBF16Bits(q.s_bits, *q.s_bits.shape), hip.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    elif sb == "f16":
        s_np = q.s.astype(np.float16).astype(np.float32)
        b_np = q.b.astype(np.float16).astype(np.float32)
        s = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape)
        b = hip.FromRaw(F16, q.b.astype(np.float16), *q.b.shape)
    else:  # arbitrary fp32 scales: q*s is not exact, so the rounding order matters
        rng = np.random.default_rng(n)
        s_np = (q.s * (1 + rng.random(q.s.shape, dtype=np.float32) * 1e-3)).astype(np.float32)
        b_np = (q.b + rng.random(q.b.shape, dtype=np.float32) * 1e-4).astype(np.float32)
        s, b = hip.FromFloats(s_np), hip.FromFloats(b_np)
    step(f"jh_dequantize {n}x{k} gs={gs} scales={sb}")
    got = hip.Floats(hip.Dequantize(w, s, b, gs, 4))
    want = oracle.dequantize(q.w, s_np, b_np, gs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = hip.Floats(hip.Dequantize(w, s, b, gs, 4, out_dtype=BF16))
    assert np.array_equal(got16, synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(want)))


@pytest.mark.parametrize("name,tol", [("f32", 2e-4), ("bf16", 5e-2)])
def test_inkling2_embed_golden(hip, name, tol):
    """The MLX golden embedding held by the reference (inkling2/testdata), with
    the dequantization on the GPU and RMSNorm (cpu/cpu_ops.go:145-162) on the host."""
    import os

    from tests.test_oracle import GOLDEN, _rmsnorm_rows

    fx = np.load(os.path.join(GOLDEN, f"inkling2_embed_{name}.npz"))
    rows = fx["w"][fx["tokens"]]
    w = hip.FromRaw(U32, rows, *rows.shape)
    if str(fx["s_dtype"]) == "BF16":
        s = hip.FromBF16Bits(fx["s"][fx["tokens"]])
        b = hip.FromBF16Bits(fx["b"][fx["tokens"]])
        norm = synth.bf16_bits_to_f32(fx["norm"])
    else:
        s, b, norm = hip.FromFloats(fx["s"][fx["tokens"]]), hip.FromFloats(fx["b"][fx["tokens"]]), fx["norm"]
    step(f"jh_dequantize inkling2 embed {name}")
    deq = hip.Floats(hip.Dequantize(w, s, b, int(fx["group_size"]), int(fx["bits"])))
    got = _rmsnorm_rows(deq, norm, float(fx["eps"]))
    ok, d, sc = rel_ok(got, fx["embed"], tol)
    assert ok, (d, sc)


# -- decode qmv ---------------------------------------------------------------

QMV_SHAPES = [
    # (N, K, gs): every fast-kernel tile (K = 256..16384), group sizes 32/64/128,
    # ragged N, the lm_head-size tile, and the generic kernel (K = 1032, gs = 8).
    # K = 12288 with N >= 2048 is the two-set pipelined tile; 3001 rows leave the
    # persistent blocks ragged pass counts and a half-filled last row pair.
    (4096, 4096, 64), (1024, 4096, 64), (33, 2048, 64), (1000, 6144, 64), (257, 8192, 64),
    (4096, 12288, 64), (3001, 12288, 32), (100, 16384, 64), (129, 1024, 64), (70, 3072, 64), (65, 512, 64),
    (48, 1536, 64), (31, 256, 64), (768, 768, 64), (300, 4096, 32), (300, 4096, 128),
    (50, 2048, 32), (40, 768, 128), (24, 1032, 8), (9, 96, 32), (65539, 4096, 64)]


@pytest.mark.parametrize("n,k,gs", QMV_SHAPES)
def test_qmv_matches_oracle(hip, oracle, n, k, gs):
    q = synth.quant_linear(1000 + n + k, n, k, gs)
    xb, x = synth.activations(2000 + k, (1, k))
    w, s, b = upload_quant(hip, q)
    xt = hip.FromBF16Bits(xb, 1, k)
    want = oracle.quant_matmul(x, q.w, q.s, q.b, gs)  # AVX2-kernel order (cpu/qmv_amd64.s)
    step(f"jh_quant_matmul rows=1 N={n} K={k} gs={gs} y=bf16")
    y16 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, gs, 4))
    ok, d, sc = rel_ok(y16, want, BF16_TOL)
    assert ok, ("bf16", d, sc)
    step(f"jh_quant_matmul rows=1 N={n} K={k} gs={gs} y=f32")
    y32 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, gs, 4, out_dtype=F32))
    ok, d, sc = rel_ok(y32, want, F32_TOL)
    assert ok, ("f32", d, sc)


def test_qmv_f32_activations(hip, oracle):
    """x in fp32 (the CPU backend's activation type) takes the decode tile with
    x rounded to bf16 in registers: within the bf16 bar of the oracle's fp32-x
    product (measured 1.3e-3 of max|y| here), and at a row length outside the
    tiles the generic kernel multiplies fp32 x unrounded (within the fp32 bar)."""
    q = synth.quant_linear(7, 200, 4096)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    w, s, b = upload_quant(hip, q)
    step("jh_quant_matmul rows=1 x=f32")
    y = hip.Floats(hip.QuantMatmul(hip.FromFloats(x), w, s, b, True, 64, 4))
    ok, d, sc = rel_ok(y, oracle.quant_matmul(x, q.w, q.s, q.b, 64), BF16_TOL)
    assert ok, (d, sc)
    q = synth.quant_linear(8, 200, 4000, 80)
    x = rng.standard_normal((1, 4000)).astype(np.float32)
    w, s, b = upload_quant(hip, q)
    step("jh_quant_matmul rows=1 x=f32, K=4000 (generic kernel)")
    y = hip.Floats(hip.QuantMatmul(hip.FromFloats(x), w, s, b, True, 80, 4))
    ok, d, sc = rel_ok(y, oracle.quant_matmul(x, q.w, q.s, q.b, 80), F32_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("name,n,k", [("q_proj", 4096, 4096), ("k_proj", 1024, 4096),
                                      ("gate_up", 24576, 4096), ("down", 4096, 12288),
                                      ("lm_head", 151936, 4096)])
def test_qwen3_8b_decode_shapes(hip, oracle, name, n, k):
    """Config-1 shapes at full size: oracle on 384 random rows, plus one-hot
    columns over the whole matrix (bit-exact with fp32 output)."""
    q = synth.quant_linear(3000 + n, n, k)
    xb, x = synth.activations(4000 + k, (1, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_quant_matmul {name} {n}x{k}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, k), w, s, b, True, 64, 4))
    rows = np.sort(np.random.default_rng(n).choice(n, size=min(n, 384), replace=False))
    want = _oracle_rows(oracle, x, q, rows)
    ok, d, sc = rel_ok(y[0, rows], want[0], BF16_TOL)
    assert ok, (d, sc)
    for j in (0, 31, k // 2 + 5, k - 1):
        e = np.zeros((1, k), np.uint16)
        e[0, j] = 0x3F80  # bf16 1.0
        step(f"jh_quant_matmul {name} one-hot column {j}")
        yc = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(e, 1, k), w, s, b, True, 64, 4, out_dtype=F32))[0]
        col = oracle.dequantize(q.w[rows], q.s[rows], q.b[rows], 64)[:, j]
        assert np.array_equal(yc[rows].view(np.uint32), col.copy().view(np.uint32))


def test_qmv_linearity_full_lm_head(hip):
    """y(a + b) == y(a) + y(b) over all 151936 rows (fp32 output), with b = a
    with random signs so that a + b (0 or 2a) is exact in bf16."""
    n, k = 151936, 4096
    q = synth.quant_linear(77, n, k)
    w, s, b = upload_quant(hip, q)
    ab, a = synth.activations(78, (1, k))
    sign = np.random.default_rng(79).integers(0, 2, (1, k)).astype(np.uint16) << np.uint16(15)
    bb = (ab ^ sign).astype(np.uint16)
    cb = synth.f32_to_bf16_bits((a + synth.bf16_bits_to_f32(bb)).astype(np.float32))
    assert np.array_equal(synth.bf16_bits_to_f32(cb), a + synth.bf16_bits_to_f32(bb))
    run = lambda xb: hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, k), w, s, b, True, 64, 4,
                                                out_dtype=F32))[0].astype(np.float64)
    step("jh_quant_matmul lm_head linearity")
    ya, yb, yc = run(ab), run(bb), run(cb)
    ok, d, sc = rel_ok(yc, ya + yb, F32_TOL)
    assert ok, (d, sc)


# -- prefill qmm ------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k,gs", [(2, 64, 512, 64), (3, 130, 1024, 64), (13, 256, 2048, 64),
                                      (128, 384, 4096, 64), (77, 200, 1024, 32), (40, 96, 768, 128),
                                      (5, 24, 1032, 8),
                                      # K a multiple of 64 but not of 256: the LDS tile, K whole
                                      # (704 = 11 steps) and K split 2 (1088 = 17 steps)
                                      (100, 300, 704, 64), (100, 300, 1088, 64)])
def test_qmm_matches_oracle(hip, oracle, m, n, k, gs):
    q = synth.quant_linear(5000 + m + n, n, k, gs)
    xb, x = synth.activations(6000 + m, (m, k))
    w, s, b = upload_quant(hip, q)
    want = oracle.quant_matmul(x, q.w, q.s, q.b, gs)  # wbuf order (cpu/cpu_misc.go:378-399)
    step(f"jh_quant_matmul rows={m} N={n} K={k} gs={gs}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, m, k), w, s, b, True, gs, 4))
    ok, d, sc = rel_ok(y, want, BF16_TOL)
    assert ok, (d, sc)
    y32 = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, m, k), w, s, b, True, gs, 4, out_dtype=F32))
    ok, d, sc = rel_ok(y32, want, 5e-3)
    assert ok, ("f32 out", d, sc)


_ROWS_W = {}


def _rows_weights(seed, n, k, gs):
    """Weights of the multi-row cases, made once per shape (lm_head-sized ones
    take seconds)."""
    if (seed, gs) not in _ROWS_W:
        _ROWS_W.clear()
        _ROWS_W[(seed, gs)] = synth.quant_linear(seed, n, k, gs)
    return _ROWS_W[(seed, gs)]


@pytest.mark.parametrize("n,k,rows,gs,sb", [
    (2048, 4096, 8, 64, "bf16"),    # 8 rows per launch (below 2^24 weights)
    (1024, 4096, 5, 64, "bf16"),    # 8 rows per launch, 5 used
    (4096, 4096, 3, 64, "f16"),     # 4 rows per launch, 3 used
    (1000, 12288, 4, 64, "bf16"),   # 2 rows per launch, two launches, ragged N
    (1000, 12288, 3, 64, "bf16"),   # two launches, the second with one row
    (4096, 12288, 2, 64, "bf16"),   # down_proj's own shape: the one-row call takes the pipelined
    (4096, 12288, 2, 64, "f16"),    #   <32,3,1,4> tile (N >= 2048), the rows kernel <32,3,2,4>
    (1300, 12288, 3, 64, "bf16"),
    (257, 8192, 3, 32, "f16"),      # 4 rows per launch
    (300, 2048, 7, 128, "bf16"),
    (33, 768, 2, 64, "bf16"),
    (70, 3072, 3, 64, "f16"),
    (100, 16384, 4, 64, "bf16"),
    (1000, 24576, 2, 64, "bf16"),   # the 64-lane 3-load tile (one launch)
    (600, 24576, 4, 64, "f16"),     # two launches of 2 rows
    (151936, 4096, 2, 64, "bf16"),  # lm_head: the one-row call's 64-lane, 2-way split
    (151936, 4096, 3, 64, "bf16"),
    (151936, 4096, 4, 64, "bf16"),
    (4095, 4096, 6, 64, "bf16"),    # just under 2^24 weights: 5..8 rows stay on the tile
    (2048, 1024, 5, 64, "bf16"),    # K = 1024, the smallest row length that keeps 5..8 rows
    (4096, 1536, 4, 64, "f16"),     # long-row tile from K = 1536 below 2^24 weights
])
def test_qmv_rows_match_one_row_calls(hip, oracle, n, k, rows, gs, sb):
    """The few-row calls the decode tiles take (every row's x in registers):
    each row of y has the bits of a one-row call on that row (fp32 out), and
    the bf16 output is within the bar of the oracle."""
    q = _rows_weights(12000 + n + k, n, k, gs)
    xb, x = synth.activations(13000 + rows, (rows, k))
    w = hip.FromRaw(U32, q.w, *q.w.shape)
    if sb == "f16":
        s_np, b_np = (v.astype(np.float16).astype(np.float32) for v in (q.s, q.b))
        s, b = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape), hip.FromRaw(F16, q.b.astype(np.float16), *q.b.shape)
    else:
        s_np, b_np = q.s, q.b
        s, b = hip.FromBF16Bits(q.s_bits, *q.s_bits.shape), hip.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    step(f"jh_quant_matmul rows={rows} N={n} K={k} gs={gs} sb={sb} (multi-row decode tile)")
    y32 = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, rows, k), w, s, b, True, gs, 4, out_dtype=F32))
    for r in range(rows):
        y1 = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb[r:r + 1], 1, k), w, s, b, True, gs, 4, out_dtype=F32))
        assert np.array_equal(y32[r].view(np.uint32), y1[0].view(np.uint32)), r
    y16 = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, rows, k), w, s, b, True, gs, 4))
    cs = np.sort(np.random.default_rng(n).choice(n, size=min(n, 96), replace=False))
    ok, d, sc = rel_ok(y16[:, cs], oracle.quant_matmul(x, q.w[cs], s_np[cs], b_np[cs], gs), BF16_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("n,k,rows,xdt", [
    (4096, 4096, 8, "bf16"),    # 2^24 weights: 5..8 rows go to the GEMM
    (12288, 4096, 5, "bf16"),
    (24576, 4096, 6, "f32"),
    (4096, 512, 7, "bf16"),     # K = 512: the GEMM at 5..8 rows
    (4096, 12288, 3, "bf16"),   # long rows from 2^24 weights: 3..4 rows go to the GEMM
    (2048, 768, 4, "f32"),      # K = 768: the GEMM at 3..4 rows
])
def test_few_rows_on_the_gemm(hip, oracle, n, k, rows, xdt):
    """The few-row calls outside the decode tiles' rule take the MFMA product
    (where it is the faster path): within the bar of the oracle, for bf16 and
    fp32 x, and the same bits on a repeated call."""
    q = _rows_weights(15000 + n + k, n, k, 64)
    xb, x = synth.activations(16000 + rows, (rows, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_quant_matmul rows={rows} N={n} K={k} x={xdt} (few rows on the GEMM)")
    xt = hip.FromBF16Bits(xb, rows, k) if xdt == "bf16" else hip.FromFloats(x.astype(np.float32), rows, k)
    y1 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4))
    y2 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    cs = np.sort(np.random.default_rng(n + rows).choice(n, size=min(n, 96), replace=False))
    ok, d, sc = rel_ok(y1[:, cs], oracle.quant_matmul(x, q.w[cs], q.s[cs], q.b[cs], 64), BF16_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("name,n,k", [("gate_up", 12288, 4096), ("down", 4096, 12288)])
def test_qmm_prefill_shapes(hip, oracle, m, name, n, k):
    """Config-2 shapes: the oracle on a random 48x96 block of the output."""
    q = synth.quant_linear(7000 + n, n, k)
    xb, x = synth.activations(8000 + m, (m, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_quant_matmul prefill {name} M={m}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, m, k), w, s, b, True, 64, 4))
    rng = np.random.default_rng(m + n)
    rs = np.sort(rng.choice(m, size=min(m, 48), replace=False))
    cs = np.sort(rng.choice(n, size=96, replace=False))
    want = oracle.quant_matmul(x[rs], q.w[cs], q.s[cs], q.b[cs], 64)
    ok, d, sc = rel_ok(y[np.ix_(rs, cs)], want, BF16_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("m,n,k,gs,sb,xf32,out_dtype", [
    # bf16 x: the LDS-ring tile (waves, steps of lead, K split)
    (500, 12288, 4096, 64, "bf16", False, BF16),   # 8 waves lead 3, K whole, M ragged
    (640, 8000, 2048, 32, "f16", False, BF16),     # 8 waves lead 3, N ragged (8000 = 31.25 tiles of 256)
    (300, 2784, 2048, 64, "bf16", False, BF16),    # 4 waves lead 3, K split 2, bf16 out via the fp32 buffer
    (128, 12288, 4096, 32, "f32", False, F32),     # 4 waves lead 3, K split 2, 4 dwords of scales per lane
    (384, 6144, 4096, 64, "f16", False, F32),      # qkv at M=384: 4 waves lead 3, K whole
    (260, 9000, 4096, 64, "bf16", False, BF16),    # 4 waves lead 3, M ragged
    (128, 4096, 12288, 64, "f16", False, BF16),    # down at M=128: 4 waves lead 3, K split 8
    (77, 1000, 4096, 64, "bf16", False, F32),      # 4 waves lead 3, K split 8, M and N ragged
    (96, 6144, 12288, 64, "bf16", False, F32),     # 4 waves lead 1 (two blocks per CU), K split 8
    (1000, 2000, 1024, 128, "f32", False, BF16),   # group 128 with fp32 scales: 4 waves lead 3
    (1536, 4096, 12288, 64, "bf16", False, BF16),  # down at M=1536: 256-row blocks, 8 waves lead 1, K split 2
    (1024, 12288, 4096, 64, "bf16", False, F32),   # 256-row blocks, K whole
    (768, 4096, 12288, 64, "f16", False, BF16),    # 256-row blocks, K split 4
    (1300, 6000, 2048, 64, "f32", False, F32),     # 256-row blocks, M ragged (5.08 blocks), fp32 scales
    (1000, 9000, 4096, 32, "bf16", False, BF16),   # 256-row blocks, N ragged, group 32
    (500, 12288, 4096, 32, "f32", False, F32),     # 8 waves lead 3 with 4 dwords of scales per lane: 160 KiB of LDS
    (1024, 12288, 4096, 32, "f32", False, BF16),   # 256-row blocks with 4 dwords of scales per lane: 160 KiB
    # up to 64 rows of bf16 x: 32- or 64-row blocks of the LDS-ring tile
    (9, 12288, 4096, 64, "bf16", False, F32),      # 32 rows, 8 waves, K split 4
    (20, 4096, 12288, 64, "f16", False, BF16),     # 32 rows, 4 waves, K split 8
    (24, 24576, 4096, 128, "f32", False, F32),     # 32 rows, 4 waves, K whole, group 128
    (50, 6144, 4096, 32, "bf16", False, F32),      # 64 rows, 4 waves, K split 4, group 32
    (48, 9000, 4096, 64, "bf16", False, BF16),     # 64 rows, 8 waves, K split 4, N ragged
    # fp32 x: rounded to bf16 into the workspace, then the LDS-ring tile
    (700, 12288, 4096, 64, "bf16", True, BF16),    # 256-row blocks
    (128, 4096, 12288, 64, "f16", True, F32),      # 4 waves lead 3, K split 8
    (9, 12288, 4096, 64, "bf16", True, F32),       # 32-row blocks, K split 4
    # group 128 with bf16/f16 scales (scales in half dwords): the register tile (waves, K split)
    (1000, 6000, 1024, 128, "bf16", True, F32),    # 6 waves, fp32 x
    (300, 2784, 2048, 128, "f16", False, F32),     # 6 waves, K split 4
    (1100, 3000, 2048, 128, "bf16", True, BF16),   # 4 waves, K whole
    (2048, 4096, 12288, 128, "bf16", False, F32),  # 8 waves, K whole
])
def test_qmm_planner_tiles(hip, oracle, m, n, k, gs, sb, xf32, out_dtype):
    """Every tile/split pair the prefill planner picks on a 256-CU MI355X (the
    LDS-ring tile in its four 128-row shapes and its 32/64/256-row blocks, for
    bf16 x and for fp32 x rounded into the workspace; the register tile with
    4/6/8 waves where the scales do not fill whole dwords; K whole or split,
    ragged M and N, bf16/f16/fp32 scales, group sizes 32/64/128 and both
    outputs): the oracle on a random block of up to 48x96 of the output."""
    q = synth.quant_linear(9000 + m + n, n, k, gs)
    xb, x = synth.activations(9500 + m, (m, k))
    w = hip.FromRaw(U32, q.w, *q.w.shape)
    if sb == "bf16":
        s_np, b_np = q.s, q.b
        s, b = hip.FromBF16Bits(q.s_bits, *q.s_bits.shape), hip.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    elif sb == "f16":
        s_np, b_np = (v.astype(np.float16).astype(np.float32) for v in (q.s, q.b))
        s, b = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape), hip.FromRaw(F16, q.b.astype(np.float16), *q.b.shape)
    else:
        s_np, b_np = q.s, q.b
        s, b = hip.FromFloats(q.s), hip.FromFloats(q.b)
    xt = hip.FromFloats(x) if xf32 else hip.FromBF16Bits(xb, m, k)
    step(f"jh_quant_matmul planner M={m} N={n} K={k} gs={gs} sb={sb} xf32={xf32} out={out_dtype}")
    y = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, gs, 4, out_dtype=out_dtype))
    rng = np.random.default_rng(m * 7 + n)
    rs = np.sort(np.concatenate([rng.choice(m - 1, size=min(47, m - 1), replace=False), [m - 1]]))
    cs = np.sort(np.concatenate([rng.choice(n - 1, size=95, replace=False), [n - 1]]))
    want = oracle.quant_matmul(x[rs], q.w[cs], s_np[cs], b_np[cs], gs)
    ok, d, sc = rel_ok(y[np.ix_(rs, cs)], want, BF16_TOL if out_dtype == BF16 else 5e-3)
    assert ok, (d, sc)


@pytest.mark.parametrize("m,n,k", [
    (64, 1000, 2048),    # 32-row blocks (two), K split 4, N ragged
    (63, 5000, 4096),    # one 64-row block with its last row empty
    (65, 5000, 4096),    # 128-row blocks from 65 rows: 4 waves lead 1, K split 8
    (129, 5000, 4096),   # two 128-row blocks, the second with one row
    (257, 12288, 4096),  # three 128-row blocks, the third with one row
    (769, 12288, 4096),  # four 256-row blocks, the fourth with one row
])
def test_qmm_row_block_edges(hip, oracle, m, n, k):
    """Row counts around the planner's block-size changes (32/64 up to 64
    rows, 128 beyond, 256 from 256 rows) and blocks holding a single row: the
    oracle on the rows next to each block edge and the last row and column."""
    q = synth.quant_linear(9700 + m + n, n, k, 64)
    xb, x = synth.activations(9750 + m, (m, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_quant_matmul row-block edges M={m} N={n} K={k}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, m, k), w, s, b, True, 64, 4, out_dtype=F32))
    edges = {0, m - 1}
    for e in (32, 64, 128, 256, 512, 768):
        edges.update(r for r in (e - 1, e) if r < m)
    rs = np.array(sorted(edges))
    rng = np.random.default_rng(m + n)
    cs = np.sort(np.concatenate([rng.choice(n - 1, size=63, replace=False), [n - 1]]))
    want = oracle.quant_matmul(x[rs], q.w[cs], q.s[cs], q.b[cs], 64)
    ok, d, sc = rel_ok(y[np.ix_(rs, cs)], want, 5e-3)
    assert ok, (d, sc)


@pytest.mark.parametrize("m,n,k,gs,sb", [
    (2048, 12288, 4096, 64, "bf16"),  # 8 waves lead 3, K whole
    (300, 2784, 2048, 64, "f16"),     # 4 waves lead 3, K split 2
    (1000, 6000, 1024, 32, "bf16"),   # 8 waves lead 3, K whole, group 32
    (128, 4096, 12288, 64, "f32"),    # 4 waves lead 3, K split 8
    (96, 6144, 12288, 64, "bf16"),    # 4 waves lead 1, K split 8
    (1000, 2000, 1024, 128, "f32"),   # 4 waves lead 3, group 128
    (9, 12288, 4096, 64, "bf16"),     # 32-row blocks, K split 4
    (33, 12288, 4096, 32, "f16"),     # 64-row blocks, K split 4
    (1024, 12288, 4096, 64, "bf16"),  # 256-row blocks, K whole
    (1300, 6000, 2048, 128, "bf16"),  # register tile (group 128, bf16 scales), M ragged
    (300, 2784, 2048, 128, "f16"),    # register tile, K split 4
])
def test_qmm_bf16_x_matches_fp32_x(hip, m, n, k, gs, sb):
    """bf16 x against the same values widened to fp32 (rounded back to bf16 in
    the workspace before the LDS-ring tile; with group 128 and bf16/f16 scales,
    the register tile, which rounds x on its way to LDS): the same bits."""
    q = synth.quant_linear(9900 + m + n, n, k, gs)
    xb, x = synth.activations(9950 + m, (m, k))
    w = hip.FromRaw(U32, q.w, *q.w.shape)
    if sb == "bf16":
        s, b = hip.FromBF16Bits(q.s_bits, *q.s_bits.shape), hip.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    elif sb == "f16":
        s, b = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape), hip.FromRaw(F16, q.b.astype(np.float16), *q.b.shape)
    else:
        s, b = hip.FromFloats(q.s), hip.FromFloats(q.b)
    step(f"jh_quant_matmul bf16 x vs fp32 x M={m} N={n} K={k} gs={gs} sb={sb}")
    y1 = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, m, k), w, s, b, True, gs, 4, out_dtype=F32))
    y2 = hip.Floats(hip.QuantMatmul(hip.FromFloats(x), w, s, b, True, gs, 4, out_dtype=F32))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), float(np.max(np.abs(y1 - y2)))


@pytest.mark.parametrize("out_dtype", [BF16, F32])
def test_qmm_split_k_is_deterministic(hip, out_dtype):
    """K split 4 ways (M=128, 12288 x 4096): the partial products are added in a
    fixed order, so repeated calls give identical bits."""
    q = synth.quant_linear(31, 12288, 4096)
    xb, _ = synth.activations(32, (128, 4096))
    w, s, b = upload_quant(hip, q)
    xt = hip.FromBF16Bits(xb, 128, 4096)
    step(f"jh_quant_matmul split-K determinism out={out_dtype}")
    y0 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype))
    for _ in range(3):
        y1 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype))
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


@pytest.mark.parametrize("m,n,k,out_dtype", [
    (128, 4096, 4096, BF16),    # o_proj: 4 waves, K split 8, 32 tiles x 8 blocks
    (128, 6144, 4096, F32),     # q/k/v: K split 4
    (96, 4096, 12288, BF16),    # down_proj: K split 8, rows 96..127 of the tile empty
    (200, 4096, 4096, F32),     # two row tiles, the second ragged: K split 4
    (100, 4000, 4096, BF16),    # N ragged (the last column tile 32 wide): K split 8
    (130, 2000, 4096, F32),     # M and N ragged (a row tile of 2 rows): K split 8
])
def test_qmm_split_sums_in_launch(hip, oracle, m, n, k, out_dtype):
    """Plans whose split partial tiles are added inside the product's launch
    (every block resident, a tile's splits on one XCD): the oracle on a random
    block of the output, identical bits on a repeat; then, with a wait bound of 0
    polls (jh_set_wait_limit), every block gives up its wait at once (each kernel
    still exits normally): the output is all NaN, the next synchronisation
    reports JH_ERR_TIMEOUT and resets the counters, and the next call with the
    default bound has the first call's bits."""
    from janis_amd import _lib

    q = synth.quant_linear(61 + m + n, n, k)
    xb, x = synth.activations(62 + m, (m, k))
    w, s, b = upload_quant(hip, q)
    xt = hip.FromBF16Bits(xb, m, k)
    step(f"jh_quant_matmul in-launch split sums M={m} N={n} K={k} out={out_dtype}")
    y0 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype))
    rng = np.random.default_rng(m + n + k)
    rs = np.sort(np.concatenate([rng.choice(m - 1, size=min(31, m - 1), replace=False), [m - 1]]))
    cs = np.sort(np.concatenate([rng.choice(n - 1, size=63, replace=False), [n - 1]]))
    want = oracle.quant_matmul(x[rs], q.w[cs], q.s[cs], q.b[cs], 64)
    ok, d, sc = rel_ok(y0[np.ix_(rs, cs)], want, BF16_TOL if out_dtype == BF16 else 5e-3)
    assert ok, (d, sc)
    y1 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype))
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    try:
        hip.SetWaitLimit(0)
        step("the same call with a wait bound of 0 polls")
        yn = hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype)
        with pytest.raises(JanisHipError) as ei:
            hip.Sync()
        assert ei.value.code == _lib.JH_ERR_TIMEOUT, str(ei.value)
        assert np.isnan(hip.Floats(yn)).all()
        hip.Sync()  # reported once, then reset
    finally:
        hip.SetWaitLimit(1 << 22)
    step("the next call, default bound")
    y2 = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=out_dtype))
    assert np.array_equal(y0.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("rows,n,k", [(128, 12288, 4096), (128, 4096, 4096), (4, 4096, 4096), (8, 12288, 4096)])
def test_quant_matmul_graph_replays(hip, oracle, rows, n, k):
    """Captured once into a HIP graph (after one eager call, which sizes the
    workspace) and replayed on new x written into the captured buffer: every
    replay matches the eager call on the same x bit for bit. 128 x 12288 rows
    take the K-split prefill tile with the summing launch (partial tiles, then
    the ordered sum, no fill), 128 x 4096 the 8-way split with the sums inside
    the launch (its counters back at zero after every replay), 4 rows the
    multi-row decode tile, 8 rows of a 2^24-weight-plus matrix the GEMM's
    32-row blocks."""
    import ctypes

    rt = hip_runtime()
    q = synth.quant_linear(41 + rows, n, k)
    w, s, b = upload_quant(hip, q)
    xs = [synth.activations(42 + i, (rows, k)) for i in range(3)]
    xt = hip.empty(BF16, rows, k)
    yt = hip.empty(BF16, rows, n)

    def put(a):
        a = np.ascontiguousarray(a)
        hip.Sync()
        hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(xt.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        hip.Sync()

    def call():
        return hip.QuantMatmul(xt, w, s, b, True, 64, 4, out=yt)

    eager = []
    for xb, _ in xs:
        put(xb)
        call()
        eager.append(hip.Floats(yt).copy())
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        hip.SetStream(stream.value)
        step(f"capture jh_quant_matmul rows={rows} N={n} K={k}")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        call()
        assert rt.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep, i in enumerate((1, 2, 0, 1, 1)):
            step(f"graph replay {rep} on x {i}")
            put(xs[i][0])
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            got = hip.Floats(yt)
            assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), rep
        cs = np.sort(np.random.default_rng(rows).choice(n, size=64, replace=False))
        rs = np.arange(min(rows, 16))
        ok, d, sc = rel_ok(got[np.ix_(rs, cs)], oracle.quant_matmul(xs[1][1][rs], q.w[cs], q.s[cs], q.b[cs], 64),
                           BF16_TOL)
        assert ok, (d, sc)
    finally:
        hip.SetStream(None)
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        if graph.value:
            rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)


def test_qmm_rows_are_independent(hip):
    """Row r of a prefill product equals the decode product of x[r] (fp32 out, 1e-3)."""
    q = synth.quant_linear(11, 512, 4096)
    xb, _ = synth.activations(12, (37, 4096))
    w, s, b = upload_quant(hip, q)
    step("jh_quant_matmul rows=37 vs rows=1")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 37, 4096), w, s, b, True, 64, 4, out_dtype=F32))
    for r in (0, 17, 36):
        yr = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb[r:r + 1], 1, 4096), w, s, b, True, 64, 4,
                                        out_dtype=F32))
        ok, d, sc = rel_ok(y[r], yr[0], 5e-3)
        assert ok, (r, d, sc)


# -- MoE gather ------------------------------------------------------------------

_STACKS = {}


def _qwen3_moe_stack(proj):
    """Config-3 expert stacks (128 experts, hidden 2048, moe_intermediate 768),
    generated once per session: gate/up [128, 768, 2048/8], down [128, 2048, 768/8]."""
    if proj not in _STACKS:
        n, k = (2048, 768) if proj == "down" else (768, 2048)
        _STACKS[proj] = synth.quant_linear({"gate": 9768, "up": 9769, "down": 11048}[proj], n, k, lead=(128,))
    return _STACKS[proj]

@pytest.mark.parametrize("n_tok", [1, 16])
@pytest.mark.parametrize("proj", ["gate", "down"])
def test_gather_qwen3_30b_a3b(hip, oracle, n_tok, proj):
    """Config 3: 128 experts, hidden 2048, moe_intermediate 768, top-8 of a
    seeded router. gate: x [T,1,1,2048] shared by the 8 slots (A=1);
    down: x [T,8,1,768] one vector per slot (A=K)."""
    E, K = 128, 8
    n, k = (768, 2048) if proj == "gate" else (2048, 768)
    A = 1 if proj == "gate" else K
    q = _qwen3_moe_stack(proj)
    idx, _ = synth.route(9100 + n_tok, n_tok, E, K)
    xb, x = synth.activations(9200 + n_tok, (n_tok, A, 1, k))
    w, s, b = upload_quant(hip, q)
    it = hip.FromInt32(idx)
    step(f"jh_gather_quant_matmul {proj} T={n_tok} U={len(np.unique(idx))}")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, n_tok, A, 1, k), w, s, b, it, True, 64, 4))
    assert y.shape == (n_tok, K, 1, n)
    want = oracle.gather_quant_matmul(x, q.w, q.s, q.b, idx, 64)
    ok, d, sc = rel_ok(y, want, BF16_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("E,n,k,gs,A", [(6, 40, 512, 64, 1), (6, 40, 512, 64, 8), (3, 100, 4096, 32, 1),
                                         (5, 64, 1032, 8, 8)])
def test_gather_small_with_collisions(hip, oracle, E, n, k, gs, A):
    """Many slots per expert (R > 1 buckets), ragged rows, generic kernel."""
    K, T = 8, 4
    q = synth.quant_linear(50 + E + k, n, k, gs, lead=(E,))
    idx = np.random.default_rng(E * k).integers(0, E, (T, K)).astype(np.int32)
    xb, x = synth.activations(60 + A, (T, A, 1, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_gather_quant_matmul E={E} n={n} k={k} gs={gs} A={A}")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, T, A, 1, k), w, s, b, hip.FromInt32(idx),
                                         True, gs, 4, out_dtype=F32))
    want = oracle.gather_quant_matmul(x, q.w, q.s, q.b, idx, gs)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)
    # f32 activations take the generic gather kernel
    yf = hip.Floats(hip.GatherQuantMatmul(hip.FromFloats(x), w, s, b, hip.FromInt32(idx), True, gs, 4))
    ok, d, sc = rel_ok(yf, want, F32_TOL)
    assert ok, ("f32 x", d, sc)


@pytest.mark.parametrize("n_tok,A", [(160, 1), (160, 8)])
def test_gather_many_slots_workspace_path(hip, oracle, n_tok, A):
    """More than 1024 (token, slot) pairs: the separate bucketing launch."""
    E, K, n, k = 16, 8, 96, 512
    q = synth.quant_linear(70 + A, n, k, lead=(E,))
    idx, _ = synth.route(71, n_tok, E, K)
    xb, x = synth.activations(72 + A, (n_tok, A, 1, k))
    w, s, b = upload_quant(hip, q)
    step(f"jh_gather_quant_matmul pairs={n_tok * K} A={A}")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, n_tok, A, 1, k), w, s, b, hip.FromInt32(idx),
                                         True, 64, 4, out_dtype=F32))
    want = oracle.gather_quant_matmul(x, q.w, q.s, q.b, idx, 64)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)


def test_gather_out_of_range_index(hip):
    q = synth.quant_linear(1, 32, 512, lead=(4,))
    w, s, b = upload_quant(hip, q)
    xb, _ = synth.activations(2, (1, 1, 1, 512))
    idx = hip.FromInt32(np.array([[0, 7, 3, -1]], np.int32))
    step("jh_gather_quant_matmul bad index, checks off")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, 1, 1, 1, 512), w, s, b, idx, True, 64, 4,
                                         out_dtype=F32))
    assert np.isfinite(y[0, 0]).all() and np.isfinite(y[0, 2]).all()
    assert np.isnan(y[0, 1]).all() and np.isnan(y[0, 3]).all()
    hip.SetChecks(True)
    try:
        step("jh_gather_quant_matmul bad index, checks on")
        with pytest.raises(JanisHipError):
            hip.GatherQuantMatmul(hip.FromBF16Bits(xb, 1, 1, 1, 512), w, s, b, idx, True, 64, 4)
    finally:
        hip.SetChecks(False)
    # past 32 pairs the buckets come from the bucketing launch: same NaN rows
    ids = np.random.default_rng(3).integers(0, 4, (10, 4)).astype(np.int32)
    ids[2, 1], ids[7, 3] = 4, -5
    xb10, _ = synth.activations(4, (10, 1, 1, 512))
    step("jh_gather_quant_matmul bad index, 40 pairs")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb10, 10, 1, 1, 512), w, s, b, hip.FromInt32(ids),
                                         True, 64, 4, out_dtype=F32))
    bad = (ids < 0) | (ids >= 4)
    assert np.isnan(y[bad]).all() and np.isfinite(y[~bad]).all()


# -- MoE expert MLP (moeApply as one operator) ----------------------------------------

def _moe_upload(hip, qs):
    return [upload_quant(hip, q) for q in qs]


def _moe_case(hip, oracle, qs, x_shape, idx, sc, out_dtype=F32):
    xb, x = synth.activations(sum(x_shape) + int(idx.sum()), x_shape)
    st = _moe_upload(hip, qs)
    out = hip.MoeSwiGLU(hip.FromBF16Bits(xb, *x_shape), *st, hip.FromInt32(idx), hip.FromFloats(sc), 64, 4,
                        out_dtype=out_dtype)
    want = oracle.moe_apply(x, *[(q.w, q.s, q.b) for q in qs], idx, sc)
    return hip.Floats(out), want


@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_swiglu_qwen3_30b_a3b(hip, oracle, n_tok):
    """Config 3 end to end: top-8 of 128 experts from a seeded router, the
    gate+up SwiGLU launch and the score-weighted down launch against the
    oracle's moeApply (qwen/moe.go:501-511). h is bf16 on the device and fp32
    in the oracle, inside the bf16 bar."""
    qs = [_qwen3_moe_stack(p) for p in ("gate", "up", "down")]
    idx, sc = synth.route(9300 + n_tok, n_tok, 128, 8)
    step(f"jh_moe_swiglu qwen3-30b-a3b T={n_tok} U={len(np.unique(idx))}")
    got, want = _moe_case(hip, oracle, qs, (n_tok, 2048), idx, sc)
    assert got.shape == (n_tok, 2048)
    ok, d, s = rel_ok(got, want, BF16_TOL)
    assert ok, (d, s)


@pytest.mark.parametrize("n_tok", [1, 4, 16])
def test_moe_swiglu_repeats_bit_for_bit(hip, n_tok):
    """The score-weighted sum over a token's slots is taken in a fixed order
    (no atomics), so repeated calls on the same inputs give the same bits --
    the one-launch-per-token combine (1 and 4 tokens) and the partials plus
    combine launch (16 tokens) alike."""
    qs, st = _t1_stacks(hip)
    idx, sc = synth.route(9350 + n_tok, n_tok, 128, 8)
    xb, _ = synth.activations(9351 + n_tok, (n_tok, 2048))
    x, it, sct = hip.FromBF16Bits(xb, n_tok, 2048), hip.FromInt32(idx), hip.FromFloats(sc)
    step(f"jh_moe_swiglu repeated calls T={n_tok}")
    first = hip.Floats(hip.MoeSwiGLU(x, *st, it, sct, 64, 4, out_dtype=F32))
    assert np.isfinite(first).all()
    for _ in range(4):
        again = hip.Floats(hip.MoeSwiGLU(x, *st, it, sct, 64, 4, out_dtype=F32))
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("n_tok,E,H,I,out_dtype", [(4, 6, 512, 256, F32), (3, 5, 1024, 768, BF16),
                                                    (2, 3, 256, 512, F32)])
def test_moe_swiglu_small_with_collisions(hip, oracle, n_tok, E, H, I, out_dtype):
    """Several slots per expert, repeated experts inside one token, bf16 output."""
    K = 8
    qs = [synth.quant_linear(400 + i + H, *(I, H) if i < 2 else (H, I), lead=(E,)) for i in range(3)]
    idx = np.random.default_rng(E * H).integers(0, E, (n_tok, K)).astype(np.int32)
    sc = np.random.default_rng(E + H).random((n_tok, K)).astype(np.float32)
    step(f"jh_moe_swiglu T={n_tok} E={E} H={H} I={I} out={out_dtype}")
    got, want = _moe_case(hip, oracle, qs, (n_tok, H), idx, sc, out_dtype)
    ok, d, s = rel_ok(got, want, BF16_TOL)
    assert ok, (d, s)


def test_moe_swiglu_many_pairs_workspace_path(hip, oracle):
    """More than 1024 (token, slot) pairs: the separate bucketing launch."""
    n_tok, E, H, I, K = 160, 16, 512, 256, 8
    qs = [synth.quant_linear(500 + i, *(I, H) if i < 2 else (H, I), lead=(E,)) for i in range(3)]
    idx, sc = synth.route(510, n_tok, E, K)
    step(f"jh_moe_swiglu pairs={n_tok * K}")
    got, want = _moe_case(hip, oracle, qs, (n_tok, H), idx, sc)
    ok, d, s = rel_ok(got, want, BF16_TOL)
    assert ok, (d, s)


def test_moe_swiglu_matches_gather_composition(hip):
    """The fused operator against the reference's composition run through this
    library's GatherQuantMatmul (fp32 h there, bf16 h here)."""
    n_tok, E, H, I, K = 2, 8, 1024, 512, 4
    qs = [synth.quant_linear(600 + i, *(I, H) if i < 2 else (H, I), lead=(E,)) for i in range(3)]
    (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = _moe_upload(hip, qs)
    idx, sc = synth.route(610, n_tok, E, K)
    xb, _ = synth.activations(611, (n_tok, H))
    it = hip.FromInt32(idx)
    x4 = hip.FromBF16Bits(xb, n_tok, 1, 1, H)
    step("jh_gather_quant_matmul x3 composition vs jh_moe_swiglu")
    g = hip.Floats(hip.GatherQuantMatmul(x4, wg, sg, bg, it, True, 64, 4, out_dtype=F32)).astype(np.float64)
    u = hip.Floats(hip.GatherQuantMatmul(x4, wu, su, bu, it, True, 64, 4, out_dtype=F32)).astype(np.float64)
    h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
    d = hip.Floats(hip.GatherQuantMatmul(hip.FromFloats(h), wd, sd, bd, it, True, 64, 4, out_dtype=F32))
    want = (d[:, :, 0, :].astype(np.float64) * sc[:, :, None]).sum(axis=1)
    got = hip.Floats(hip.MoeSwiGLU(hip.FromBF16Bits(xb, n_tok, H), (wg, sg, bg), (wu, su, bu), (wd, sd, bd),
                                   it, hip.FromFloats(sc), 64, 4))
    ok, dd, s = rel_ok(got, want, BF16_TOL)
    assert ok, (dd, s)


def test_moe_swiglu_out_of_range_and_unsupported(hip, oracle):
    E, H, I = 4, 512, 256
    qs = [synth.quant_linear(700 + i, *(I, H) if i < 2 else (H, I), lead=(E,)) for i in range(3)]
    st = _moe_upload(hip, qs)
    xb, _ = synth.activations(701, (2, H))
    x = hip.FromBF16Bits(xb, 2, H)
    idx = hip.FromInt32(np.array([[0, 3], [1, 9]], np.int32))
    sc = hip.FromFloats(np.full((2, 2), 0.5, np.float32))
    step("jh_moe_swiglu bad index, checks off")
    y = hip.Floats(hip.MoeSwiGLU(x, *st, idx, sc, 64, 4))
    assert np.isfinite(y[0]).all() and np.isnan(y[1]).all()
    hip.SetChecks(True)
    try:
        step("jh_moe_swiglu bad index, checks on")
        with pytest.raises(JanisHipError):
            hip.MoeSwiGLU(x, *st, idx, sc, 64, 4)
    finally:
        hip.SetChecks(False)
    # past 32 pairs the buckets come from the bucketing launch: same NaN row, and
    # the other tokens as the oracle has them
    ids = np.random.default_rng(5).integers(0, E, (9, 4)).astype(np.int32)
    ids[6, 2] = E
    scn = np.random.default_rng(6).random((9, 4)).astype(np.float32)
    step("jh_moe_swiglu bad index, 36 pairs")
    xb9, x9 = synth.activations(702, (9, H))
    got = hip.Floats(hip.MoeSwiGLU(hip.FromBF16Bits(xb9, 9, H), *st, hip.FromInt32(ids), hip.FromFloats(scn), 64, 4,
                                   out_dtype=F32))
    assert np.isnan(got[6]).all()
    good = [t for t in range(9) if t != 6]
    want = oracle.moe_apply(x9[good], *[(q.w, q.s, q.b) for q in qs], ids[good], scn[good])
    ok, d, sc_ = rel_ok(got[good], want, BF16_TOL)  # h is bf16 between the launches
    assert ok, (d, sc_)
    step("jh_moe_swiglu no slots -> zeros")
    z = hip.Floats(hip.MoeSwiGLU(x, *st, hip.FromInt32(np.zeros((2, 0), np.int32)),
                                 hip.FromFloats(np.zeros((2, 0), np.float32)), 64, 4))
    assert z.shape == (2, H) and not z.any()
    step("jh_moe_swiglu f32 x / untiled hidden -> unsupported")
    with pytest.raises(JanisHipError):
        hip.MoeSwiGLU(hip.FromFloats(np.zeros((2, H), np.float32)), *st, idx, sc, 64, 4)
    q6 = [synth.quant_linear(710 + i, *(I, 640) if i < 2 else (640, I), lead=(E,)) for i in range(3)]
    xb6, _ = synth.activations(711, (2, 640))
    with pytest.raises(JanisHipError):
        hip.MoeSwiGLU(hip.FromBF16Bits(xb6, 2, 640), *_moe_upload(hip, q6), idx, sc, 64, 4)


# -- MoE expert MLP, one decode token ----------------------------------------------------

def _t1_stacks(hip):
    qs = [_qwen3_moe_stack(p) for p in ("gate", "up", "down")]
    if "_dev" not in _STACKS:
        _STACKS["_dev"] = _moe_upload(hip, qs)
    return qs, _STACKS["_dev"]


def _t1_call(hip, st, xb, idx, sc, out_dtype=F32):
    return hip.Floats(hip.MoeSwiGLU(hip.FromBF16Bits(xb, 1, 2048), *st, hip.FromInt32(idx), hip.FromFloats(sc),
                                    64, 4, out_dtype=out_dtype))


@pytest.mark.parametrize("k,out_dtype,collide", [(8, F32, True), (2, F32, False), (5, BF16, False),
                                                 (8, BF16, True)])
def test_moe_swiglu_one_token(hip, oracle, k, out_dtype, collide):
    """A decode token at the Qwen3-30B-A3B expert shapes: fewer slots than 8, a
    repeated expert, bf16 output, against the oracle's moeApply
    (qwen/moe.go:501-511)."""
    qs, st = _t1_stacks(hip)
    rng = np.random.default_rng(9400 + k)
    idx = rng.choice(128, k, replace=False).astype(np.int32)[None, :]
    if collide:
        idx[0, 1] = idx[0, 0]
        idx[0, k - 1] = idx[0, 0]
    sc = rng.random((1, k)).astype(np.float32)
    xb, x = synth.activations(9401 + k, (1, 2048))
    step(f"jh_moe_swiglu one token k={k} out={out_dtype} collide={collide}")
    got = _t1_call(hip, st, xb, idx, sc, out_dtype)
    want = oracle.moe_apply(x, *[(q.w, q.s, q.b) for q in qs], idx, sc)
    ok, d, s_ = rel_ok(got, want, BF16_TOL)
    assert ok, (d, s_)


def test_moe_swiglu_one_token_bad_index(hip, oracle):
    """One token over 8 slots at the Qwen3-30B-A3B shapes: an expert index
    outside [0, E) gives the token a NaN row with checks off and an error with
    checks on; the next call with good indices is the oracle's again."""
    qs, st = _t1_stacks(hip)
    idx, sc = synth.route(9450, 1, 128, 8)
    xb, x = synth.activations(9451, (1, 2048))
    bad = idx.copy()
    bad[0, 3] = 128
    step("jh_moe_swiglu one token, index 128 of 128 experts, checks off")
    assert np.isnan(_t1_call(hip, st, xb, bad, sc)).all()
    hip.SetChecks(True)
    try:
        with pytest.raises(JanisHipError):
            _t1_call(hip, st, xb, bad, sc)
    finally:
        hip.SetChecks(False)
    step("jh_moe_swiglu one token after the bad call")
    got = _t1_call(hip, st, xb, idx, sc)
    ok, d, s_ = rel_ok(got, oracle.moe_apply(x, *[(q.w, q.s, q.b) for q in qs], idx, sc), BF16_TOL)
    assert ok, (d, s_)


def test_moe_swiglu_one_token_graph_replays(hip, oracle):
    """Captured once into a HIP graph and replayed on new tokens and routes
    (written into the captured buffers between replays): every replay matches
    the oracle on its inputs, so no replay reuses an earlier call's state."""
    import ctypes

    rt = hip_runtime()
    qs, st = _t1_stacks(hip)
    xt, it, sct = hip.empty(BF16, 1, 2048), hip.empty(I32, 1, 8), hip.empty(F32, 1, 8)
    outt = hip.empty(F32, 1, 2048)

    def put(t, a):
        a = np.ascontiguousarray(a)
        hip.Sync()
        hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(t.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        hip.Sync()

    cases = []
    for i in range(3):
        idx, sc = synth.route(9800 + i, 1, 128, 8)
        xb, x = synth.activations(9810 + i, (1, 2048))
        cases.append((xb, x, idx, sc, oracle.moe_apply(x, *[(q.w, q.s, q.b) for q in qs], idx, sc)))

    def load(i):
        xb, _, idx, sc, _ = cases[i]
        put(xt, xb), put(it, idx.astype(np.int32)), put(sct, sc.astype(np.float32))

    load(0)
    hip.MoeSwiGLU(xt, *st, it, sct, 64, 4, out=outt)  # warm outside the capture
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        hip.SetStream(stream.value)
        step("capture jh_moe_swiglu (one token)")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        hip.MoeSwiGLU(xt, *st, it, sct, 64, 4, out=outt)
        assert rt.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep, i in enumerate((1, 2, 0, 1, 1)):
            step(f"graph replay {rep} on case {i}")
            load(i)
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            ok, d, s_ = rel_ok(hip.Floats(outt), cases[i][4], BF16_TOL)
            assert ok, (rep, d, s_)
    finally:
        hip.SetStream(None)
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        if graph.value:
            rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)


# -- MoE router on the device ------------------------------------------------------------

def _route_oracle(oracle, logits, k, norm):
    """MoEBlock.Forward's routing (qwen/moe.go:455-481) with the pinned oracle
    softmax and selection-sort top-k; renorm by the in-order fp32 sum when > 0."""
    n, E = logits.shape
    idx = np.empty((n, k), np.int32)
    sc = np.empty((n, k), np.float32)
    for t in range(n):
        i, v = oracle.topk(oracle.softmax_row(logits[t]), k)
        if norm:
            s = np.float32(0)
            for u in v:
                s = np.float32(s + u)
            if s > 0:
                v = (v / s).astype(np.float32)
        idx[t], sc[t] = i, v
    return idx, sc


@pytest.mark.parametrize("n,E,k,norm,kind", [(16, 128, 8, True, "normal"), (16, 128, 8, False, "normal"),
                                             (9, 128, 8, True, "ties"), (5, 60, 60, True, "ties"),
                                             (7, 257, 1, True, "normal"), (4, 64, 4, True, "bf16")])
def test_moe_route_bit_exact(hip, oracle, n, E, k, norm, kind):
    """Indices and scores identical to the CPU path, ties included (the selection
    sort's swaps decide them)."""
    rng = np.random.default_rng(n * E + k)
    if kind == "ties":
        logits = rng.integers(0, 4, (n, E)).astype(np.float32)
    else:
        logits = rng.standard_normal((n, E)).astype(np.float32)
    if kind == "bf16":
        bits = synth.f32_to_bf16_bits(logits)
        logits = synth.bf16_bits_to_f32(bits)
        t = hip.FromBF16Bits(bits, n, E)
    else:
        t = hip.FromFloats(logits)
    step(f"jh_moe_route n={n} E={E} k={k} norm={norm} {kind}")
    it, st = hip.MoeRoute(t, k, norm)
    got_i, got_s = hip.Ints(it), hip.Floats(st)
    want_i, want_s = _route_oracle(oracle, logits, k, norm)
    assert np.array_equal(got_i, want_i)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


def test_moe_block_on_device(hip, oracle):
    """A whole MoE block without a host round trip: 8-bit router QuantMatmul,
    jh_moe_route, jh_moe_swiglu, against the oracle's moeApply on the same
    routing (computed from the device logits, so near-ties cannot diverge)."""
    n_tok, E, H, I, K = 4, 16, 512, 256, 4
    qs = [synth.quant_linear(800 + i, *(I, H) if i < 2 else (H, I), lead=(E,)) for i in range(3)]
    st = [upload_quant(hip, q) for q in qs]
    rw, rs, rb = _width_case(8, E, H, 64, seed=801)
    router = _upload_width(hip, rw, rs, rb)
    xb, x = synth.activations(802, (n_tok, H))
    xt = hip.FromBF16Bits(xb, n_tok, H)
    step("router QuantMatmul (8-bit) -> jh_moe_route -> jh_moe_swiglu")
    logits = hip.QuantMatmul(xt, *router, True, 64, 8, out_dtype=F32)
    it, sct = hip.MoeRoute(logits, K, True)
    out = hip.Floats(hip.MoeSwiGLU(xt, *st, it, sct, 64, 4))
    lg = hip.Floats(logits)
    ok, d, sc = rel_ok(lg, oracle.quant_matmul(x, rw, rs, rb, 64, bits=8), F32_TOL)
    assert ok, ("router", d, sc)
    idx, scores = _route_oracle(oracle, lg, K, True)
    assert np.array_equal(hip.Ints(it), idx)
    want = oracle.moe_apply(x, *[(q.w, q.s, q.b) for q in qs], idx, scores)
    ok, d, sc = rel_ok(out, want, BF16_TOL)
    assert ok, (d, sc)


# -- other widths (2- and 8-bit: 32/bits codes per word) ----------------------------

def _width_case(bits, N, K, gs, E=None, seed=0, sb_f32=False):
    """Random packed words of `bits`-wide codes with bf16 (or f32) scales/biases."""
    rng = np.random.default_rng(seed)
    lead = () if E is None else (E,)
    P = K * bits // 32
    w = rng.integers(0, 2**32, lead + (N, P), dtype=np.uint64).astype(np.uint32)
    s = (np.abs(rng.standard_normal(lead + (N, K // gs))) * 0.02).astype(np.float32)
    b = (-(2 ** (bits - 1)) * s + rng.standard_normal(s.shape) * 1e-3).astype(np.float32)
    if not sb_f32:
        s = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(s))
        b = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(b))
    return w, s, b


def _upload_width(hip, w, s, b, sb_f32=False):
    if sb_f32:
        return hip.FromRaw(U32, w, *w.shape), hip.FromFloats(s), hip.FromFloats(b)
    return (hip.FromRaw(U32, w, *w.shape), hip.FromBF16Bits(synth.f32_to_bf16_bits(s)),
            hip.FromBF16Bits(synth.f32_to_bf16_bits(b)))


@pytest.mark.parametrize("bits,gs,sb_f32", [(8, 64, False), (8, 32, True), (2, 64, False), (2, 128, True)])
def test_dequantize_other_widths_bit_exact(hip, oracle, bits, gs, sb_f32):
    """cpu/cpu_misc.go:134-161 for any 32/bits codes per word, bit for bit."""
    N, K = 48, 1024
    w, s, b = _width_case(bits, N, K, gs, seed=bits * 100 + gs, sb_f32=sb_f32)
    tw, ts, tb = _upload_width(hip, w, s, b, sb_f32)
    step(f"jh_dequantize bits={bits} gs={gs} f32 scales={sb_f32}")
    got = hip.Floats(hip.Dequantize(tw, ts, tb, gs, bits))
    want = oracle.dequantize(w, s, b, gs, bits)
    assert got.shape == (N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    gotb = hip.Floats(hip.Dequantize(tw, ts, tb, gs, bits, out_dtype=BF16))
    np.testing.assert_array_equal(gotb, synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(want)))


@pytest.mark.parametrize("bits", [8, 2])
@pytest.mark.parametrize("rows", [1, 5])
def test_quant_matmul_other_widths(hip, oracle, bits, rows):
    """Decode (rows = 1, cpu/cpu_misc.go:350-375) and prefill (rows > 1, the wbuf
    path) at 2 and 8 bits, e.g. the 8-bit MoE router of mlx-community checkpoints
    (qwen/config.go:57-60)."""
    N, K, gs = 128, 2048, 64
    w, s, b = _width_case(bits, N, K, gs, seed=7 * bits + rows)
    tw, ts, tb = _upload_width(hip, w, s, b)
    xb, x = synth.activations(40 + bits + rows, (rows, K))
    step(f"jh_quant_matmul bits={bits} rows={rows}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, rows, K), tw, ts, tb, True, gs, bits, out_dtype=F32))
    want = oracle.quant_matmul(x, w, s, b, gs, bits=bits)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)
    yb = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, rows, K), tw, ts, tb, True, gs, bits))
    ok, d, sc = rel_ok(yb, want, BF16_TOL)
    assert ok, ("bf16 y", d, sc)


@pytest.mark.parametrize("K,gs,sb", [(128, 32, BF16), (256, 64, BF16), (384, 128, "f16"), (512, 32, BF16),
                                     (768, 64, BF16), (1024, 128, BF16), (1536, 64, "f16"), (2048, 64, BF16),
                                     (3072, 32, BF16), (4096, 64, BF16), (6144, 128, BF16), (8192, 64, "f16"),
                                     (12288, 64, BF16)])
def test_quant_matvec_8bit_tiles(hip, oracle, K, gs, sb):
    """The 8-bit register tiles (each code as two nibbles against (x, 16x), the
    4-bit word dots): every row length of the tile table (P = K/4 words), groups
    of 32/64/128, bf16 and f16 scales, a ragged row count, fp32 and bf16 y."""
    N = 517
    q = synth.quant_linear(K + gs, N, K, gs, bits=8)
    w, s, b = upload_quant(hip, q)
    sc_, bi_ = q.s, q.b
    if sb == "f16":
        sc_, bi_ = (a.astype(np.float16).astype(np.float32) for a in (q.s, q.b))
        s, b = hip.FromRaw(F16, sc_.astype(np.float16), *q.s.shape), hip.FromRaw(F16, bi_.astype(np.float16), *q.b.shape)
    xb, x = synth.activations(K + 3, (1, K))
    step(f"jh_quant_matmul 8-bit tile K={K} gs={gs} scales={sb}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, K), w, s, b, True, gs, 8, out_dtype=F32))
    want = oracle.quant_matmul(x, q.w, sc_, bi_, gs, bits=8)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)
    yb = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, K), w, s, b, True, gs, 8))
    ok, d, sc = rel_ok(yb, want, BF16_TOL)
    assert ok, ("bf16 y", d, sc)


@pytest.mark.parametrize("N,K", [(2500, 6144), (4096, 6144)])
def test_quant_matvec_8bit_pipelined_tile(hip, oracle, N, K):
    """8-bit rows of K = 6144 (1536 words, like the 4-bit K = 12288) at N >= 2048
    take the pipelined tile: a persistent grid whose blocks walk several passes
    with two register sets. N = 2500 leaves the blocks uneven pass counts."""
    q = synth.quant_linear(K + N, N, K, 64, bits=8)
    w, s, b = upload_quant(hip, q)
    xb, x = synth.activations(K + 5, (1, K))
    step(f"jh_quant_matmul 8-bit pipelined tile N={N} K={K}")
    y = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, K), w, s, b, True, 64, 8, out_dtype=F32))
    want = oracle.quant_matmul(x, q.w, q.s, q.b, 64, bits=8)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)


def test_gather_8bit(hip, oracle):
    E, N, K, gs, T, Kk = 5, 64, 512, 64, 3, 4
    w, s, b = _width_case(8, N, K, gs, E=E, seed=99)
    tw, ts, tb = _upload_width(hip, w, s, b)
    idx = np.random.default_rng(98).integers(0, E, (T, Kk)).astype(np.int32)
    xb, x = synth.activations(97, (T, 1, 1, K))
    step("jh_gather_quant_matmul bits=8")
    y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, T, 1, 1, K), tw, ts, tb, hip.FromInt32(idx),
                                         True, gs, 8, out_dtype=F32))
    want = oracle.gather_quant_matmul(x, w, s, b, idx, gs, bits=8)
    ok, d, sc = rel_ok(y, want, F32_TOL)
    assert ok, (d, sc)


# -- errors (the reference panics) ---------------------------------------------------

def test_bad_arguments_raise(hip):
    q = synth.quant_linear(1, 16, 256)
    w, s, b = upload_quant(hip, q)
    xb, _ = synth.activations(1, (1, 256))
    x = hip.FromBF16Bits(xb, 1, 256)
    with pytest.raises(JanisHipError):  # 3-bit codes do not divide a word
        hip.Dequantize(w, s, b, 64, 3)
    with pytest.raises(JanisHipError):  # transpose=false takes x of out_features (16) features
        hip.QuantMatmul(x, w, s, b, False, 64, 4)
    with pytest.raises(JanisHipError):  # group does not divide K
        hip.QuantMatmul(x, w, s, b, True, 96, 4)
    with pytest.raises(JanisHipError):  # feature mismatch
        hip.QuantMatmul(hip.FromBF16Bits(np.zeros((1, 128), np.uint16)), w, s, b, True, 64, 4)
