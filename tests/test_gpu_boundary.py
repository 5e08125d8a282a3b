"""The rest of the engine boundary around the quantized products, on the GPU
through the C ABI: QuantMatmul / GatherQuantMatmul with transpose=false, the
Softmax / Mean / ScalarMul / ScalarAdd that MoEBlock.Forward calls
(qwen/moe.go:458-510), that MoE block made call for call, workspace growth
under captured graphs, and the failure paths (out of memory, NaN scales, the
NaN/Inf read-back checks of ggml/ggml.go:622-677).

Operators whose CPU order is sequential are compared bit for bit with the
oracle (fp32 outputs); compositions through bf16 products within the relOK bar.
"""
import numpy as np
import pytest

from janis_amd import _lib, synth
from janis_amd.engine import BF16, F32, U8, HipBackend, JanisHipError
from tests.conftest import Graph, hip_runtime, put, rel_ok, step, upload_quant

pytestmark = pytest.mark.gpu

F32_TOL = 1e-3
# the prefill GEMM feeds the MFMAs bf16-rounded dequantized weights, so its fp32
# outputs carry ~2^-9 relative rounding per weight (the bar used for that path
# in test_gpu_parity.py)
QMM_F32_TOL = 5e-3
BF16_TOL = 1e-2


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _x(hip, rng_seed, shape, dt, zero_every=0):
    """Seeded activations as a device tensor of dtype dt and their fp32 values
    (bf16-exact either way), with every zero_every-th column set to 0."""
    xb, x = synth.activations(rng_seed, shape)
    if zero_every:
        xb[..., ::zero_every] = 0
        x = synth.bf16_bits_to_f32(xb)
    t = hip.FromBF16Bits(xb, *shape) if dt == BF16 else hip.FromFloats(x, *shape)
    return t, x


# -- transpose=false: MatMul(x, Dequantize(w)) (cpu/cpu_misc.go:233-236) ----------------

@pytest.mark.parametrize("rows,n,k,gs,bits,xdt", [
    (1, 256, 512, 64, 4, F32), (3, 96, 256, 32, 4, BF16), (2, 64, 128, 64, 8, F32),
    (1, 40, 64, 16, 2, F32), (5, 128, 1024, 128, 4, BF16), (2, 24, 16, 8, 4, F32)])
def test_quant_matmul_transpose_false_bit_exact(hip, oracle, rows, n, k, gs, bits, xdt):
    """y [rows, k] = x [rows, n] . Dequantize(W [n, k]) with the CPU backend's
    order (increasing n, zero x skipped, rounded product then add): fp32
    results equal the oracle bit for bit; a NaN scale in a row whose x is 0 is
    skipped as the CPU backend skips it."""
    q = synth.quant_linear(700 + n + k, n, k, gs, bits=bits)
    nan_row = n // 3
    q.s_bits[nan_row, 0] = 0x7FC0  # NaN scale, multiplied only by x == 0 below
    xt, x = _x(hip, 701 + rows, (rows, n), xdt, zero_every=7)
    if nan_row % 7:
        xb = synth.f32_to_bf16_bits(x)
        xb[:, nan_row] = 0
        x = synth.bf16_bits_to_f32(xb)
        xt = hip.FromBF16Bits(xb, rows, n) if xdt == BF16 else hip.FromFloats(x, rows, n)
    w, s, b = upload_quant(hip, q)
    step(f"jh_quant_matmul transpose=0 rows={rows} N={n} K={k} gs={gs} bits={bits}")
    y = hip.Floats(hip.QuantMatmul(xt, w, s, b, False, gs, bits, out_dtype=F32))
    want = oracle.matmul_dequant(x, q.w, q.s, q.b, gs, bits)
    assert y.shape == (rows, k)
    assert np.isfinite(want).all()
    assert _bits_equal(y, want)
    yb = hip.Floats(hip.QuantMatmul(xt, w, s, b, False, gs, bits, out_dtype=BF16))
    ok, d, sc = rel_ok(yb, want, BF16_TOL)
    assert ok, (d, sc)


@pytest.mark.parametrize("A,n,k", [(1, 64, 64), (4, 64, 64), (4, 96, 256)])
def test_gather_transpose_false_bit_exact(hip, oracle, A, n, k):
    """Each slot is its expert's transposed product (cpu/cpu_misc.go:224 with
    :233-236): x [lead, A, 1, n] -> y [lead, K, 1, k], bit-exact fp32; an
    out-of-range expert index gives that slot a row of NaN."""
    E, lead, K = 5, 3, 4
    q = synth.quant_linear(720 + A + k, n, k, 32, lead=(E,))
    idx = np.random.default_rng(A).integers(0, E, (lead, K)).astype(np.int32)
    idx[0, 0] = idx[0, 1]  # two slots of one token on one expert
    xt, x = _x(hip, 721 + A, (lead, A, 1, n), F32)
    w, s, b = upload_quant(hip, q)
    step(f"jh_gather_quant_matmul transpose=0 A={A} n={n} k={k}")
    y = hip.Floats(hip.GatherQuantMatmul(xt, w, s, b, hip.FromInt32(idx, lead, K), False, 32, 4, out_dtype=F32))
    want = oracle.gather_matmul_dequant(x.reshape(lead, A, n), q.w, q.s, q.b, idx, 32)
    assert y.shape == (lead, K, 1, k)
    assert _bits_equal(y.reshape(lead, K, k), want)
    bad = idx.copy()
    bad[1, 2] = E + 3
    y = hip.Floats(hip.GatherQuantMatmul(xt, w, s, b, hip.FromInt32(bad, lead, K), False, 32, 4, out_dtype=F32))
    assert np.isnan(y[1, 2]).all()
    mask = np.ones((lead, K), bool)
    mask[1, 2] = False
    assert _bits_equal(y.reshape(lead, K, k)[mask], want[mask])


# -- Softmax, Mean, ScalarMul/ScalarAdd ---------------------------------------------------

@pytest.mark.parametrize("shape,axis,dt", [((16, 128), -1, F32), ((5, 60), -1, BF16), ((3, 7, 5), 1, F32),
                                           ((4, 3), 0, F32), ((2, 8192), -1, F32)])
def test_softmax_bit_exact(hip, oracle, shape, axis, dt):
    """Backend.Softmax (cpu/cpu.go:461-499): the CPU backend's max, double exp,
    sequential fp32 sum and fp32 division, bit for bit, along any axis."""
    xt, x = _x(hip, 730 + len(shape), shape, dt)
    step(f"jh_softmax shape={shape} axis={axis}")
    got = hip.Floats(hip.Softmax(xt, axis))
    assert _bits_equal(got, oracle.softmax(x, axis))


def test_softmax_long_line(hip):
    """Lines beyond 8192 sum in a tree: within a few ulp of the float64 softmax."""
    xt, x = _x(hip, 739, (2, 20000), F32)
    step("jh_softmax 2 x 20000 (tree sum)")
    got = hip.Floats(hip.Softmax(xt, -1))
    e = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    want = e / e.sum(-1, keepdims=True)
    assert np.max(np.abs(got - want) / want) < 1e-5


@pytest.mark.parametrize("shape,axis", [((16, 8, 2048), 1), ((5, 33), 0), ((7, 3, 4), -1), ((1, 6, 8, 64), 2)])
def test_mean_bit_exact(hip, oracle, shape, axis):
    """Backend.Mean (cpu/cpu_ops.go:113-142): sequential fp32 sum along the
    axis, then / len, bit for bit; the axis is removed."""
    xt, x = _x(hip, 740 + len(shape), shape, F32)
    step(f"jh_mean shape={shape} axis={axis}")
    got = hip.Floats(hip.Mean(xt, axis))
    want = oracle.mean(x, axis)
    assert got.shape == want.shape
    assert _bits_equal(got, want)
    # the order matters: 1e8 + 1 rounds back to 1e8 in fp32
    t = hip.FromFloats(np.array([1e8, 1, -1e8, 1], np.float32), 1, 4)
    assert hip.Floats(hip.Mean(t, 1))[0] == np.float32(0.25)


def test_scalar_ops_bit_exact(hip, oracle):
    xt, x = _x(hip, 750, (3, 1000), F32)
    step("jh_scalar mul/add")
    assert _bits_equal(hip.Floats(hip.ScalarMul(xt, 8.0)), oracle.scalar_mul(x, 8.0))
    assert _bits_equal(hip.Floats(hip.ScalarMul(xt, 0.1)), oracle.scalar_mul(x, 0.1))
    assert _bits_equal(hip.Floats(hip.ScalarAdd(xt, -2.5)), oracle.scalar_add(x, -2.5))
    bt, xb = _x(hip, 751, (3, 1000), BF16)
    assert _bits_equal(hip.Floats(hip.ScalarMul(bt, 3.0, out_dtype=F32)), oracle.scalar_mul(xb, 3.0))


def test_broadcast_mul_matches_numpy(hip):
    """Mul with a [.., K, 1] operand against [.., K, H] (the score weighting of
    qwen/moe.go:510) broadcasts like the CPU backend's elementwise ops."""
    at, a = _x(hip, 752, (1, 3, 4, 16), F32)
    bt, b = _x(hip, 753, (1, 3, 4, 1), F32)
    step("broadcast Mul")
    assert _bits_equal(hip.Floats(hip.Mul(at, bt)), (a * b).astype(np.float32))
    assert _bits_equal(hip.Floats(hip.Add(bt, at)), (a + b).astype(np.float32))


# -- MoEBlock.Forward as the model code writes it -------------------------------------------

def test_moe_block_reference_calls(hip, oracle):
    """MoEBlock.Forward (qwen/moe.go:448-510, resident stacks indexed by global
    expert id) made call for call on this backend: router QuantMatmul, Softmax,
    Floats, host top-k + NormTopk, FromInt32, ExpandDims twice, three
    GatherQuantMatmuls, SiLU, Mul, Reshape, FromFloats, broadcast Mul, Mean,
    ScalarMul. Softmax is checked bit for bit against the oracle on the same
    logits, and the block's output against or_moe_apply on the same routes."""
    E, H, I, K, n_tok = 32, 1024, 512, 8, 5
    router = synth.quant_linear(760, E, H, 64)
    gate = synth.quant_linear(761, I, H, 64, lead=(E,))
    up = synth.quant_linear(762, I, H, 64, lead=(E,))
    down = synth.quant_linear(763, H, I, 64, lead=(E,))
    wr, sr, br = upload_quant(hip, router)
    stacks = [upload_quant(hip, q) for q in (gate, up, down)]
    xt, x = _x(hip, 764, (1, n_tok, H), F32)  # [..lead.., hidden], lead [1, seq]
    step("MoEBlock.Forward call for call")
    logits = hip.QuantMatmul(xt, wr, sr, br, True, 64, 4)
    probs = hip.Softmax(logits, -1)
    pf = hip.Floats(probs).reshape(n_tok, E)
    assert _bits_equal(pf, oracle.softmax(hip.Floats(logits).reshape(n_tok, E), -1))
    ri = np.empty((n_tok, K), np.int32)
    scores = np.empty((n_tok, K), np.float32)
    for t in range(n_tok):
        i, sc = oracle.topk(pf[t], K)
        s = np.float32(0)
        for v in sc:
            s = np.float32(s + v)
        if s > 0:
            sc = (sc / s).astype(np.float32)
        ri[t], scores[t] = i, sc
    nd = 3
    ridx = hip.FromInt32(ri, 1, n_tok, K)
    xe = hip.ExpandDims(hip.ExpandDims(xt, nd - 1), nd - 1)
    g = hip.GatherQuantMatmul(xe, *stacks[0], ridx, True, 64, 4)
    u = hip.GatherQuantMatmul(xe, *stacks[1], ridx, True, 64, 4)
    hh = hip.Mul(hip.SiLU(g), u)
    d = hip.GatherQuantMatmul(hh, *stacks[2], ridx, True, 64, 4)
    d2 = hip.Reshape(d, 1, n_tok, K, H)
    scT = hip.FromFloats(scores, 1, n_tok, K, 1)
    out = hip.ScalarMul(hip.Mean(hip.Mul(d2, scT), nd - 1), float(K))
    got = hip.Floats(out)
    assert got.shape == (1, n_tok, H)
    want = oracle.moe_apply(x[0], *[(q.w, q.s, q.b) for q in (gate, up, down)], ri, scores)
    ok, dd, sc = rel_ok(got[0], want, F32_TOL)
    assert ok, (dd, sc)


# -- workspace growth and captured graphs ---------------------------------------------------

def test_graph_survives_workspace_growth(oracle):
    """A graph captured after its warm-up call keeps the workspace it was
    captured with: a later call that grows the context's workspace (a larger
    split-K prefill) retires the old buffer instead of freeing it, so replays
    stay bit-identical to the eager call and memory allocated after the growth
    is never written by them. Growth during a capture is refused."""
    import ctypes

    hip = HipBackend(0)  # a fresh context: its workspace starts empty
    try:
        q = synth.quant_linear(780, 4096, 4096)
        w, s, b = upload_quant(hip, q)
        xs = [synth.activations(781 + i, (16, 4096)) for i in range(2)]
        xt, yt = hip.empty(BF16, 16, 4096), hip.empty(F32, 16, 4096)
        put(hip, xt, xs[0][0])
        # 16 rows split K (partials in the workspace): capturing the first such
        # call, with no workspace yet, is refused with a clear error
        rt = hip_runtime()
        stream, graph = ctypes.c_void_p(), ctypes.c_void_p()
        assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
        hip.SetStream(stream.value)
        step("capture before any warm-up call: workspace growth refused")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        err = None
        try:
            hip.QuantMatmul(xt, w, s, b, True, 64, 4, out=yt)
        except JanisHipError as e:
            err = e
        rt.hipStreamEndCapture(stream, ctypes.byref(graph))
        hip.SetStream(None)
        if graph.value:
            rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)
        assert err is not None and err.code == _lib.JH_ERR_INVALID and "captured" in str(err), err
        eager = []
        for xb, _ in xs:
            put(hip, xt, xb)
            hip.QuantMatmul(xt, w, s, b, True, 64, 4, out=yt)
            eager.append(hip.Floats(yt))
        ok, d, sc = rel_ok(eager[1][:, :64], oracle.quant_matmul(xs[1][1], q.w[:64], q.s[:64], q.b[:64], 64),
                           QMM_F32_TOL)
        assert ok, (d, sc)
        step("capture a split-K jh_quant_matmul (16 rows)")
        g = Graph(hip, lambda: hip.QuantMatmul(xt, w, s, b, True, 64, 4, out=yt))
        try:
            for i in (1, 0):
                put(hip, xt, xs[i][0])
                g.replay()
                assert _bits_equal(hip.Floats(yt), eager[i])
            # grow: 128 rows of a 12288-row matrix split K over a larger partial buffer
            big = synth.quant_linear(782, 12288, 4096)
            wb, sb, bb = upload_quant(hip, big)
            xbb, xbig = synth.activations(783, (128, 4096))
            step("grow the workspace: jh_quant_matmul 128 x 12288 x 4096")
            ybig = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xbb, 128, 4096), wb, sb, bb, True, 64, 4,
                                              out_dtype=F32))
            cs = np.arange(0, 12288, 997)
            ok, d, sc = rel_ok(ybig[:16][:, cs], oracle.quant_matmul(xbig[:16], big.w[cs], big.s[cs], big.b[cs], 64),
                               QMM_F32_TOL)
            assert ok, (d, sc)
            # fresh allocations of the old workspace's size, filled with a pattern
            junk = [hip.empty(U8, 4 << 20) for _ in range(8)]
            pattern = np.full(4 << 20, 0xA5, np.uint8)
            for t in junk:
                put(hip, t, pattern)
            for i in (0, 1):
                step(f"graph replay after growth on x {i}")
                put(hip, xt, xs[i][0])
                g.replay()
                assert _bits_equal(hip.Floats(yt), eager[i])
            for t in junk:
                assert np.array_equal(np.frombuffer(hip.Bytes(t), np.uint8), pattern)
        finally:
            g.close()
    finally:
        hip.Close()


def test_decode_step_graph_survives_workspace_growth(oracle):
    """The fused decode step of a small Qwen3 captured into a graph at
    position 300 (its attention splits the keys and uses the workspace), then
    a larger prefill call grows the workspace, then the graph is replayed: the
    logits equal the eager step's bit for bit before and after."""
    from janis_amd.qwen3_decode import Qwen3Config, decode_step, random_model

    hip = HipBackend(0)
    try:
        cfg = Qwen3Config(hidden=512, inter=1024, n_heads=4, n_kv=2, head_dim=128, vocab=1000, layers=2)
        m, _ = random_model(hip, cfg, 512, seed=7)
        for L in m.layers:  # seeded N(0,1) keys and values in every row
            for c, sd in ((L.k_cache, 1), (L.v_cache, 2)):
                put(hip, c, synth.f32_to_bf16_bits(synth.normal(790 + sd, c.numel).astype(np.float32)))
        tok = hip.FromInt32(np.array([17], np.int32))
        arena = hip.make_arena(8 << 20)
        pos = 300

        def run():
            with hip.use_arena(arena):
                return decode_step(hip, m, tok, pos)

        step("eager fused decode step at pos 300")
        logits, _ = run()
        eager = hip.Floats(logits).copy()
        g = Graph(hip, run)
        try:
            g.replay()
            assert _bits_equal(hip.Floats(logits), eager)
            big = synth.quant_linear(791, 12288, 4096)
            wb, sb, bb = upload_quant(hip, big)
            xbb, _ = synth.activations(792, (128, 4096))
            step("grow the workspace with a prefill call, then replay")
            hip.QuantMatmul(hip.FromBF16Bits(xbb, 128, 4096), wb, sb, bb, True, 64, 4, out_dtype=F32)
            hip.Sync()
            for _ in range(2):
                g.replay()
                assert _bits_equal(hip.Floats(logits), eager)
        finally:
            g.close()
    finally:
        hip.Close()


# -- failure paths -----------------------------------------------------------------------

def test_out_of_memory_status(hip):
    """jh_alloc and workspace growth asked for more than the device holds return
    JH_ERR_OOM (the reference panics on OOM, ggml/ggml.go:610-614), and the
    context keeps working afterwards."""

    step("jh_alloc 1 TiB")
    with pytest.raises(JanisHipError) as e:
        hip.empty(U8, 1 << 40)
    assert e.value.code == _lib.JH_ERR_OOM
    # a gather of 64 slots over a stack that claims 2^37 experts: its bucketing
    # workspace (4 bytes per expert and slot) is about 1 TiB; no kernel runs
    q = synth.quant_linear(800, 64, 256, lead=(2,))
    w, s, b = upload_quant(hip, q)
    x = hip.FromBF16Bits(synth.activations(801, (16, 1, 256))[0], 16, 1, 256)
    idx = hip.FromInt32(np.zeros((16, 4), np.int32), 16, 4)
    y = hip.empty(BF16, 16, 4, 64)
    step("jh_gather_quant_matmul whose workspace cannot be allocated")
    rc = hip._L.jh_gather_quant_matmul(hip._ctx, x.ptr, BF16, 16, 1, w.ptr, s.ptr, b.ptr, BF16, 1 << 37, 64, 256,
                                       idx.ptr, 4, 1, 64, 4, y.ptr, BF16)
    assert rc == _lib.JH_ERR_OOM, rc
    assert b"workspace" in hip._L.jh_last_error(hip._ctx)
    # still usable
    xb, xf = synth.activations(802, (1, 256))
    got = hip.Floats(hip.QuantMatmul(hip.FromBF16Bits(xb, 1, 256), w, s, b, True, 64, 4, out_dtype=F32))
    assert got.shape == (1, 64) and np.isfinite(got).all()


@pytest.mark.parametrize("rows", [1, 4, 128])
def test_nan_scale_propagates(hip, oracle, rows):
    """A NaN scale poisons exactly its output row, as in the CPU backend
    (s * sum(x q) is NaN there too): the decode GEMV, the multi-row tile and
    the prefill GEMM all give NaN in that column and the oracle's values
    elsewhere. With JH_CHECK_VALUES the product reports JH_ERR_NONFINITE with
    the count and the first index; jh_check_finite counts the same."""
    n, k, r0 = 512, 4096, 37
    q = synth.quant_linear(810, n, k)
    q.s_bits[r0, 5] = 0x7FC0
    w, s, b = upload_quant(hip, q)
    xb, x = synth.activations(811 + rows, (rows, k))
    xt = hip.FromBF16Bits(xb, rows, k)
    step(f"NaN scale, jh_quant_matmul rows={rows}")
    y = hip.Floats(hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=F32))
    assert np.isnan(y[:, r0]).all()
    others = np.setdiff1d(np.arange(n), [r0])
    assert np.isfinite(y[:, others]).all()
    cs = others[::5]
    ok, d, sc = rel_ok(y[:, cs], oracle.quant_matmul(x, q.w[cs], q.s[cs], q.b[cs], 64),
                       QMM_F32_TOL if rows > 8 else F32_TOL)
    assert ok, (d, sc)
    yt = hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=F32)
    assert hip.CheckFinite(yt) == (rows, r0)
    hip.SetChecks(_lib.JH_CHECK_VALUES)
    try:
        with pytest.raises(JanisHipError) as e:
            hip.QuantMatmul(xt, w, s, b, True, 64, 4, out_dtype=F32)
        assert e.value.code == _lib.JH_ERR_NONFINITE
        assert f"{rows} of {rows * n}" in str(e.value) and f"index {r0}" in str(e.value), str(e.value)
        # a clean product passes with the checks on
        q2 = synth.quant_linear(812, n, k)
        w2, s2, b2 = upload_quant(hip, q2)
        hip.QuantMatmul(xt, w2, s2, b2, True, 64, 4, out_dtype=F32)
    finally:
        hip.SetChecks(0)


def test_value_checks_on_decode_operators(hip):
    """JH_CHECK_VALUES covers the other float operators too (here RMSNorm and
    Softmax fed an Inf), and refuses a stream under capture."""
    x = np.ones((2, 64), np.float32)
    x[1, 3] = np.inf
    xt = hip.FromFloats(x, 2, 64)
    wt = hip.FromFloats(np.ones(64, np.float32), 64)
    hip.SetChecks(_lib.JH_CHECK_VALUES | _lib.JH_CHECK_INDICES)
    try:
        step("value checks: RMSNorm, Softmax with an Inf input")
        with pytest.raises(JanisHipError) as e:
            hip.RMSNorm(xt, wt, 1e-6)
        assert e.value.code == _lib.JH_ERR_NONFINITE and "jh_rms_norm" in str(e.value)
        with pytest.raises(JanisHipError) as e:
            hip.Softmax(xt, -1)
        assert e.value.code == _lib.JH_ERR_NONFINITE
        ok = hip.Softmax(hip.FromFloats(np.ones((2, 64), np.float32), 2, 64), -1)
        assert np.allclose(hip.Floats(ok), 1 / 64)
    finally:
        hip.SetChecks(0)
    with pytest.raises(JanisHipError):
        hip.SetChecks(8)  # unknown flag
