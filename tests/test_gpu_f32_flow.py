"""The dtype flow unchanged janis model code produces on this backend, operator
by operator, through the C ABI: fp32 activations into the quantized products
(Dequantize returns F32 and every operator keeps its input's dtype,
cpu/cpu_misc.go:257-276 takes fp32 x), and f16 KV caches (KVCache.Update casts
F32 keys and values to F16 on a RawReader backend, qwen/cache.go:90-93).

Bars: an fp32-x product has the bits of the bf16-x product on bf16(x) (the
tiles round x in registers) and is within 1e-2 of max|y| of the oracle's fp32-x
product; f16 cache appends are the IEEE nearest-even conversion; attention over
f16 caches within 1e-3 of the oracle (as over bf16 ones) and bit for bit the
composition of the backend's own operators. Also here: the fused launch's
bounded wait failing loudly, and the value checks of the no-allocation entry.
"""
import numpy as np
import pytest

from janis_amd import _lib, synth
from janis_amd.engine import BF16, F16, F32, U32, JanisHipError
from tests.conftest import rel_ok, step, upload_quant

pytestmark = pytest.mark.gpu


def _bf16(a):
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.asarray(a, np.float32)))


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _put(hip, a, dt):
    a = np.asarray(a, np.float32)
    if dt == BF16:
        return hip.FromBF16Bits(synth.f32_to_bf16_bits(a), *a.shape)
    if dt == F16:
        return hip.FromRaw(F16, a.astype(np.float16), *a.shape)
    return hip.FromFloats(a, *a.shape)


def _weights(hip, q, sb):
    w = hip.FromRaw(U32, q.w, *q.w.shape)
    if sb == "f16":
        s_np, b_np = (v.astype(np.float16).astype(np.float32) for v in (q.s, q.b))
        s, b = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape), hip.FromRaw(F16, q.b.astype(np.float16),
                                                                                *q.b.shape)
        return (w, s, b), s_np, b_np
    return upload_quant(hip, q), q.s, q.b


# every row length of the decode tiles (4-bit K = 8 x words; 8-bit K = 4 x words)
@pytest.mark.parametrize("n,k,gs,bits,sb", [
    (4096, 4096, 64, 4, "bf16"), (1024, 4096, 64, 4, "bf16"), (6144, 4096, 64, 4, "f16"),
    (4096, 12288, 64, 4, "bf16"), (1000, 12288, 64, 4, "bf16"), (300, 8192, 128, 4, "bf16"),
    (257, 16384, 64, 4, "bf16"), (500, 2048, 32, 4, "f16"), (700, 6144, 64, 4, "bf16"),
    (130, 1024, 64, 4, "bf16"), (90, 3072, 64, 4, "bf16"), (64, 512, 32, 4, "bf16"),
    (33, 1536, 64, 4, "bf16"), (20, 256, 32, 4, "bf16"), (17, 768, 64, 4, "bf16"),
    (151936, 4096, 64, 4, "bf16"), (2048, 4096, 64, 8, "bf16"), (600, 12288, 64, 8, "bf16"),
    (1000, 2048, 64, 8, "f16"), (100, 1000, 40, 4, "bf16"),
])
def test_f32_x_takes_the_tiles(hip, oracle, n, k, gs, bits, sb):
    """QuantMatmul with fp32 x (one row): the bits of the same call with bf16 x
    = bf16(x), on every tile row length (the last case is outside the tiles:
    the generic kernel multiplies fp32 x unrounded, checked against the oracle
    only), and within the bar of the oracle's fp32-x product."""
    q = synth.quant_linear(21000 + n + k + bits, n, k, gs, bits=bits)
    (w, s, b), s_np, b_np = _weights(hip, q, sb)
    x = (1.5 * np.random.default_rng(n + k).standard_normal((1, k))).astype(np.float32)
    step(f"jh_quant_matmul fp32 x N={n} K={k} gs={gs} bits={bits} sb={sb}")
    y32 = hip.Floats(hip.QuantMatmul(hip.FromFloats(x), w, s, b, True, gs, bits))
    tiles = not (k == 1000)
    if tiles:
        yb = hip.Floats(hip.QuantMatmul(_put(hip, x, BF16), w, s, b, True, gs, bits, out_dtype=F32))
        assert np.array_equal(y32.view(np.uint32), yb.view(np.uint32))
    rows = np.sort(np.random.default_rng(k).choice(n, size=min(n, 128), replace=False))
    want = oracle.quant_matmul(x, q.w[rows], s_np[rows], b_np[rows], gs, bits)
    ok, d, sc = rel_ok(y32[:, rows], want, 1e-2)
    assert ok, (d, sc)


@pytest.mark.parametrize("n,k,rows,sb", [(4096, 4096, 2, "bf16"), (2048, 4096, 7, "f16"), (1300, 12288, 3, "bf16"),
                                         (1000, 24576, 2, "bf16"), (24576, 4096, 4, "bf16")])
def test_f32_x_rows_match_one_row_calls(hip, oracle, n, k, rows, sb):
    """fp32 rows the multi-row tile takes (2 rows; up to 8 below 2^24 weights):
    each row has the bits of a one-row fp32 call and of the bf16 multi-row call
    on bf16(x)."""
    gs = 64
    q = synth.quant_linear(22000 + n + k, n, k, gs)
    (w, s, b), s_np, b_np = _weights(hip, q, sb)
    x = np.random.default_rng(rows * k).standard_normal((rows, k)).astype(np.float32)
    step(f"jh_quant_matmul fp32 rows={rows} N={n} K={k} sb={sb}")
    y = hip.Floats(hip.QuantMatmul(hip.FromFloats(x), w, s, b, True, gs, 4))
    yb = hip.Floats(hip.QuantMatmul(_put(hip, x, BF16), w, s, b, True, gs, 4, out_dtype=F32))
    assert np.array_equal(y.view(np.uint32), yb.view(np.uint32))
    for r in range(rows):
        y1 = hip.Floats(hip.QuantMatmul(hip.FromFloats(x[r:r + 1]), w, s, b, True, gs, 4))
        assert np.array_equal(y[r].view(np.uint32), y1[0].view(np.uint32)), r
    cs = np.sort(np.random.default_rng(n).choice(n, size=96, replace=False))
    ok, d, sc = rel_ok(y[:, cs], oracle.quant_matmul(x, q.w[cs], s_np[cs], b_np[cs], gs), 1e-2)
    assert ok, (d, sc)


def test_kv_append_f16(hip):
    """f16 caches: f16, bf16 and fp32 rows appended are the nearest-even f16 values."""
    rng = np.random.default_rng(31)
    B, Hk, cap, Dh = 1, 8, 64, 128
    kc, vc = hip.empty(F16, B, Hk, cap, Dh), hip.empty(F16, B, Hk, cap, Dh)
    k0, v0 = _f16(rng.standard_normal((B, Hk, 10, Dh))), _f16(rng.standard_normal((B, Hk, 10, Dh)))
    k1, v1 = (3.0 * rng.standard_normal((B, Hk, 1, Dh))).astype(np.float32), rng.standard_normal((B, Hk, 1, Dh))
    k2 = _bf16(rng.standard_normal((B, Hk, 2, Dh)))
    step("jh_kv_append into f16 caches")
    hip.AppendKVRows(kc, vc, 0, _put(hip, k0, F16), _put(hip, v0, F16))
    hip.AppendKVRows(kc, vc, 10, _put(hip, k1, F32), _put(hip, v1, F32))
    hip.AppendKVRows(kc, vc, 11, _put(hip, k2, BF16), _put(hip, k2, BF16))
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    assert np.array_equal(gk[:, :, :10], k0) and np.array_equal(gv[:, :, :10], v0)
    assert np.array_equal(gk[:, :, 10:11], _f16(k1)) and np.array_equal(gv[:, :, 10:11], _f16(v1))
    assert np.array_equal(gk[:, :, 11:13], _f16(k2))
    # the mirror's Cast + AppendKV, as KVCache.Update makes them
    k3 = rng.standard_normal((B, Hk, 1, Dh)).astype(np.float32)
    buf, view = hip.AppendKV(kc, hip.Slice(kc, 2, 0, 13), 13, hip.Cast(hip.FromFloats(k3), F16))
    assert view.shape == (B, Hk, 14, Dh) and view.dtype == F16
    assert np.array_equal(hip.Floats(kc)[:, :, 13:14], _f16(k3))


@pytest.mark.parametrize("Lk,q_dt", [(1, F32), (100, F32), (512, F32), (8192, BF16)])
def test_sdpa_decode_f16_cache(hip, oracle, Lk, q_dt):
    """One query row per head over f16 caches with spare capacity (the
    split-over-keys kernel), fp32 or bf16 q."""
    B, Hq, Hk, Dh, cap = 1, 32, 8, 128, Lk + 37
    rng = np.random.default_rng(Lk + 5)
    q = rng.standard_normal((B, Hq, 1, Dh)).astype(np.float32)
    if q_dt == BF16:
        q = _bf16(q)
    k, v = _f16(rng.standard_normal((B, Hk, cap, Dh))), _f16(rng.standard_normal((B, Hk, cap, Dh)))
    step(f"jh_sdpa decode f16 cache Lk={Lk}")
    got = hip.Floats(hip.SDPA(_put(hip, q, q_dt), _put(hip, k, F16), _put(hip, v, F16), Dh ** -0.5, False,
                              kv_len=Lk, out_dtype=F32))
    ok, dd, sc = rel_ok(got, oracle.sdpa(q, k[:, :, :Lk], v[:, :, :Lk], Dh ** -0.5, False), 1e-3)
    assert ok, (dd, sc)


def test_sdpa_rows_f16_cache(hip, oracle):
    """Prefill-shaped SDPA (the per-row kernel) over f16 k/v with the causal mask."""
    rng = np.random.default_rng(77)
    q = rng.standard_normal((1, 8, 5, 128)).astype(np.float32)
    k, v = _f16(rng.standard_normal((1, 2, 13, 128))), _f16(rng.standard_normal((1, 2, 13, 128)))
    step("jh_sdpa rows f16 cache")
    got = hip.Floats(hip.SDPA(_put(hip, q, F32), _put(hip, k, F16), _put(hip, v, F16), 128 ** -0.5, True))
    ok, dd, sc = rel_ok(got, oracle.sdpa(q, k, v, 128 ** -0.5, True), 1e-4)
    assert ok, (dd, sc)


def _attention_oracle_f16(oracle, qkv, qn, kn, k_old, v_old, Hq, Hk, pos, scale):
    Dh = 128
    qh = qkv[0, :Hq * Dh].reshape(1, Hq, 1, Dh)
    kh = qkv[0, Hq * Dh:(Hq + Hk) * Dh].reshape(1, Hk, 1, Dh)
    vh = qkv[0, (Hq + Hk) * Dh:].reshape(1, Hk, 1, Dh)
    qh, kh = oracle.rms_norm(qh, qn, 1e-6), oracle.rms_norm(kh, kn, 1e-6)
    q = oracle.rope(qh, Dh, False, 1e6, 1.0, pos)
    kc, vc = k_old.copy(), v_old.copy()
    kc[:, :, pos:pos + 1], vc[:, :, pos:pos + 1] = _f16(oracle.rope(kh, Dh, False, 1e6, 1.0, pos)), _f16(vh)
    return oracle.sdpa(q, kc[:, :, :pos + 1], vc[:, :, :pos + 1], scale, False).reshape(1, Hq * Dh), kc, vc


@pytest.mark.parametrize("Hq,Hk,pos", [(32, 8, 0), (32, 8, 15), (32, 8, 512), (32, 8, 3000), (16, 8, 700),
                                       (32, 4, 600)])
def test_attention_decode_f16_cache(hip, oracle, Hq, Hk, pos):
    """jh_attention_decode over f16 caches: against the oracle over the updated
    cache, and against the backend's own QKNormRoPEAppend + SDPA; the new rows
    written are the f16 key and value, the other rows untouched."""
    rng = np.random.default_rng(Hq * 1000 + pos + 3)
    Dh, cap = 128, pos + 9
    scale = Dh ** -0.5
    qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
    qn, kn = _bf16(1 + 0.1 * rng.standard_normal(Dh)), _bf16(1 + 0.1 * rng.standard_normal(Dh))
    k_old, v_old = _f16(rng.standard_normal((1, Hk, cap, Dh))), _f16(rng.standard_normal((1, Hk, cap, Dh)))
    want, kc_want, vc_want = _attention_oracle_f16(oracle, qkv, qn, kn, k_old, v_old, Hq, Hk, pos, scale)
    kc, vc = _put(hip, k_old, F16), _put(hip, v_old, F16)
    qnd, knd = _put(hip, qn, BF16), _put(hip, kn, BF16)
    step(f"jh_attention_decode f16 cache Hq={Hq} Hk={Hk} pos={pos}")
    got = hip.Floats(hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc, vc, scale,
                                         out_dtype=F32))
    ok, dd, sc = rel_ok(got, want, 1e-3)
    assert ok, (dd, sc)
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    assert np.array_equal(gv, vc_want)
    ok, dd, sc = rel_ok(gk[:, :, pos], kc_want[:, :, pos], 1e-3)
    assert ok, (dd, sc)
    assert np.array_equal(np.delete(gk, pos, axis=2), np.delete(kc_want, pos, axis=2))
    kc2, vc2 = _put(hip, k_old, F16), _put(hip, v_old, F16)
    qr = hip.QKNormRoPEAppend(hip.FromFloats(qkv), Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2)
    comp = hip.Floats(hip.SDPA(qr, kc2, vc2, scale, False, kv_len=pos + 1, out_dtype=F32)).reshape(1, -1)
    ok, dd, sc = rel_ok(got, comp, 1e-4)
    assert ok, (dd, sc)
    assert np.array_equal(hip.Floats(kc2), gk)


def _qkv_case(hip, rng, Hq, Hk, K, cap, cache_dt):
    Dh = 128
    q = synth.quant_linear(Hq + K + cap, (Hq + 2 * Hk) * Dh, K, 64)
    w, s, b = upload_quant(hip, q)
    h = (2.0 * rng.standard_normal((1, K))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(K))
    qn, kn = _bf16(1 + 0.1 * rng.standard_normal(Dh)), _bf16(1 + 0.1 * rng.standard_normal(Dh))
    cv = _f16 if cache_dt == F16 else _bf16
    k_old, v_old = cv(rng.standard_normal((1, Hk, cap, Dh))), cv(rng.standard_normal((1, Hk, cap, Dh)))
    u, st = hip.NormPrepare(hip.FromFloats(h), _put(hip, nw, BF16))
    return (w, s, b), _put(hip, qn, BF16), _put(hip, kn, BF16), k_old, v_old, u, st


@pytest.mark.parametrize("pos", [15, 512, 3000])
def test_qkv_attention_decode_f16_cache(hip, oracle, pos):
    """The fused q/k/v product + attention over f16 caches: bit for bit the
    product then jh_attention_decode on copies of the same caches."""
    Hq, Hk, K, Dh = 32, 8, 4096, 128
    rng = np.random.default_rng(pos + 17)
    cap = pos + 9
    (w, s, b), qnd, knd, k_old, v_old, u, st = _qkv_case(hip, rng, Hq, Hk, K, cap, F16)
    step(f"jh_qkv_attention_decode f16 cache pos={pos}")
    kc1, vc1 = _put(hip, k_old, F16), _put(hip, v_old, F16)
    qkv1 = hip.empty(F32, 1, (Hq + 2 * Hk) * Dh)
    got = hip.Floats(hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv1, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0,
                                            pos, kc1, vc1, Dh ** -0.5, out_dtype=F32))
    kc2, vc2 = _put(hip, k_old, F16), _put(hip, v_old, F16)
    qkv2 = hip.QuantMatvecFused(u, w, s, b, 64, 4, _lib.JH_PRO_NORMED, eps=1e-6, stats=st, out_dtype=F32)
    want = hip.Floats(hip.AttentionDecode(qkv2, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2, Dh ** -0.5,
                                          out_dtype=F32))
    assert np.array_equal(hip.Floats(qkv1), hip.Floats(qkv2))
    assert np.array_equal(got, want)
    assert np.array_equal(hip.Floats(kc1), hip.Floats(kc2)) and np.array_equal(hip.Floats(vc1), hip.Floats(vc2))


def test_fused_wait_gives_up_loudly(hip):
    """jh_set_wait_limit(0): every attention block of the fused launch gives up
    its wait at once (each kernel still exits normally). The call's output is
    all NaN, the next synchronisation reports JH_ERR_TIMEOUT and resets the
    synchronisation state, and the next call with the default bound has the
    bits of the two-launch composition."""
    Hq, Hk, K, Dh, pos = 32, 8, 4096, 128, 700
    rng = np.random.default_rng(555)
    cap = pos + 9
    (w, s, b), qnd, knd, k_old, v_old, u, st = _qkv_case(hip, rng, Hq, Hk, K, cap, BF16)
    qkv = hip.empty(F32, 1, (Hq + 2 * Hk) * Dh)
    try:
        hip.SetWaitLimit(0)
        step("jh_qkv_attention_decode with a wait bound of 0 polls")
        kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
        out = hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc,
                                     vc, Dh ** -0.5, out_dtype=F32)
        with pytest.raises(JanisHipError) as ei:
            hip.Sync()
        assert ei.value.code == _lib.JH_ERR_TIMEOUT, str(ei.value)
        assert np.isnan(hip.Floats(out)).all()
        hip.Sync()  # reported once, then reset
    finally:
        hip.SetWaitLimit(1 << 22)
    step("the next call, default bound, against the two-launch composition")
    for t in range(2):
        kc1, vc1 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
        got = hip.Floats(hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0,
                                                pos, kc1, vc1, Dh ** -0.5, out_dtype=F32))
        kc2, vc2 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
        q2 = hip.QuantMatvecFused(u, w, s, b, 64, 4, _lib.JH_PRO_NORMED, eps=1e-6, stats=st, out_dtype=F32)
        want = hip.Floats(hip.AttentionDecode(q2, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2, Dh ** -0.5,
                                              out_dtype=F32))
        assert np.isfinite(got).all() and np.array_equal(got, want), t
    with pytest.raises(JanisHipError):
        hip.SetWaitLimit(-1)


def test_noalloc_attention_honours_value_checks(hip):
    """jh_attention_decode_noalloc with JH_CHECK_VALUES: a NaN in q gives
    JH_ERR_NONFINITE naming the operator, as jh_attention_decode does."""
    Hq, Hk, Dh, pos = 32, 8, 128, 40
    rng = np.random.default_rng(8)
    qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
    qkv[0, 5] = np.nan
    kc, vc = _put(hip, _bf16(rng.standard_normal((1, Hk, pos + 4, Dh))), BF16), \
        _put(hip, _bf16(rng.standard_normal((1, Hk, pos + 4, Dh))), BF16)
    step("jh_attention_decode_noalloc with value checks")
    hip.SetChecks(_lib.JH_CHECK_VALUES)
    try:
        for noalloc in (False, True):
            with pytest.raises(JanisHipError) as ei:
                hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, None, None, 1e-6, 1e6, 1.0, pos, kc, vc,
                                    Dh ** -0.5, out_dtype=F32, noalloc=noalloc)
            assert ei.value.code == _lib.JH_ERR_NONFINITE and "attention_decode" in str(ei.value), noalloc
    finally:
        hip.SetChecks(False)


def test_mirror_has_every_backend_method(hip):
    """The mirror answers every method of engine.Backend (engine/backend.go:
    142-287, the 40 a Go type needs for cpu/assert.go:6's assertion); the ones
    off this path raise JH_ERR_UNSUPPORTED, and Eval waits for the stream."""
    names = ["Version", "FromFloats", "FromInt32", "FromRaw", "Add", "Concat", "Slice", "Eval", "Mul", "SiLU",
             "RMSNorm", "LayerNorm", "Erf", "Mean", "RoPE", "RoPEFreqs", "Reshape", "Transpose", "SDPA", "MatMul",
             "Tanh", "Exp", "Sigmoid", "Softplus", "Conv1dDepthwise", "GatedDeltaScan", "Softmax", "ExpandDims",
             "Gelu", "ScalarMul", "ScalarAdd", "Cast", "TakeAxis", "Dequantize", "QuantMatmul", "GatherQuantMatmul",
             "Floats", "Argmax", "Ints", "Close"]
    assert len(names) == 40 and all(callable(getattr(hip, n)) for n in names)
    x = hip.FromFloats(np.ones((2, 3), np.float32))
    hip.Eval(x)
    for n, args in (("MatMul", (x, x)), ("LayerNorm", (x, x, x, 1e-5)), ("Erf", (x,)), ("Tanh", (x,)),
                    ("Exp", (x,)), ("Sigmoid", (x,)), ("Softplus", (x,)), ("Conv1dDepthwise", (x, x)),
                    ("GatedDeltaScan", (x, x, x, x, x, x)), ("Gelu", (x,))):
        with pytest.raises(JanisHipError) as ei:
            getattr(hip, n)(*args)
        assert ei.value.code == _lib.JH_ERR_UNSUPPORTED, n
