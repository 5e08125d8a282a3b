"""GPU parity of the decode-step operators (RMSNorm, RoPE, SDPA, element-wise,
Argmax, row gather, KV append) against the CPU oracle, through the C ABI.

Bar: fp32 outputs within 1e-5 of max|oracle| where the kernel follows the
oracle's arithmetic up to reduction order (norms, RoPE), 1e-3 for attention
(online softmax with fp32 exp against the oracle's double exp); bf16 outputs
within 1e-2; indices and copies exact.
"""
import numpy as np
import pytest

from janis_amd import synth
from janis_amd.engine import BF16, F16, F32, I32, U32, JanisHipError
from tests.conftest import hip_runtime, rel_ok, step, upload_quant

pytestmark = pytest.mark.gpu


def _bf16(a):
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.asarray(a, np.float32)))


def _put(hip, a, dt):
    a = np.asarray(a, np.float32)
    if dt == BF16:
        return hip.FromBF16Bits(synth.f32_to_bf16_bits(a), *a.shape)
    return hip.FromFloats(a, *a.shape)


@pytest.mark.parametrize("rows,d,dt", [(5, 4096, BF16), (40, 128, F32), (3, 1000, F32)])
def test_rms_norm(hip, oracle, rows, d, dt):
    rng = np.random.default_rng(rows * d)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    if dt == BF16:
        x, w = _bf16(x), _bf16(w)
    step(f"jh_rms_norm rows={rows} d={d}")
    got = hip.Floats(hip.RMSNorm(_put(hip, x, dt), _put(hip, w, dt), 1e-6, out_dtype=F32))
    ok, dd, sc = rel_ok(got, oracle.rms_norm(x, w, 1e-6), 1e-5)
    assert ok, (dd, sc)


@pytest.mark.parametrize("traditional,dims,offset", [(False, 128, 511), (True, 128, 3), (False, 64, 8191)])
def test_rope(hip, oracle, traditional, dims, offset):
    rng = np.random.default_rng(dims + offset)
    x = rng.standard_normal((1, 40, 3, 128)).astype(np.float32)
    step(f"jh_rope dims={dims} traditional={traditional} offset={offset}")
    got = hip.Floats(hip.RoPE(_put(hip, x, F32), dims, traditional, 1e6, 1.0, offset))
    want = oracle.rope(x, dims, traditional, 1e6, 1.0, offset)
    ok, dd, sc = rel_ok(got, want, 1e-5)
    assert ok, (dd, sc)
    assert np.array_equal(got[..., dims:], x[..., dims:])


def test_rope_freqs(hip, oracle):
    x = np.random.default_rng(7).standard_normal((1, 8, 2, 128)).astype(np.float32)
    freqs = (5e5 ** (np.arange(64) * 2.0 / 128) * np.linspace(1, 4, 64)).astype(np.float32)
    step("jh_rope with freqs")
    got = hip.Floats(hip.RoPEFreqs(_put(hip, x, F32), 128, False, 1.0, 77, hip.FromFloats(freqs)))
    ok, dd, sc = rel_ok(got, oracle.rope(x, 128, False, 1.0, 1.0, 77, freqs=freqs), 1e-5)
    assert ok, (dd, sc)


def _cache(rng, B, Hk, cap, Dh):
    k = _bf16(rng.standard_normal((B, Hk, cap, Dh)))
    v = _bf16(rng.standard_normal((B, Hk, cap, Dh)))
    return k, v


@pytest.mark.parametrize("Lk,q_dt", [(1, BF16), (100, F32), (512, BF16), (8192, BF16)])
def test_sdpa_decode_qwen3(hip, oracle, Lk, q_dt):
    """One query row per head at the Qwen3-8B shape (32 query heads on 8 kv
    heads, head_dim 128) over a bf16 cache with spare capacity: the split-over-
    keys path."""
    B, Hq, Hk, Dh, cap = 1, 32, 8, 128, Lk + 37
    rng = np.random.default_rng(Lk)
    q = rng.standard_normal((B, Hq, 1, Dh)).astype(np.float32)
    if q_dt == BF16:
        q = _bf16(q)
    k, v = _cache(rng, B, Hk, cap, Dh)
    step(f"jh_sdpa decode Lk={Lk}")
    got = hip.Floats(hip.SDPA(_put(hip, q, q_dt), _put(hip, k, BF16), _put(hip, v, BF16), Dh ** -0.5, False,
                              kv_len=Lk, out_dtype=F32))
    want = oracle.sdpa(q, k[:, :, :Lk], v[:, :, :Lk], Dh ** -0.5, False)
    ok, dd, sc = rel_ok(got, want, 1e-3)
    assert ok, (dd, sc)
    # causal is the same mask for a single query row
    got_c = hip.Floats(hip.SDPA(_put(hip, q, q_dt), _put(hip, k, BF16), _put(hip, v, BF16), Dh ** -0.5, True,
                                kv_len=Lk, out_dtype=F32))
    ok, dd, sc = rel_ok(got_c, want, 1e-3)
    assert ok, (dd, sc)


@pytest.mark.parametrize("Hq,Hk", [(8, 8), (8, 4), (16, 2)])
def test_sdpa_decode_groups(hip, oracle, Hq, Hk):
    B, Dh, Lk = 2, 128, 300
    rng = np.random.default_rng(Hq * 10 + Hk)
    q = _bf16(rng.standard_normal((B, Hq, 1, Dh)))
    k, v = _cache(rng, B, Hk, Lk, Dh)
    step(f"jh_sdpa decode B=2 Hq={Hq} Hk={Hk}")
    got = hip.Floats(hip.SDPA(_put(hip, q, BF16), _put(hip, k, BF16), _put(hip, v, BF16), 0.1, False, out_dtype=F32))
    ok, dd, sc = rel_ok(got, oracle.sdpa(q, k, v, 0.1, False), 1e-3)
    assert ok, (dd, sc)


@pytest.mark.parametrize("Hq,Hk,Lq,Lk,Dh,causal,kv_dt", [(8, 2, 5, 13, 64, True, F32), (4, 4, 6, 6, 128, True, BF16),
                                                         (6, 3, 1, 40, 64, False, F32), (4, 1, 3, 9, 96, False, F32)])
def test_sdpa_rows(hip, oracle, Hq, Hk, Lq, Lk, Dh, causal, kv_dt):
    """Prefill-shaped and other calls: the per-row kernel with the offset causal mask."""
    rng = np.random.default_rng(Hq + Lq * 7 + Lk)
    q = rng.standard_normal((1, Hq, Lq, Dh)).astype(np.float32)
    k = rng.standard_normal((1, Hk, Lk, Dh)).astype(np.float32)
    v = rng.standard_normal((1, Hk, Lk, Dh)).astype(np.float32)
    if kv_dt == BF16:
        k, v = _bf16(k), _bf16(v)
    step(f"jh_sdpa rows Hq={Hq} Hk={Hk} Lq={Lq} Lk={Lk} Dh={Dh} causal={causal}")
    got = hip.Floats(hip.SDPA(_put(hip, q, F32), _put(hip, k, kv_dt), _put(hip, v, kv_dt), Dh ** -0.5, causal))
    ok, dd, sc = rel_ok(got, oracle.sdpa(q, k, v, Dh ** -0.5, causal), 1e-4)
    assert ok, (dd, sc)


@pytest.mark.parametrize("dt", [F32, BF16])
def test_elementwise(hip, oracle, dt):
    rng = np.random.default_rng(11)
    a = rng.standard_normal(12289).astype(np.float32) * 4
    b = rng.standard_normal(12289).astype(np.float32)
    if dt == BF16:
        a, b = _bf16(a), _bf16(b)
    ta, tb = _put(hip, a, dt), _put(hip, b, dt)
    step(f"jh_elementwise dtype={dt}")
    np.testing.assert_array_equal(hip.Floats(hip.Add(ta, tb, out_dtype=F32)), (a + b).astype(np.float32))
    np.testing.assert_array_equal(hip.Floats(hip.Mul(ta, tb, out_dtype=F32)), (a * b).astype(np.float32))
    s = oracle.silu(a)
    ok, dd, sc = rel_ok(hip.Floats(hip.SiLU(ta, out_dtype=F32)), s, 1e-6)
    assert ok, (dd, sc)
    ok, dd, sc = rel_ok(hip.Floats(hip.SiLUMul(ta, tb, out_dtype=F32)), s * b, 1e-6)
    assert ok, (dd, sc)


def test_argmax(hip, oracle):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 151936)).astype(np.float32)
    x[1, 70000] = x[1, 123] = 50.0  # tie: the first index wins
    x[2] = -np.inf
    step("jh_argmax vocab=151936")
    got = hip.Ints(hip.Argmax(hip.FromFloats(x)))
    assert list(got) == list(oracle.argmax(x)) == [int(np.argmax(x[0])), 123, 0]


def test_argmax_one_launch_rows_and_repeats(hip, oracle):
    """Up to 2048 rows take the one-launch argmax (the last block of a row
    merges its candidates and resets the row's counter); more rows the two
    launches. Repeated calls, NaN rows and rows past the counted ones."""
    rng = np.random.default_rng(31)
    for rows, n in ((1, 151936), (7, 5000), (2049, 300)):
        x = rng.standard_normal((rows, n)).astype(np.float32)
        x[0, n - 1] = x[0, 1] = 9.0  # tie
        if rows > 3:
            x[3] = np.nan
            x[2, n // 2] = np.inf
        step(f"jh_argmax rows={rows} n={n} (3 calls)")
        t = hip.FromFloats(x)
        want = oracle.argmax(x)
        for _ in range(3):
            assert np.array_equal(hip.Ints(hip.Argmax(t)), want)


def test_argmax_graph_replays(hip, oracle):
    """The one-launch argmax captured in a HIP graph and replayed on new logits,
    with eager argmax calls between the replays (the row counter is reset by
    the launch itself)."""
    import ctypes

    rt = hip_runtime()
    rng = np.random.default_rng(32)
    x = rng.standard_normal((1, 151936)).astype(np.float32)
    t = hip.FromFloats(x)
    other = hip.FromFloats(rng.standard_normal((2, 9000)).astype(np.float32))
    out = hip.empty(I32, 1)

    def put(a):
        hip.Sync()
        hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(t.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        hip.Sync()

    def call():
        from janis_amd._lib import check
        check(hip._ctx, hip._L.jh_argmax(hip._ctx, t.ptr, F32, 1, 151936, out.ptr))

    call()  # eager call before the capture
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        hip.SetStream(stream.value)
        step("capture jh_argmax")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        call()
        assert rt.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for k in range(4):
            step(f"argmax graph replay {k}")
            x2 = rng.standard_normal((1, 151936)).astype(np.float32)
            x2[0, 1000 * k + 5] = 20.0
            put(x2)
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            assert hip.Ints(out)[0] == 1000 * k + 5 == oracle.argmax(x2)[0]
            hip.Ints(hip.Argmax(other))  # eager work between replays
    finally:
        hip.SetStream(None)
        rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)


@pytest.mark.parametrize("bits,d,gs,sb", [(4, 4096, 64, BF16), (8, 4096, 64, F32), (2, 1024, 32, BF16),
                                          (4, 2560, 128, F32)])
def test_embed_norm_prepare_matches_separate_calls(hip, bits, d, gs, sb):
    """jh_embed_norm_prepare = TakeAxis x3 + Dequantize, NormPrepare and
    RoPETable, bit for bit; an id outside the table gives the zero row."""
    q = synth.quant_linear(40 + bits, 300, d, group_size=gs, bits=bits)
    w = hip.FromRaw(U32, q.w, *q.w.shape)
    if sb == F32:
        s, b = hip.FromFloats(q.s, *q.s.shape), hip.FromFloats(q.b, *q.b.shape)
    else:
        s, b = hip.FromBF16Bits(q.s_bits, *q.s_bits.shape), hip.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    nw = hip.FromBF16Bits(synth.f32_to_bf16_bits((1 + 0.1 * np.random.default_rng(d).standard_normal(d))
                                                 .astype(np.float32)), d)
    for tok, pos in ((299, 511), (0, 8191), (17, 0), (300, 3)):
        step(f"jh_embed_norm_prepare bits={bits} d={d} gs={gs} token={tok} pos={pos}")
        ids = hip.FromInt32(np.array([tok], np.int32))
        h, u, st, cs = hip.EmbedNormPrepare(ids, w, s, b, gs, bits, nw, rope=(128, 1e6, 1.0, pos))
        h2 = hip.Dequantize(hip.TakeAxis(w, ids), hip.TakeAxis(s, ids), hip.TakeAxis(b, ids), gs, bits)
        u2, st2 = hip.NormPrepare(h2, nw)
        cs2 = hip.RoPETable(128, 1e6, 1.0, pos)
        for a, c in ((h, h2), (st, st2), (cs, cs2)):
            assert np.array_equal(hip.Floats(a).view(np.uint32), hip.Floats(c).view(np.uint32))
        assert hip.Bytes(u) == hip.Bytes(u2)
        if tok >= 300:
            assert not hip.Floats(h).any()
    _, _, _, none = hip.EmbedNormPrepare(hip.FromInt32(np.array([5], np.int32)), w, s, b, gs, bits, nw)
    assert none is None
    hip.SetChecks(True)
    try:
        with pytest.raises(JanisHipError):
            hip.EmbedNormPrepare(hip.FromInt32(np.array([300], np.int32)), w, s, b, gs, bits, nw)
    finally:
        hip.SetChecks(False)


def test_quant_embedding_rows(hip, oracle):
    """QuantEmbedding.Forward (qwen/embed.go:78-83): TakeAxis of the packed
    words, scales and biases, then Dequantize; bit-exact."""
    q = synth.quant_linear(13, 1000, 4096)
    w, s, b = upload_quant(hip, q)
    ids = np.array([0, 999, 17, 17], np.int32)
    it = hip.FromInt32(ids)
    step("jh_take_rows + jh_dequantize (embedding)")
    rows = hip.Dequantize(hip.TakeAxis(w, it), hip.TakeAxis(s, it), hip.TakeAxis(b, it), 64, 4)
    got = hip.Floats(rows)
    want = oracle.dequantize(q.w[ids], q.s[ids], q.b[ids], 64)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    bad = hip.FromInt32(np.array([3, 1000], np.int32))
    z = hip.Ints(hip.TakeAxis(w, bad))
    assert np.array_equal(z[0], q.w[3].view(np.int32)) and not z[1].any()
    hip.SetChecks(True)
    try:
        with pytest.raises(JanisHipError):
            hip.TakeAxis(w, bad)
    finally:
        hip.SetChecks(False)


def test_append_kv(hip):
    rng = np.random.default_rng(14)
    B, Hk, cap, Dh = 1, 8, 64, 128
    kc, vc = hip.empty(BF16, B, Hk, cap, Dh), hip.empty(BF16, B, Hk, cap, Dh)
    k0, v0 = _bf16(rng.standard_normal((B, Hk, 10, Dh))), _bf16(rng.standard_normal((B, Hk, 10, Dh)))
    k1 = rng.standard_normal((B, Hk, 1, Dh)).astype(np.float32)
    v1 = rng.standard_normal((B, Hk, 1, Dh)).astype(np.float32)
    step("jh_kv_append")
    hip.AppendKVRows(kc, vc, 0, _put(hip, k0, BF16), _put(hip, v0, BF16))
    hip.AppendKVRows(kc, vc, 10, _put(hip, k1, F32), _put(hip, v1, F32))  # fp32 rows into the bf16 cache
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    assert np.array_equal(gk[:, :, :10], k0) and np.array_equal(gk[:, :, 10:11], _bf16(k1))
    assert np.array_equal(gv[:, :, :10], v0) and np.array_equal(gv[:, :, 10:11], _bf16(v1))
    with pytest.raises(JanisHipError):
        hip.AppendKVRows(kc, vc, 64, _put(hip, k1, F32), _put(hip, v1, F32))


def test_qk_norm_rope_append_matches_separate_ops(hip, oracle):
    """jh_qk_norm_rope_append against the oracle's RMSNorm + RoPE and the cache rows."""
    rng = np.random.default_rng(15)
    Hq, Hk, Dh, cap, pos = 32, 8, 128, 40, 33
    qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
    qn, kn = _bf16(1 + 0.1 * rng.standard_normal(Dh)), _bf16(1 + 0.1 * rng.standard_normal(Dh))
    kc, vc = hip.empty(BF16, 1, Hk, cap, Dh), hip.empty(BF16, 1, Hk, cap, Dh)
    step("jh_qk_norm_rope_append")
    q = hip.Floats(hip.QKNormRoPEAppend(hip.FromFloats(qkv), Hq, Hk, _put(hip, qn, BF16), _put(hip, kn, BF16), 1e-6,
                                        1e6, 1.0, pos, kc, vc, out_dtype=F32))
    qh = qkv[0, :Hq * Dh].reshape(1, Hq, 1, Dh)
    kh = qkv[0, Hq * Dh:(Hq + Hk) * Dh].reshape(1, Hk, 1, Dh)
    vh = qkv[0, (Hq + Hk) * Dh:].reshape(1, Hk, 1, Dh)
    want_q = oracle.rope(oracle.rms_norm(qh, qn, 1e-6), Dh, False, 1e6, 1.0, pos)
    want_k = oracle.rope(oracle.rms_norm(kh, kn, 1e-6), Dh, False, 1e6, 1.0, pos)
    ok, dd, sc = rel_ok(q, want_q, 1e-5)
    assert ok, (dd, sc)
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    ok, dd, sc = rel_ok(gk[:, :, pos:pos + 1], want_k, 1e-2)
    assert ok, (dd, sc)
    assert np.array_equal(gv[:, :, pos:pos + 1], _bf16(vh))


def _fused_case(rng, N, K, gs=64, seed=0, bits=4):
    q = synth.quant_linear(seed or N + K, N, K, gs, bits=bits)
    h = (3.0 * rng.standard_normal((1, K))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(K))
    return q, h, nw


@pytest.mark.parametrize("N,K,bits", [(6144, 4096, 4), (70000, 4096, 4), (4096, 12288, 4), (300, 960, 4),
                                      (6144, 4096, 8)])
def test_quant_matvec_fused_rmsnorm(hip, oracle, N, K, bits):
    """RMSNorm -> QuantMatmul in one call (the norm feeding q/k/v, gate/up and
    the LM head): against the oracle's RMSNorm, bf16 rounding, QuantMatmul, and
    against the backend's own two-launch composition. (300, 960) is outside the
    register tiles and takes the composed path, as do 8-bit weights with this
    prologue."""
    from janis_amd import _lib
    rng = np.random.default_rng(N + K)
    q, h, nw = _fused_case(rng, N, K, bits=bits)
    w, s, b = upload_quant(hip, q)
    hd, nwd = hip.FromFloats(h), _put(hip, nw, BF16)
    step(f"jh_quant_matvec_fused RMSNorm N={N} K={K} bits={bits}")
    got = hip.Floats(hip.QuantMatvecFused(hd, w, s, b, 64, bits, _lib.JH_PRO_RMSNORM, nwd, 1e-6, out_dtype=F32))
    xn = _bf16(oracle.rms_norm(h, nw, 1e-6))
    want = oracle.quant_matmul(xn, q.w, q.s, q.b, 64, bits=bits)
    ok, dd, sc = rel_ok(got, want, 1e-2)
    assert ok, (dd, sc)
    comp = hip.Floats(hip.QuantMatmul(hip.RMSNorm(hd, nwd, 1e-6, out_dtype=BF16), w, s, b, True, 64, bits,
                                      out_dtype=F32))
    # the one-launch path rounds x*w (not x*w/rms) to bf16: a different rounding
    # of the same input, about 2^-9 / sqrt(3) of the product's spread apart
    ok, dd, sc = rel_ok(got, comp, 5e-3)
    assert ok, (dd, sc)
    gb = hip.Floats(hip.QuantMatvecFused(hd, w, s, b, 64, bits, _lib.JH_PRO_RMSNORM, nwd, 1e-6, out_dtype=BF16))
    ok, dd, sc = rel_ok(gb, want, 1e-2)
    assert ok, (dd, sc)


@pytest.mark.parametrize("N,K", [(4096, 12288), (1024, 3072), (200, 960)])
def test_quant_matvec_fused_swiglu_resid(hip, oracle, N, K):
    """Mul(SiLU(gate), up) -> QuantMatmul -> Add(resid, .) in one call (the
    down product of MLP.Forward and the block's second residual add), written
    in place into the fp32 residual stream."""
    from janis_amd import _lib
    rng = np.random.default_rng(N * 3 + K)
    q = synth.quant_linear(N + 7 * K, N, K, 64)
    w, s, b = upload_quant(hip, q)
    gu = _bf16(2.0 * rng.standard_normal((1, 2 * K)))
    resid = (10.0 * rng.standard_normal((1, N))).astype(np.float32)
    hd = hip.FromFloats(resid)
    step(f"jh_quant_matvec_fused SiLU*mul + resid N={N} K={K}")
    out = hip.QuantMatvecFused(_put(hip, gu, BF16), w, s, b, 64, 4, _lib.JH_PRO_SILU_MUL, resid=hd, out=hd)
    assert out is hd
    got = hip.Floats(hd)
    act = _bf16(oracle.silu(gu[:, :K]) * gu[:, K:])
    prod = oracle.quant_matmul(act, q.w, q.s, q.b, 64)
    ok, dd, sc = rel_ok(got - resid, prod, 1e-2)
    assert ok, (dd, sc)
    ok, dd, sc = rel_ok(got, resid + prod, 1e-3)
    assert ok, (dd, sc)


@pytest.mark.parametrize("N,K,sb", [(4096, 4096, BF16), (4096, 4096, "f16")])
def test_quant_matvec_fused_resid_only(hip, oracle, N, K, sb):
    """QuantMatmul -> Add(resid, .) (the o product and the block's first
    residual add); with f16 scales it is composed from two launches."""
    from janis_amd import _lib
    rng = np.random.default_rng(N + K + 1)
    q = synth.quant_linear(N + K + 3, N, K, 64)
    w, s, b = upload_quant(hip, q)
    if sb == "f16":
        s = hip.FromRaw(F16, q.s.astype(np.float16), *q.s.shape)
        b = hip.FromRaw(F16, q.b.astype(np.float16), *q.b.shape)
    x = _bf16(rng.standard_normal((1, K)))
    resid = rng.standard_normal((1, N)).astype(np.float32)
    hd = hip.FromFloats(resid)
    step(f"jh_quant_matvec_fused resid N={N} K={K} scales={sb}")
    hip.QuantMatvecFused(_put(hip, x, BF16), w, s, b, 64, 4, resid=hd, out=hd)
    got = hip.Floats(hd)
    sc_ = q.s.astype(np.float16).astype(np.float32) if sb == "f16" else q.s
    bi_ = q.b.astype(np.float16).astype(np.float32) if sb == "f16" else q.b
    want = resid + oracle.quant_matmul(x, q.w, sc_, bi_, 64)
    ok, dd, sc = rel_ok(got, want, 1e-3)
    assert ok, (dd, sc)
    with pytest.raises(JanisHipError):
        hip.QuantMatvecFused(_put(hip, x, BF16), w, s, b, 64, 4, resid=hip.FromFloats(resid[:, :10]))


@pytest.mark.parametrize("I,K,gs", [(12288, 4096, 64), (1024, 512, 32), (300, 960, 64)])
def test_quant_matvec_fused_rmsnorm_swiglu(hip, oracle, I, K, gs):
    """RMSNorm -> Gate/Up products -> Mul(SiLU(gate), up) in one call (the first
    half of MLP.Forward after the block's PostNorm), W = [gate rows; up rows].
    (300, 960) is outside the register tiles and takes the composed path."""
    from janis_amd import _lib
    rng = np.random.default_rng(I + K)
    q = synth.quant_linear(I + 3 * K, 2 * I, K, gs)
    w, s, b = upload_quant(hip, q)
    h = (2.0 * rng.standard_normal((1, K))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(K))
    step(f"jh_quant_matvec_fused RMSNorm + SwiGLU I={I} K={K} gs={gs}")
    got = hip.Floats(hip.QuantMatvecFused(hip.FromFloats(h), w, s, b, gs, 4, _lib.JH_PRO_RMSNORM,
                                          _put(hip, nw, BF16), 1e-6, epilogue=_lib.JH_EPI_SWIGLU,
                                          out_dtype=F32))
    assert got.shape == (1, I)
    gu = oracle.quant_matmul(_bf16(oracle.rms_norm(h, nw, 1e-6)), q.w, q.s, q.b, gs)[0]
    want = oracle.silu(gu[:I]) * gu[I:]
    ok, dd, sc = rel_ok(got[0], want, 1e-2)
    assert ok, (dd, sc)


def _attention_case(rng, Hq, Hk, cap, pos, with_norm):
    Dh = 128
    qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
    qn = _bf16(1 + 0.1 * rng.standard_normal(Dh)) if with_norm else None
    kn = _bf16(1 + 0.1 * rng.standard_normal(Dh)) if with_norm else None
    k_old, v_old = _cache(rng, 1, Hk, cap, Dh)
    return qkv, qn, kn, k_old, v_old


def _attention_oracle(oracle, qkv, qn, kn, k_old, v_old, Hq, Hk, pos, scale):
    Dh = 128
    qh = qkv[0, :Hq * Dh].reshape(1, Hq, 1, Dh)
    kh = qkv[0, Hq * Dh:(Hq + Hk) * Dh].reshape(1, Hk, 1, Dh)
    vh = qkv[0, (Hq + Hk) * Dh:].reshape(1, Hk, 1, Dh)
    if qn is not None:
        qh, kh = oracle.rms_norm(qh, qn, 1e-6), oracle.rms_norm(kh, kn, 1e-6)
    q = oracle.rope(qh, Dh, False, 1e6, 1.0, pos)
    k_new = _bf16(oracle.rope(kh, Dh, False, 1e6, 1.0, pos))
    kc, vc = k_old.copy(), v_old.copy()
    kc[:, :, pos:pos + 1], vc[:, :, pos:pos + 1] = k_new, _bf16(vh)
    out = oracle.sdpa(q, kc[:, :, :pos + 1], vc[:, :, :pos + 1], scale, False).reshape(1, Hq * Dh)
    return out, kc, vc


@pytest.mark.parametrize("Hq,Hk,pos,with_norm,table", [(32, 8, 0, True, False), (32, 8, 15, True, True),
                                                       (32, 8, 16, True, False), (32, 8, 512, True, True),
                                                       (32, 8, 8192, True, True), (8, 8, 300, False, False),
                                                       (16, 8, 1000, True, True), (64, 8, 777, True, False),
                                                       (32, 8, 64, True, True), (32, 8, 65, True, False),
                                                       (32, 4, 600, True, True), (64, 16, 900, True, False),
                                                       (32, 8, 3000, True, True)])
def test_attention_decode(hip, oracle, Hq, Hk, pos, with_norm, table):
    """jh_attention_decode (q/k norm, RoPE, KV append, SDPA in one launch)
    against the oracle's RMSNorm + RoPE + SDPA over the updated cache, and
    against the backend's separate operators (QKNormRoPEAppend + SDPA); the
    cache rows written must be the bf16 new key and value, the others untouched."""
    rng = np.random.default_rng(Hq * 100000 + pos)
    Dh, cap = 128, pos + 9
    scale = Dh ** -0.5
    qkv, qn, kn, k_old, v_old = _attention_case(rng, Hq, Hk, cap, pos, with_norm)
    want, kc_want, vc_want = _attention_oracle(oracle, qkv, qn, kn, k_old, v_old, Hq, Hk, pos, scale)
    kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    qnd = _put(hip, qn, BF16) if with_norm else None
    knd = _put(hip, kn, BF16) if with_norm else None
    step(f"jh_attention_decode Hq={Hq} Hk={Hk} pos={pos} norm={with_norm} table={table}")
    cs = hip.RoPETable(Dh, 1e6, 1.0, pos) if table else None
    got = hip.Floats(hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc, vc, scale,
                                         out_dtype=F32, rope_cs=cs))
    ok, dd, sc = rel_ok(got, want, 1e-3)
    assert ok, (dd, sc)
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    assert np.array_equal(gv, vc_want)
    ok, dd, sc = rel_ok(gk[:, :, pos], kc_want[:, :, pos], 1e-2)  # the rotated key, bf16
    assert ok, (dd, sc)
    assert np.array_equal(np.delete(gk, pos, axis=2), np.delete(kc_want, pos, axis=2))
    if with_norm:
        kc2, vc2 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
        q = hip.QKNormRoPEAppend(hip.FromFloats(qkv), Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2)
        comp = hip.Floats(hip.SDPA(q, kc2, vc2, scale, False, kv_len=pos + 1, out_dtype=F32)).reshape(1, -1)
        ok, dd, sc = rel_ok(got, comp, 1e-4)
        assert ok, (dd, sc)
        assert np.array_equal(hip.Floats(kc2), gk)


def test_attention_decode_consecutive_tokens(hip, oracle):
    """Three tokens in a row through one context, each seeing the rows the
    previous launches appended (positions 1023 to 1025)."""
    rng = np.random.default_rng(99)
    Hq, Hk, Dh, cap, pos0 = 32, 8, 128, 1100, 1023
    scale = Dh ** -0.5
    _, qn, kn, k_old, v_old = _attention_case(rng, Hq, Hk, cap, pos0, True)
    kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    kh, vh = k_old.copy(), v_old.copy()
    for t in range(3):
        pos = pos0 + t
        qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
        step(f"jh_attention_decode token {t} pos={pos}")
        got = hip.Floats(hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, _put(hip, qn, BF16), _put(hip, kn, BF16),
                                             1e-6, 1e6, 1.0, pos, kc, vc, scale, out_dtype=F32))
        want, kh, vh = _attention_oracle(oracle, qkv, qn, kn, kh, vh, Hq, Hk, pos, scale)
        ok, dd, sc = rel_ok(got, want, 1e-3)
        assert ok, (t, dd, sc)
    with pytest.raises(JanisHipError):
        hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, None, None, 1e-6, 1e6, 1.0, cap, kc, vc, scale)


def test_attention_decode_consecutive_short_cache(hip, oracle):
    """Tokens in a row through a short cache (positions 500 to 503), where the
    launch merges its own splits: every token sees the rows the previous ones
    appended and none reads an earlier call's partials."""
    rng = np.random.default_rng(98)
    Hq, Hk, Dh, cap, pos0 = 32, 8, 128, 600, 500
    scale = Dh ** -0.5
    _, qn, kn, k_old, v_old = _attention_case(rng, Hq, Hk, cap, pos0, True)
    kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    kh, vh = k_old.copy(), v_old.copy()
    qnd, knd = _put(hip, qn, BF16), _put(hip, kn, BF16)
    for t in range(4):
        pos = pos0 + t
        qkv = rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32)
        step(f"jh_attention_decode short cache, token {t} pos={pos}")
        got = hip.Floats(hip.AttentionDecode(hip.FromFloats(qkv), Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc, vc, scale,
                                             out_dtype=F32))
        want, kh, vh = _attention_oracle(oracle, qkv, qn, kn, kh, vh, Hq, Hk, pos, scale)
        ok, dd, sc = rel_ok(got, want, 1e-3)
        assert ok, (t, dd, sc)


def test_attention_decode_graph_replays(hip, oracle):
    """A short-cache attention captured into a HIP graph and replayed on new
    q/k/v rows: every replay matches the eager call on the same inputs bit for
    bit (the merge's call tags come from device state, not from captured
    arguments) and the oracle within 1e-3."""
    import ctypes

    rt = hip_runtime()
    rng = np.random.default_rng(97)
    Hq, Hk, Dh, cap, pos = 32, 8, 128, 300, 255
    scale = Dh ** -0.5
    _, qn, kn, k_old, v_old = _attention_case(rng, Hq, Hk, cap, pos, True)
    kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    qnd, knd = _put(hip, qn, BF16), _put(hip, kn, BF16)
    qkvs = [rng.standard_normal((1, (Hq + 2 * Hk) * Dh)).astype(np.float32) for _ in range(3)]
    xt = hip.empty(F32, 1, (Hq + 2 * Hk) * Dh)
    ot = hip.empty(F32, 1, Hq * Dh)

    def put(a):
        hip.Sync()
        hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(xt.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        hip.Sync()

    def call():
        return hip.AttentionDecode(xt, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc, vc, scale, out=ot)

    eager = []
    for a in qkvs:
        put(a)
        call()
        eager.append(hip.Floats(ot).copy())
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        hip.SetStream(stream.value)
        step("capture jh_attention_decode pos=255")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        call()
        assert rt.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep, i in enumerate((1, 2, 0, 1, 1)):
            step(f"graph replay {rep} on q/k/v {i}")
            put(qkvs[i])
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            got = hip.Floats(ot)
            assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), rep
            want, _, _ = _attention_oracle(oracle, qkvs[i], qn, kn, k_old, v_old, Hq, Hk, pos, scale)
            ok, dd, sc = rel_ok(got, want, 1e-3)
            assert ok, (rep, dd, sc)
    finally:
        hip.SetStream(None)
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        if graph.value:
            rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)


@pytest.mark.parametrize("dims,pos,freqs", [(128, 0, False), (128, 8191, False), (64, 77, True)])
def test_rope_table(hip, oracle, dims, pos, freqs):
    """jh_rope_table: the oracle's RoPE applied to (1, 0) pairs gives exactly
    (cos, sin) of each angle (a*c - 0*s = c), so the table must match bit for bit."""
    half = dims // 2
    fr = (5e5 ** (np.arange(half) * 2.0 / dims) * np.linspace(1, 4, half)).astype(np.float32) if freqs else None
    x = np.zeros((1, 1, 1, dims), np.float32)
    x[..., :half] = 1.0
    r = oracle.rope(x, dims, False, 1e6, 1.0, pos, freqs=fr)[0, 0, 0]
    step(f"jh_rope_table dims={dims} pos={pos}")
    got = hip.Floats(hip.RoPETable(dims, 1e6, 1.0, pos, hip.FromFloats(fr) if freqs else None))
    assert np.array_equal(got, r)


@pytest.mark.parametrize("N1,K1,N2,bits", [(4096, 4096, 6144, 4), (4096, 12288, 24576, 4), (4096, 4096, 70000, 4),
                                           (960, 512, 300, 4), (512, 1024, 512, 4), (4096, 4096, 6144, 8),
                                           (2048, 4096, 12288, 8)])
def test_split_rmsnorm_producer_consumer(hip, oracle, N1, K1, N2, bits):
    """JH_EPI_RESID_NORM then JH_PRO_NORMED: h = resid + x.W1^T (fp32, in place),
    u = bf16(h * w) written by the producer with per-block sums of h^2, and the
    consumer's (u.W2^T) / rms(h) equals RMSNorm(h, w) -> QuantMatmul(W2) within the
    bf16 rounding of the product's input. With N2 = 24576 the consumer also
    takes the SwiGLU epilogue. (960, 512, 300) is outside the register tiles
    (composed launches). bits = 8: the 8-bit tiles with both fusions (and the
    SwiGLU epilogue at N2 = 12288)."""
    from janis_amd import _lib
    rng = np.random.default_rng(N1 + K1 + N2)
    q1 = synth.quant_linear(N1 + 5, N1, K1, 64, bits=bits)
    q2 = synth.quant_linear(N2 + 9, N2, N1, 64, bits=bits)
    w1, s1, b1 = upload_quant(hip, q1)
    w2, s2, b2 = upload_quant(hip, q2)
    x = _bf16(rng.standard_normal((1, K1)))
    resid = (3.0 * rng.standard_normal((1, N1))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(N1))
    h_d, u_d = hip.FromFloats(resid), hip.empty(BF16, 1, N1)
    st = hip.empty(F32, _lib.JH_NORM_STATS)
    step(f"split RMSNorm producer N={N1} K={K1} bits={bits}")
    hip.QuantMatvecFused(_put(hip, x, BF16), w1, s1, b1, 64, bits, norm=_put(hip, nw, BF16),
                         epilogue=_lib.JH_EPI_RESID_NORM, resid=h_d, out=h_d, stats=st, norm_out=u_d)
    h = hip.Floats(h_d)
    want_h = resid + oracle.quant_matmul(x, q1.w, q1.s, q1.b, 64, bits=bits)
    ok, dd, sc = rel_ok(h, want_h, 1e-3)
    assert ok, (dd, sc)
    assert np.array_equal(hip.Floats(u_d), _bf16(h * nw))  # exactly bf16(h * w) of the stored h
    stats = hip.Floats(st)
    assert abs(float(stats.astype(np.float64).sum()) - float((h.astype(np.float64) ** 2).sum())) <= \
        1e-5 * float((h.astype(np.float64) ** 2).sum())
    swiglu = N2 in (24576, 12288)
    step(f"split RMSNorm consumer N={N2} swiglu={swiglu} bits={bits}")
    got = hip.Floats(hip.QuantMatvecFused(u_d, w2, s2, b2, 64, bits, _lib.JH_PRO_NORMED, eps=1e-6, stats=st,
                                          epilogue=_lib.JH_EPI_SWIGLU if swiglu else _lib.JH_EPI_STORE,
                                          out_dtype=F32))
    y = oracle.quant_matmul(_bf16(oracle.rms_norm(h, nw, 1e-6)), q2.w, q2.s, q2.b, 64, bits=bits)[0]
    if swiglu:
        y = oracle.silu(y[:N2 // 2]) * y[N2 // 2:]
    ok, dd, sc = rel_ok(got[0], y, 1e-2)
    assert ok, (dd, sc)


def test_norm_prepare(hip, oracle):
    from janis_amd import _lib
    rng = np.random.default_rng(77)
    x = (2.0 * rng.standard_normal((1, 4096))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(4096))
    step("jh_norm_prepare")
    u, st = hip.NormPrepare(hip.FromFloats(x), _put(hip, nw, BF16))
    assert np.array_equal(hip.Floats(u), _bf16(x * nw))
    s = hip.Floats(st)
    assert s.shape == (_lib.JH_NORM_STATS,) and not s[2:].any()  # 4096 elements: two block partials
    ref = float((x.astype(np.float64) ** 2).sum())
    assert abs(float(s.astype(np.float64).sum()) - ref) <= 1e-5 * ref
    with pytest.raises(JanisHipError):  # one norm weight and one statistics buffer per call
        q = synth.quant_linear(3, 256, 4096, 64)
        w, s_, b_ = upload_quant(hip, q)
        hip.QuantMatvecFused(hip.FromFloats(x), w, s_, b_, 64, 4, _lib.JH_PRO_RMSNORM, _put(hip, nw, BF16), 1e-6,
                             epilogue=_lib.JH_EPI_RESID_NORM, resid=hip.FromFloats(np.zeros((1, 256), np.float32)),
                             stats=st, norm_out=hip.empty(BF16, 1, 256))


def _qkv_attn_case(hip, rng, seed, Hq, Hk, K, cap, pos):
    from janis_amd import _lib
    Dh = 128
    q = synth.quant_linear(seed, (Hq + 2 * Hk) * Dh, K, 64)
    w, s, b = upload_quant(hip, q)
    h = (2.0 * rng.standard_normal((1, K))).astype(np.float32)
    nw = _bf16(1 + 0.1 * rng.standard_normal(K))
    qn, kn = _bf16(1 + 0.1 * rng.standard_normal(Dh)), _bf16(1 + 0.1 * rng.standard_normal(Dh))
    k_old, v_old = _cache(rng, 1, Hk, cap, Dh)
    u, st = hip.NormPrepare(hip.FromFloats(h), _put(hip, nw, BF16))
    return q, (w, s, b), h, nw, qn, kn, k_old, v_old, u, st


@pytest.mark.parametrize("Hq,Hk,K,pos,qdt", [(32, 8, 4096, 0, F32), (32, 8, 4096, 15, F32), (32, 8, 4096, 512, F32),
                                             (32, 8, 4096, 512, BF16), (32, 8, 4096, 3000, F32),
                                             (32, 8, 4096, 8192, F32), (64, 8, 4096, 700, F32),
                                             (16, 8, 4096, 257, BF16), (32, 4, 4096, 600, F32),
                                             (32, 8, 2048, 300, F32)])
def test_qkv_attention_decode_matches_two_calls(hip, oracle, Hq, Hk, K, pos, qdt):
    """jh_qkv_attention_decode (the q/k/v product with the prepared norm and the
    attention in one launch, or the two operators where it does not apply:
    Hk = 4, K = 2048) against QuantMatvecFused(PRO_NORMED) then AttentionDecode
    on copies of the same caches: the q/k/v rows, the attention output and the
    cache rows written must be bit for bit the same; the output also against the
    oracle's RMSNorm -> QuantMatmul -> q/k norm -> RoPE -> SDPA within 1e-2."""
    from janis_amd import _lib
    rng = np.random.default_rng(Hq * 7919 + Hk * 31 + pos + K)
    Dh, cap = 128, pos + 9
    scale = Dh ** -0.5
    q, (w, s, b), h, nw, qn, kn, k_old, v_old, u, st = _qkv_attn_case(hip, rng, pos + 11, Hq, Hk, K, cap, pos)
    qnd, knd = _put(hip, qn, BF16), _put(hip, kn, BF16)
    cs = hip.RoPETable(Dh, 1e6, 1.0, pos)
    step(f"jh_qkv_attention_decode Hq={Hq} Hk={Hk} K={K} pos={pos} qkv={'f32' if qdt == F32 else 'bf16'}")
    kc1, vc1 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    qkv1 = hip.empty(qdt, 1, (Hq + 2 * Hk) * Dh)
    got = hip.Floats(hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv1, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0,
                                            pos, kc1, vc1, scale, rope_cs=cs, out_dtype=F32))
    step("the same as two calls")
    kc2, vc2 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    qkv2 = hip.QuantMatvecFused(u, w, s, b, 64, 4, _lib.JH_PRO_NORMED, eps=1e-6, stats=st, out_dtype=qdt)
    want2 = hip.Floats(hip.AttentionDecode(qkv2, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2, scale,
                                           out_dtype=F32, rope_cs=cs))
    assert np.array_equal(hip.Floats(qkv1), hip.Floats(qkv2))
    assert np.array_equal(got, want2)
    assert np.array_equal(hip.Floats(kc1), hip.Floats(kc2)) and np.array_equal(hip.Floats(vc1), hip.Floats(vc2))
    qkv_o = oracle.quant_matmul(_bf16(oracle.rms_norm(h, nw, 1e-6)), q.w, q.s, q.b, 64)
    if qdt == BF16:
        qkv_o = _bf16(qkv_o)
    want, _, _ = _attention_oracle(oracle, qkv_o, qn, kn, k_old, v_old, Hq, Hk, pos, scale)
    ok, dd, sc = rel_ok(got, want, 1e-2)
    assert ok, (dd, sc)


def test_qkv_attention_decode_tokens_and_graph_replays(hip, oracle):
    """Consecutive tokens through one context (each sees the rows the previous
    launches appended), then the launch captured in a HIP graph and replayed on
    new inputs with eager work between the replays: every replay equals the
    eager call bit for bit (the launch's arrival counters are cleared by the
    launch itself)."""
    import ctypes

    from janis_amd import _lib
    rt = hip_runtime()
    rng = np.random.default_rng(4242)
    Hq, Hk, K, Dh, cap, pos0 = 32, 8, 4096, 128, 1100, 1021
    scale = Dh ** -0.5
    q, (w, s, b), h, nw, qn, kn, k_old, v_old, u, st = _qkv_attn_case(hip, rng, 77, Hq, Hk, K, cap, pos0)
    qnd, knd = _put(hip, qn, BF16), _put(hip, kn, BF16)
    kc, vc = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    kc2, vc2 = _put(hip, k_old, BF16), _put(hip, v_old, BF16)
    qkv = hip.empty(F32, 1, (Hq + 2 * Hk) * Dh)
    for t in range(3):
        pos = pos0 + t
        step(f"jh_qkv_attention_decode token {t} pos={pos}")
        got = hip.Floats(hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0,
                                                pos, kc, vc, scale, out_dtype=F32))
        q2 = hip.QuantMatvecFused(u, w, s, b, 64, 4, _lib.JH_PRO_NORMED, eps=1e-6, stats=st, out_dtype=F32)
        want = hip.Floats(hip.AttentionDecode(q2, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc2, vc2, scale,
                                              out_dtype=F32))
        assert np.array_equal(got, want), t
    # graph: the same launch on new norm inputs, replayed
    pos = pos0 + 3
    hs = [(2.0 * rng.standard_normal((1, K))).astype(np.float32) for _ in range(3)]
    h_d = hip.FromFloats(hs[0])
    nwd = _put(hip, nw, BF16)
    out = hip.empty(F32, 1, Hq * Dh)

    def call():
        hip.NormPrepare(h_d, nwd, norm_out=u, stats=st)
        return hip.QkvAttentionDecode(u, st, 1e-6, w, s, b, 64, 4, qkv, Hq, Hk, qnd, knd, 1e-6, 1e6, 1.0, pos, kc, vc,
                                      scale, out=out)

    def put(a):
        hip.Sync()
        hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(h_d.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        hip.Sync()

    eager = []
    for a in hs:
        put(a)
        call()
        eager.append(hip.Floats(out).copy())
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        hip.SetStream(stream.value)
        step("capture jh_qkv_attention_decode")
        assert rt.hipStreamBeginCapture(stream, 0) == 0
        call()
        assert rt.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep, i in enumerate((1, 2, 0, 1)):
            step(f"graph replay {rep} on input {i}")
            put(hs[i])
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            assert np.array_equal(hip.Floats(out), eager[i]), (rep, i)
            hip.Floats(hip.QuantMatvecFused(u, w, s, b, 64, 4, _lib.JH_PRO_NORMED, eps=1e-6, stats=st,
                                            out_dtype=F32))  # eager work between replays
    finally:
        hip.SetStream(None)
        rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)
        rt.hipStreamDestroy(stream)
