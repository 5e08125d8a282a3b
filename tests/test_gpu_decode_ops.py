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
from janis_amd.engine import BF16, F32, I32, U32, JanisHipError
from tests.conftest import rel_ok, step, upload_quant

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
    hip.AppendKV(kc, vc, 0, _put(hip, k0, BF16), _put(hip, v0, BF16))
    hip.AppendKV(kc, vc, 10, _put(hip, k1, F32), _put(hip, v1, F32))  # fp32 rows into the bf16 cache
    gk, gv = hip.Floats(kc), hip.Floats(vc)
    assert np.array_equal(gk[:, :, :10], k0) and np.array_equal(gk[:, :, 10:11], _bf16(k1))
    assert np.array_equal(gv[:, :, :10], v0) and np.array_equal(gv[:, :, 10:11], _bf16(v1))
    with pytest.raises(JanisHipError):
        hip.AppendKV(kc, vc, 64, _put(hip, k1, F32), _put(hip, v1, F32))
