"""GPU checks of the layout operators of the engine mirror -- Slice, Transpose,
ExpandDims (views), Reshape of a view, Concat, Cast (jh_copy_strided) -- and of
the engine capabilities built on them: KVAppender (engine/backend.go:56-61, the
MLX backend's growth rule mlxc/mlxc.go:283-306) and Sweeper / Freer
(engine/backend.go:43-93). Copies are exact; casts round to nearest even."""
import numpy as np
import pytest

from janis_amd import synth
from janis_amd.engine import BF16, F16, F32, I32, U32, JanisHipError
from tests.conftest import step

pytestmark = pytest.mark.gpu


def _bf16(a):
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.asarray(a, np.float32)))


def test_views_and_copies(hip):
    rng = np.random.default_rng(3)
    a = rng.standard_normal((2, 3, 5, 7)).astype(np.float32)
    t = hip.FromFloats(a)
    step("Slice / Transpose / ExpandDims / Reshape views")
    assert np.array_equal(hip.Floats(hip.Slice(t, 2, 1, 4)), a[:, :, 1:4])
    assert np.array_equal(hip.Floats(hip.Slice(t, -1, 6, 7)), a[..., 6:7])
    tr = hip.Transpose(t, 0, 2, 1, 3)
    assert not tr.contiguous and np.array_equal(hip.Floats(tr), a.transpose(0, 2, 1, 3))
    assert np.array_equal(hip.Floats(hip.Transpose(t, 3, 1, 0, 2)), a.transpose(3, 1, 0, 2))
    assert np.array_equal(hip.Floats(hip.Reshape(tr, 2, 5, 21)), a.transpose(0, 2, 1, 3).reshape(2, 5, 21))
    assert np.array_equal(hip.Floats(hip.ExpandDims(hip.Slice(t, 1, 1, 2), 0)), a[None, :, 1:2])
    assert np.array_equal(hip.Floats(hip.Slice(hip.Transpose(t, 1, 0, 2, 3), 0, 2, 3)), a.transpose(1, 0, 2, 3)[2:3])
    with pytest.raises(JanisHipError):
        hip.Slice(t, 1, 2, 4)
    with pytest.raises(JanisHipError):
        hip.Transpose(t, 0, 1, 1, 3)


def test_concat_and_cast(hip):
    rng = np.random.default_rng(4)
    a = rng.standard_normal((2, 3, 4)).astype(np.float32)
    b = rng.standard_normal((2, 5, 4)).astype(np.float32)
    step("Concat / Cast")
    got = hip.Floats(hip.Concat(hip.FromFloats(a), hip.FromFloats(b), 1))
    assert np.array_equal(got, np.concatenate([a, b], axis=1))
    c = rng.standard_normal((2, 3, 6)).astype(np.float32)
    got = hip.Floats(hip.Concat(hip.Transpose(hip.FromFloats(c), 0, 1, 2), hip.FromFloats(a), 2))
    assert np.array_equal(got, np.concatenate([c, a], axis=2))
    x = (rng.standard_normal(1000) * 100).astype(np.float32)
    assert np.array_equal(hip.Floats(hip.Cast(hip.FromFloats(x), BF16)), _bf16(x))
    assert np.array_equal(hip.Floats(hip.Cast(hip.FromFloats(x), F16)), x.astype(np.float16).astype(np.float32))
    ids = np.arange(12, dtype=np.int32).reshape(3, 4)
    assert np.array_equal(hip.Ints(hip.Transpose(hip.FromInt32(ids), 1, 0)), ids.T)
    with pytest.raises(JanisHipError):
        hip.Cast(hip.FromInt32(ids), F32)


def test_append_kv_grows_like_the_reference(hip):
    """AppendKV(buf, view, n, x): a new buffer for the first call, in-place writes
    while there is room, a grown buffer (view copied in first) when there is
    not; the returned view is always the first n+L tokens."""
    rng = np.random.default_rng(5)
    B, H, D = 1, 2, 128
    hip.ReserveCache(300)
    buf, view, n, hist = None, None, 0, []
    step("AppendKV growth")
    for L in (7, 1, 1, 250, 1, 300):
        x = rng.standard_normal((B, H, L, D)).astype(np.float32)
        hist.append(_bf16(x))
        buf, view = hip.AppendKV(buf, view, n, hip.Cast(hip.FromFloats(x), BF16))
        n += L
        assert view.shape == (B, H, n, D) and buf.shape[2] >= n and buf.shape[2] % hip.KV_STEP == 0
        assert np.array_equal(hip.Floats(view), np.concatenate(hist, axis=2))
    hip.ReserveCache(0)


def test_sdpa_reads_kv_views_in_place(hip, oracle):
    rng = np.random.default_rng(6)
    B, Hq, Hk, D = 1, 8, 2, 128
    k_all = _bf16(rng.standard_normal((B, Hk, 40, D)))
    v_all = _bf16(rng.standard_normal((B, Hk, 40, D)))
    q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    kb, kv = hip.AppendKV(None, None, 0, hip.Cast(hip.FromFloats(k_all), BF16))
    vb, vv = hip.AppendKV(None, None, 0, hip.Cast(hip.FromFloats(v_all), BF16))
    step("SDPA over AppendKV views")
    got = hip.Floats(hip.SDPA(hip.FromFloats(q), hip.Slice(kv, 2, 0, 33), hip.Slice(vv, 2, 0, 33), D ** -0.5, False,
                              out_dtype=F32))
    want = oracle.sdpa(q, k_all[:, :, :33], v_all[:, :, :33], D ** -0.5, False)
    assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max()


def test_sweeper_and_free():
    """On a context of its own, so the tracking does not reach other tests' tensors."""
    from janis_amd.engine import HipBackend
    hb = HipBackend(0)
    try:
        step("Sweeper")
        w = hb.FromFloats(np.ones(16, np.float32))
        hb.PinAll()
        a = hb.FromFloats(np.arange(8, dtype=np.float32))
        b = hb.FromFloats(np.arange(8, dtype=np.float32) * 2)
        hb.Pin(b)
        assert hb.Sweep() >= 1
        assert a.ptr == 0 and b.ptr != 0 and w.ptr != 0
        with pytest.raises(JanisHipError):
            hb.Floats(a)
        assert np.array_equal(hb.Floats(b), np.arange(8) * 2)
        hb.Unpin(b)
        c = hb.FromFloats(np.zeros(4, np.float32))
        hb.Free(c)
        assert c.ptr == 0
        hb.Sweep()
        assert b.ptr == 0 and w.ptr != 0
    finally:
        hb.Close()
