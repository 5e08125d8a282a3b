"""GPU checks of the layout operators of the engine mirror -- Slice, Transpose,
ExpandDims (views), Reshape of a view, Concat, Cast (jh_copy_strided) -- and of
the engine capabilities built on them: KVAppender (engine/backend.go:56-61, the
MLX backend's growth rule mlxc/mlxc.go:283-306) and Sweeper / Freer
(engine/backend.go:43-93). Copies are exact; casts round to nearest even."""
import numpy as np
import pytest

from janis_amd import synth
from janis_amd.engine import BF16, F16, F32, I32, U32, JanisHipError
from tests.conftest import rel_ok, step

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


def _raw(hip, t, dtype, shape):
    return np.frombuffer(hip.Bytes(t), dtype=dtype).reshape(shape)


@pytest.mark.parametrize("dt,np_dt,shape,n_idx", [
    (U32, np.uint32, (37, 129), 11),          # 516-byte rows: 4-byte words
    (BF16, np.uint16, (16, 24), 20),          # 48-byte rows: 16-byte words
    (F32, np.float32, (5, 70001), 7),         # rows over several 64 KiB chunks
    (U32, np.uint32, (600, 8), 700),          # more indices than one launch takes
])
def test_scatter_rows_matches_oracle(hip, oracle, dt, np_dt, shape, n_idx):
    """RowScatterer.ScatterRows (engine/backend.go:95-105) against the CPU
    semantics (cpu/cpu_ops.go:215-233), bit-exact, with repeated indices (the
    last update stays) and dst left as it was."""
    rng = np.random.default_rng(shape[0] * 7 + n_idx)
    dst = rng.integers(0, 2**16 if np_dt == np.uint16 else 2**31, shape).astype(np_dt)
    idx = rng.integers(0, shape[0], n_idx).astype(np.int32)
    upd = rng.integers(0, 2**16 if np_dt == np.uint16 else 2**31, (n_idx,) + shape[1:]).astype(np_dt)
    td, tu = hip.FromRaw(dt, dst, *shape), hip.FromRaw(dt, upd, n_idx, *shape[1:])
    step(f"jh_scatter_rows {shape} n_idx={n_idx}")
    out = hip.ScatterRows(td, idx, tu)
    assert tuple(out.shape) == shape
    assert np.array_equal(_raw(hip, out, np_dt, shape), oracle.scatter_rows(dst, idx, upd))
    assert np.array_equal(_raw(hip, td, np_dt, shape), dst)


def test_scatter_rows_edges(hip, oracle):
    """No indices (a copy), a U8 tensor (1-byte words), in place through the
    C ABI (out == dst), and out-of-range indices rejected before any write."""
    import ctypes

    from janis_amd.engine import U8
    rng = np.random.default_rng(5)
    dst = rng.integers(0, 255, (9, 7)).astype(np.uint8)
    td = hip.FromRaw(U8, dst, 9, 7)
    step("jh_scatter_rows empty / u8 / in place / out of range")
    assert np.array_equal(_raw(hip, hip.ScatterRows(td, [], hip.FromRaw(U8, np.zeros((0, 7), np.uint8), 0, 7)),
                               np.uint8, (9, 7)), dst)
    upd = rng.integers(0, 255, (3, 7)).astype(np.uint8)
    got = _raw(hip, hip.ScatterRows(td, [8, 0, 4], hip.FromRaw(U8, upd, 3, 7)), np.uint8, (9, 7))
    assert np.array_equal(got, oracle.scatter_rows(dst, [8, 0, 4], upd))
    idx = np.array([3, 3, 1], np.int32)
    tu = hip.FromRaw(U8, upd, 3, 7)
    rc = hip._L.jh_scatter_rows(hip._ctx, td.ptr, td.ptr, 9, 7, idx.ctypes.data_as(ctypes.c_void_p), 3, tu.ptr)
    assert rc == 0
    assert np.array_equal(_raw(hip, td, np.uint8, (9, 7)), oracle.scatter_rows(dst, idx, upd))
    before = _raw(hip, td, np.uint8, (9, 7)).copy()
    for bad in ([9], [-1], [0, 2, 12]):
        with pytest.raises(JanisHipError):
            hip.ScatterRows(td, bad, hip.FromRaw(U8, upd[:len(bad)], len(bad), 7))
    with pytest.raises(JanisHipError):
        hip.ScatterRows(td, [1, 2], tu)  # 3 update rows for 2 indices
    assert np.array_equal(_raw(hip, td, np.uint8, (9, 7)), before)


def test_slot_cache_scatter_then_gather(hip, oracle):
    """The MoE slot cache's use of ScatterRows (qwen/slotcache.go:60-186): the
    missed experts' W / scales / biases rows land in victim slots of persistent
    [slots, ...] stacks, and GatherQuantMatmul over the slot stacks with slot
    indices equals the gather over the full expert stacks with expert indices."""
    E, S, n, k = 12, 5, 64, 512
    q = synth.quant_linear(81, n, k, lead=(E,))
    w, s, b = (hip.FromRaw(U32, q.w, *q.w.shape), hip.FromBF16Bits(q.s_bits, *q.s_bits.shape),
               hip.FromBF16Bits(q.b_bits, *q.b_bits.shape))
    slots = [hip.FromRaw(U32, np.zeros((S,) + q.w.shape[1:], np.uint32), S, *q.w.shape[1:]),
             hip.FromBF16Bits(np.zeros((S,) + q.s_bits.shape[1:], np.uint16), S, *q.s_bits.shape[1:]),
             hip.FromBF16Bits(np.zeros((S,) + q.b_bits.shape[1:], np.uint16), S, *q.b_bits.shape[1:])]
    slot_of = {}
    xb, x = synth.activations(82, (1, 1, 1, k))
    for tok, experts in enumerate(([3, 7, 1], [7, 9, 3], [11, 0, 9])):
        miss = [e for e in experts if e not in slot_of]
        held = {slot_of[e] for e in experts if e in slot_of}
        free = [v for v in range(S) if v not in slot_of.values()] + \
               [v for v in range(S) if v in slot_of.values() and v not in held]
        victims = free[:len(miss)]
        for v in victims:
            slot_of = {e: sl for e, sl in slot_of.items() if sl != v}
        for e, v in zip(miss, victims):
            slot_of[e] = v
        ids = np.array(miss, np.int32)
        step(f"slot cache token {tok}: miss {miss} -> slots {victims}")
        slots = [hip.ScatterRows(t, victims, hip.TakeAxis(src, hip.FromInt32(ids), 0))
                 for t, src in zip(slots, (w, s, b))]
        sidx = np.array([[slot_of[e] for e in experts]], np.int32)
        y = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, 1, 1, 1, k), *slots, hip.FromInt32(sidx),
                                             True, 64, 4, out_dtype=F32))
        full = hip.Floats(hip.GatherQuantMatmul(hip.FromBF16Bits(xb, 1, 1, 1, k), w, s, b,
                                                hip.FromInt32(np.array([experts], np.int32)), True, 64, 4,
                                                out_dtype=F32))
        assert np.array_equal(y, full), tok
        want = oracle.gather_quant_matmul(x, q.w, q.s, q.b, np.array([experts], np.int32), 64)
        ok, d, sc = rel_ok(y, want, 1e-3)
        assert ok, (tok, d, sc)
