"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every oracle function is checked against at least one of: the reference's own
known answer (cpu/cpu_test.go:121-149), the MLX-produced golden embedding held
by the reference (inkling2/testdata, via tests/golden/), closed forms
(one-hot and all-ones inputs), float64 brute force, and bit-identity between
two independent restatements of the same kernel (scalar lane order vs AVX2
intrinsics).
"""
import os

import numpy as np
import pytest

from janis_amd import synth
from tests.conftest import rel_ok

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def brute_f64(x, q):
    """float64 brute force: dequantize exactly, then a dense product."""
    from oracle import oracle as o

    wd = o.dequantize(q.w, q.s, q.b, q.group_size).astype(np.float64)
    return np.asarray(x, dtype=np.float64) @ wd.T


# -- the reference's only numeric known answer -----------------------------

def test_dequantize_known_answer(oracle):
    """cpu/cpu_test.go:121-149: word 0x87654321, group 4, S={2,0.1}, B={0.5,-1}."""
    w = np.array([[0x87654321]], dtype=np.uint32)
    s = np.array([[2.0, 0.1]], dtype=np.float32)
    b = np.array([[0.5, -1.0]], dtype=np.float32)
    got = oracle.dequantize(w, s, b, 4, 4)
    want = np.array([2.5, 4.5, 6.5, 8.5, -0.5, -0.4, -0.3, -0.2], dtype=np.float32)
    np.testing.assert_allclose(got[0], want, rtol=0, atol=1e-6)
    y = oracle.quant_matmul(np.ones((1, 8), np.float32), w, s, b, 4, 4)
    assert abs(float(y[0, 0]) - 20.6) < 1e-5


def test_dequantize_is_fl32_q_times_s_plus_b(oracle):
    q = synth.quant_linear(11, 16, 256)
    got = oracle.dequantize(q.w, q.s, q.b, 64)
    codes = ((q.w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(16, 256)
    g = np.arange(256) // 64
    want = (codes.astype(np.float32) * q.s[:, g]).astype(np.float32) + q.b[:, g]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


# -- MLX goldens held by the reference -------------------------------------

def _rmsnorm_rows(x, w, eps):
    """cpu/cpu_ops.go:145-162 order in float32."""
    x = x.astype(np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        ss = np.float32(0)
        for v in x[r]:
            ss = np.float32(ss + np.float32(v * v))
        inv = np.float32(1.0) / np.float32(np.sqrt(np.float64(np.float32(ss / np.float32(x.shape[1])) + np.float32(eps))))
        out[r] = (x[r] * inv).astype(np.float32) * w
    return out


@pytest.mark.parametrize("name,tol", [("f32", 2e-4), ("bf16", 5e-2)])
def test_inkling2_embed_golden(oracle, name, tol):
    """inkling2/reference_test.go:100-122: embed = RMSNorm(Dequantize(rows))."""
    fx = np.load(os.path.join(GOLDEN, f"inkling2_embed_{name}.npz"))
    wide = (lambda a, dt: synth.bf16_bits_to_f32(a) if str(dt) == "BF16" else a.astype(np.float32))
    s, b = wide(fx["s"], fx["s_dtype"]), wide(fx["b"], fx["b_dtype"])
    norm = wide(fx["norm"], fx["norm_dtype"])
    rows = fx["w"][fx["tokens"]]
    deq = oracle.dequantize(rows, s[fx["tokens"]], b[fx["tokens"]], int(fx["group_size"]), int(fx["bits"]))
    got = _rmsnorm_rows(deq, norm, float(fx["eps"]))
    ok, d, scale = rel_ok(got, fx["embed"], tol)
    assert ok, (d, scale)


def test_golden_catches_reversed_nibble_order(oracle):
    """A plausible mistake (most-significant nibble first), planted on the CPU
    side, must fail the golden: the fixture pins the code order."""
    fx = np.load(os.path.join(GOLDEN, "inkling2_embed_f32.npz"))
    rows = fx["w"][fx["tokens"]]
    rev = np.zeros_like(rows)
    for l in range(8):
        rev |= ((rows >> np.uint32(4 * l)) & np.uint32(0xF)) << np.uint32(4 * (7 - l))
    deq = oracle.dequantize(rev, fx["s"][fx["tokens"]], fx["b"][fx["tokens"]], 64, 4)
    got = _rmsnorm_rows(deq, fx["norm"], float(fx["eps"]))
    ok, _, _ = rel_ok(got, fx["embed"], 2e-4)
    assert not ok


# -- the per-channel kernel -------------------------------------------------

SHAPES = [(1, 1), (1, 8), (2, 8), (4, 8), (32, 8), (16, 2), (8, 16), (3, 4)]  # cpu/qmv_test.go:40-42


@pytest.mark.parametrize("groups,wpg", SHAPES)
def test_avx2_intrinsics_bit_identical_to_lane_order(oracle, groups, wpg):
    if not oracle.have_avx2_fma():
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(groups * 100 + wpg)
    for _ in range(20):
        n = groups * wpg
        w = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        x = (rng.random(n * 8, dtype=np.float32) * 2 - 1).astype(np.float32)
        s = (rng.random(groups, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
        b = (rng.random(groups, dtype=np.float32) * 0.2 - 0.1).astype(np.float32)
        a = np.float32(oracle.qchannel4("avx2", w, x, s, b, groups, wpg))
        o = np.float32(oracle.qchannel4("avx2_order", w, x, s, b, groups, wpg))
        assert a.view(np.uint32) == o.view(np.uint32)


@pytest.mark.parametrize("groups,wpg", SHAPES)
def test_lane_order_matches_scalar_ref(oracle, groups, wpg):
    """cpu/qmv_test.go:34-70 tolerance 1e-3*(1+|want|), against float64 too."""
    rng = np.random.default_rng(42 + groups * 7 + wpg)
    n = groups * wpg
    w = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    x = (rng.random(n * 8, dtype=np.float32) * 2 - 1).astype(np.float32)
    s = (rng.random(groups, dtype=np.float32) * 0.1 + 0.01).astype(np.float32)
    b = (rng.random(groups, dtype=np.float32) * 0.2 - 0.1).astype(np.float32)
    got = oracle.qchannel4("avx2_order", w, x, s, b, groups, wpg)
    want = oracle.qchannel4("ref", w, x, s, b, groups, wpg)
    assert abs(got - want) <= 1e-3 * (1 + abs(want))
    codes = ((w[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(-1).astype(np.float64)
    gi = np.arange(n * 8) // (wpg * 8)
    exact = float(np.sum(x.astype(np.float64) * (codes * s[gi] + b[gi])))
    assert abs(got - exact) <= 1e-4 * (1 + abs(exact))


def test_one_hot_input_returns_dequantized_column_exactly(oracle):
    """x = e_j: the factored decode kernel reduces to fl32(q*s+b) bit for bit,
    and so does the prefill (wbuf) path. Pins lane mapping and nibble order."""
    q = synth.quant_linear(5, 24, 512)
    deq = oracle.dequantize(q.w, q.s, q.b, 64)
    for j in (0, 1, 7, 8, 63, 64, 200, 511):
        x = np.zeros((1, 512), np.float32)
        x[0, j] = 1.0
        for simd in (True, False):
            y = oracle.quant_matmul(x, q.w, q.s, q.b, 64, simd=simd)[0]
            assert np.array_equal(y.view(np.uint32), deq[:, j].copy().view(np.uint32)), (j, simd)
        x2 = np.repeat(x, 2, axis=0)
        y2 = oracle.quant_matmul(x2, q.w, q.s, q.b, 64)
        assert np.array_equal(y2[1].view(np.uint32), deq[:, j].copy().view(np.uint32))


def test_all_ones_input_closed_form(oracle):
    q = synth.quant_linear(6, 32, 1024)
    codes = ((q.w[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(32, 1024)
    qsum = codes.reshape(32, 16, 64).sum(axis=2).astype(np.float64)
    want = (q.s.astype(np.float64) * qsum + 64.0 * q.b.astype(np.float64)).sum(axis=1)
    for simd in (True, False):
        y = oracle.quant_matmul(np.ones((1, 1024), np.float32), q.w, q.s, q.b, 64, simd=simd)[0]
        ok, d, sc = rel_ok(y, want, 1e-5)
        assert ok, (d, sc)


@pytest.mark.parametrize("rows", [1, 3, 13])
def test_quant_matmul_matches_float64(oracle, rows):
    q = synth.quant_linear(7, 96, 2048)
    _, x = synth.activations(8, (rows, 2048))
    for simd in (True, False):
        y = oracle.quant_matmul(x, q.w, q.s, q.b, 64, simd=simd)
        ok, d, sc = rel_ok(y, brute_f64(x, q), 1e-5)
        assert ok, (rows, simd, d, sc)


def test_quant_matmul_is_linear_in_x(oracle):
    q = synth.quant_linear(9, 64, 1024)
    _, x1 = synth.activations(10, (1, 1024))
    _, x2 = synth.activations(11, (1, 1024))
    y = oracle.quant_matmul((2.0 * x1 + x2).astype(np.float32), q.w, q.s, q.b, 64)
    y1 = oracle.quant_matmul(x1, q.w, q.s, q.b, 64)
    y2 = oracle.quant_matmul(x2, q.w, q.s, q.b, 64)
    ok, d, sc = rel_ok(y, 2.0 * y1.astype(np.float64) + y2, 1e-5)
    assert ok, (d, sc)


@pytest.mark.parametrize("workers", [1, 3, 16])
def test_blocked_go_path(oracle, workers):
    """The 4-channel blocked decode loop (cpu/cpu_misc.go:277-347) with the
    remainder lanes exercised by chunk sizes that are not multiples of 4."""
    q = synth.quant_linear(12, 70, 1024)
    _, x = synth.activations(13, (1, 1024))
    y = oracle.qmv_blocked_go(x[0], q.w, q.s, q.b, 64, workers)
    ok, d, sc = rel_ok(y, brute_f64(x, q)[0], 1e-5)
    assert ok, (d, sc)


def test_generic_width_path_8bit(oracle):
    rng = np.random.default_rng(3)
    N, K, gs = 16, 256, 64
    w = rng.integers(0, 2**32, (N, K // 4), dtype=np.uint64).astype(np.uint32)
    s = (rng.random((N, K // gs), dtype=np.float32) * 0.01).astype(np.float32)
    b = (-rng.random((N, K // gs), dtype=np.float32)).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = oracle.quant_matmul(x, w, s, b, gs, bits=8)
    wd = oracle.dequantize(w, s, b, gs, 8).astype(np.float64)
    ok, d, sc = rel_ok(y[0], x[0].astype(np.float64) @ wd.T, 1e-5)
    assert ok, (d, sc)
    codes = ((w[:, :, None] >> (8 * np.arange(4, dtype=np.uint32))) & 0xFF).reshape(N, K)
    g = np.arange(K) // gs
    qs = (codes.astype(np.float32) * s[:, g]).astype(np.float32)  # rounded product, then the add
    assert np.array_equal(wd.astype(np.float32), (qs + b[:, g]).astype(np.float32))


def test_generic_width_path_2bit(oracle):
    rng = np.random.default_rng(4)
    N, K, gs = 8, 512, 64
    w = rng.integers(0, 2**32, (N, K // 16), dtype=np.uint64).astype(np.uint32)
    s = (rng.random((N, K // gs), dtype=np.float32) * 0.01).astype(np.float32)
    b = (-rng.random((N, K // gs), dtype=np.float32)).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    wd = oracle.dequantize(w, s, b, gs, 2).astype(np.float64)
    codes = ((w[:, :, None] >> (2 * np.arange(16, dtype=np.uint32))) & 0x3).reshape(N, K)
    g = np.arange(K) // gs
    qs = (codes.astype(np.float32) * s[:, g]).astype(np.float32)
    assert np.array_equal(wd.astype(np.float32), (qs + b[:, g]).astype(np.float32))
    for rows in (1, 3):
        xr = np.repeat(x, rows, 0)
        y = oracle.quant_matmul(xr, w, s, b, gs, bits=2)
        ok, d, sc = rel_ok(y, xr.astype(np.float64) @ wd.T, 1e-5)
        assert ok, (rows, d, sc)


# -- gather ------------------------------------------------------------------

@pytest.mark.parametrize("n_lead,A", [(1, 1), (1, 8), (4, 1), (4, 8)])
def test_gather_reduces_to_per_slot_quant_matmul(oracle, n_lead, A):
    E, N, K, k = 6, 40, 512, 8
    q = synth.quant_linear(14, N, K, lead=(E,))
    idx = np.random.default_rng(n_lead * 10 + A).integers(0, E, (n_lead, k)).astype(np.int32)
    _, x = synth.activations(15, (n_lead, A, 1, K))
    y = oracle.gather_quant_matmul(x, q.w, q.s, q.b, idx, 64)
    assert y.shape == (n_lead, k, 1, N)
    for l in range(n_lead):
        for j in range(k):
            e = idx[l, j]
            R = int((idx == e).sum())  # rows the reference batches for this expert
            xv = x[l, 0 if A == 1 else j, 0][None]
            want = oracle.quant_matmul(np.repeat(xv, R, 0), q.w[e], q.s[e], q.b[e], 64)[0]
            assert np.array_equal(y[l, j, 0], want), (l, j, e, R)


def test_gather_rejects_out_of_range_index(oracle):
    q = synth.quant_linear(16, 8, 64, lead=(2,))
    with pytest.raises(IndexError):
        oracle.gather_quant_matmul(np.zeros((1, 1, 1, 64), np.float32), q.w, q.s, q.b,
                                   np.array([[0, 2]], np.int32), 64)


# -- moeApply ------------------------------------------------------------------

def _moe_stacks(seed, E, H, I):
    gate = synth.quant_linear(seed, I, H, lead=(E,))
    up = synth.quant_linear(seed + 1, I, H, lead=(E,))
    down = synth.quant_linear(seed + 2, H, I, lead=(E,))
    return [(q.w, q.s, q.b) for q in (gate, up, down)]


def moe_f64(oracle, x, stacks, idx, scores):
    """float64 brute force of qwen/moe.go:501-511 over exactly dequantized stacks:
    out[t] = sum_k score[t,k] * Wd[e] (silu(Wg[e] x_t) * (Wu[e] x_t))."""
    deq = [[oracle.dequantize(w[e], s[e], b[e], 64).astype(np.float64) for e in range(w.shape[0])]
           for (w, s, b) in stacks]
    x = np.asarray(x, np.float64)
    out = np.zeros((x.shape[0], deq[2][0].shape[0]))
    for t in range(x.shape[0]):
        for k in range(idx.shape[1]):
            e = idx[t, k]
            g, u = deq[0][e] @ x[t], deq[1][e] @ x[t]
            out[t] += scores[t, k] * (deq[2][e] @ (g / (1.0 + np.exp(-g)) * u))
    return out


@pytest.mark.parametrize("n_tok", [1, 3])
def test_moe_apply_matches_float64(oracle, n_tok):
    E, H, I, K = 6, 256, 128, 4
    stacks = _moe_stacks(30, E, H, I)
    _, x = synth.activations(31, (n_tok, H))
    idx, sc = synth.route(32, n_tok, E, K)
    out = oracle.moe_apply(x, *stacks, idx, sc)
    ok, d, s = rel_ok(out, moe_f64(oracle, x, stacks, idx, sc), 1e-4)
    assert ok, (d, s)


def test_moe_apply_is_the_gather_composition(oracle):
    """Bit-identical to composing the pinned gather the way moeApply does:
    g, u with A = 1, h = SiLU(g)*u (cpu/cpu.go:327-329), d with A = K, then
    fl32(fl32(sum_k d*score) / K) * K (cpu/cpu_ops.go:113-142)."""
    E, H, I, K, n = 5, 256, 128, 3, 2
    stacks = _moe_stacks(33, E, H, I)
    _, x = synth.activations(34, (n, H))
    idx, sc = synth.route(35, n, E, K)
    (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = stacks
    g = oracle.gather_quant_matmul(x[:, None, None, :], wg, sg, bg, idx, 64)
    u = oracle.gather_quant_matmul(x[:, None, None, :], wu, su, bu, idx, 64)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    h = ((g / (np.float32(1) + e)).astype(np.float32) * u).astype(np.float32)
    d = oracle.gather_quant_matmul(h, wd, sd, bd, idx, 64)[:, :, 0, :]
    acc = np.zeros((n, H), np.float32)
    for k in range(K):
        acc = (acc + (d[:, k, :] * sc[:, k, None]).astype(np.float32)).astype(np.float32)
    want = ((acc / np.float32(K)).astype(np.float32) * np.float32(K)).astype(np.float32)
    assert np.array_equal(oracle.moe_apply(x, *stacks, idx, sc), want)


def test_moe_f64_catches_swapped_scores(oracle):
    """The float64 check fails on a planted mistake: each slot weighted by its
    neighbour's score."""
    E, H, I, K = 6, 256, 128, 4
    stacks = _moe_stacks(36, E, H, I)
    _, x = synth.activations(37, (1, H))
    idx, sc = synth.route(38, 1, E, K)
    out = oracle.moe_apply(x, *stacks, idx, sc[:, ::-1].copy())
    ok, _, _ = rel_ok(out, moe_f64(oracle, x, stacks, idx, sc), 1e-3)
    assert not ok


def test_moe_apply_rejects_out_of_range_index(oracle):
    stacks = _moe_stacks(39, 2, 256, 128)
    with pytest.raises(IndexError):
        oracle.moe_apply(np.zeros((1, 256), np.float32), *stacks, np.array([[0, 2]], np.int32),
                         np.ones((1, 2), np.float32))


# -- router helpers ------------------------------------------------------------

def test_topk_selection_sort_ties(oracle):
    idx, val = oracle.topk(np.array([2, 2, 9], np.float32), 2)
    assert list(idx) == [2, 1]  # the swap moves index 0 behind index 1
    i2, _ = synth.topk_rows(np.array([[2, 2, 9]], np.float32), 2)
    assert list(i2[0]) == [2, 1]


def test_synth_router_matches_oracle(oracle):
    idx, sc = synth.route(21, 16, 128, 8)
    logits = synth.normal(synth.stream_seed(21, 4), 16 * 128).astype(np.float32).reshape(16, 128)
    for t in range(16):
        p = oracle.softmax_row(logits[t])
        np.testing.assert_allclose(p.sum(), 1.0, rtol=1e-5)
        oi, ov = oracle.topk(p, 8)
        assert list(oi) == list(idx[t])
        np.testing.assert_allclose(sc[t], ov / ov.sum(), rtol=1e-5)
        assert list(oi) == list(np.argsort(-p.astype(np.float64), kind="stable")[:8])


# -- decode-step operators ----------------------------------------------------------

def test_rms_norm_float64_and_weight(oracle):
    rng = np.random.default_rng(50)
    x = rng.standard_normal((5, 4096)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    out = oracle.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    ok, d, sc = rel_ok(out, want, 1e-6)
    assert ok, (d, sc)
    # a planted mistake (weight ignored) fails the same check
    ok, _, _ = rel_ok(oracle.rms_norm(x, np.ones_like(w), 1e-6), want, 1e-6)
    assert not ok


def _rope64(x, dims, traditional, base, offset):
    x = x.astype(np.float64)
    out = x.copy()
    L = x.shape[-2]
    half = dims // 2
    inv = base ** (-np.arange(half) * 2.0 / dims)
    pos = offset + np.arange(L)[:, None]
    th = pos * inv[None, :]
    c, s = np.cos(th), np.sin(th)
    i0 = 2 * np.arange(half) if traditional else np.arange(half)
    i1 = i0 + 1 if traditional else i0 + half
    a, b = x[..., i0], x[..., i1]
    out[..., i0] = a * c - b * s
    out[..., i1] = a * s + b * c
    return out


@pytest.mark.parametrize("traditional", [False, True])
@pytest.mark.parametrize("dims", [128, 64])
def test_rope_float64_and_invariants(oracle, traditional, dims):
    rng = np.random.default_rng(51 + dims)
    x = rng.standard_normal((2, 8, 7, 128)).astype(np.float32)
    out = oracle.rope(x, dims, traditional, 1e6, 1.0, 301)
    ok, d, sc = rel_ok(out, _rope64(x, dims, traditional, 1e6, 301), 2e-5)
    assert ok, (d, sc)
    assert np.array_equal(out[..., dims:], x[..., dims:])  # pass-through
    # position 0 is the identity
    assert np.array_equal(oracle.rope(x[:, :, :1], dims, traditional, 1e6, 1.0, 0), x[:, :, :1])
    # each rotated pair keeps its length
    half = dims // 2
    i0 = 2 * np.arange(half) if traditional else np.arange(half)
    i1 = i0 + 1 if traditional else i0 + half
    n_in = np.hypot(x[..., i0].astype(np.float64), x[..., i1])
    n_out = np.hypot(out[..., i0].astype(np.float64), out[..., i1])
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)


def test_rope_freqs_matches_base_form(oracle):
    """RoPEFreqs with freqs = base^(2i/dims) equals RoPE with that base."""
    x = np.random.default_rng(52).standard_normal((1, 4, 3, 64)).astype(np.float32)
    freqs = (1e4 ** (np.arange(32) * 2.0 / 64)).astype(np.float32)
    a = oracle.rope(x, 64, False, 1e4, 1.0, 17, freqs=freqs)
    b = oracle.rope(x, 64, False, 1e4, 1.0, 17)
    ok, d, sc = rel_ok(a, b, 1e-5)
    assert ok, (d, sc)


def _sdpa64(q, k, v, scale, causal):
    B, Hq, Lq, Dh = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    g = Hq // Hk
    kk = np.repeat(k.astype(np.float64), g, axis=1)
    vv = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk) * scale
    if causal:
        mask = np.arange(Lk)[None, :] > (Lk - Lq) + np.arange(Lq)[:, None]
        s = np.where(mask, -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, vv)


@pytest.mark.parametrize("Hq,Hk,Lq,Lk,causal", [(8, 2, 1, 37, False), (8, 2, 1, 37, True), (4, 4, 6, 6, True),
                                               (6, 3, 5, 13, True), (4, 1, 3, 9, False)])
def test_sdpa_float64(oracle, Hq, Hk, Lq, Lk, causal):
    rng = np.random.default_rng(Hq * 100 + Lk)
    q = rng.standard_normal((2, Hq, Lq, 64)).astype(np.float32)
    k = rng.standard_normal((2, Hk, Lk, 64)).astype(np.float32)
    v = rng.standard_normal((2, Hk, Lk, 64)).astype(np.float32)
    out = oracle.sdpa(q, k, v, 64 ** -0.5, causal)
    ok, d, sc = rel_ok(out, _sdpa64(q, k, v, 64 ** -0.5, causal), 1e-5)
    assert ok, (d, sc)


def test_sdpa_invariants(oracle):
    rng = np.random.default_rng(53)
    q = rng.standard_normal((1, 4, 4, 32)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 2, 1, 32)).astype(np.float32), 10, axis=2)
    v = rng.standard_normal((1, 2, 10, 32)).astype(np.float32)
    # identical keys: every query gets the mean of the values (non-causal)
    out = oracle.sdpa(q, k, v, 0.2, False)
    np.testing.assert_allclose(out, np.repeat(v.mean(axis=2, keepdims=True), 2, axis=1).repeat(4, axis=2),
                               rtol=1e-5, atol=1e-6)
    # causal: keys after a row's limit do not change that row
    k2 = rng.standard_normal((1, 2, 10, 32)).astype(np.float32)
    a = oracle.sdpa(q, k2, v, 0.2, True)
    k3, v3 = k2.copy(), v.copy()
    k3[:, :, 9], v3[:, :, 9] = 100.0, -100.0  # only the last row may see key 9
    b = oracle.sdpa(q, k3, v3, 0.2, True)
    assert np.array_equal(a[:, :, :3], b[:, :, :3]) and not np.array_equal(a[:, :, 3], b[:, :, 3])


def test_silu_and_argmax(oracle):
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    ok, d, sc = rel_ok(oracle.silu(x), x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64))), 1e-6)
    assert ok, (d, sc)
    t = np.array([[1, 5, 5, 2], [-np.inf, -np.inf, -np.inf, -np.inf], [np.nan, 1, 3, 3]], np.float32)
    assert list(oracle.argmax(t)) == [1, 0, 2]


def test_scatter_rows_known_answer(oracle):
    """ScatterRows (cpu/cpu_ops.go:215-233) on a hand-worked case: rows 2 and 0
    replaced, row 2 twice (the later update stays), rows 1 and 3 untouched."""
    dst = np.arange(12, dtype=np.uint32).reshape(4, 3)
    upd = np.array([[100, 101, 102], [200, 201, 202], [300, 301, 302]], dtype=np.uint32)
    want = np.array([[200, 201, 202], [3, 4, 5], [300, 301, 302], [9, 10, 11]], dtype=np.uint32)
    got = oracle.scatter_rows(dst, [2, 0, 2], upd)
    assert np.array_equal(got, want)
    assert np.array_equal(dst, np.arange(12, dtype=np.uint32).reshape(4, 3))  # dst itself unchanged
    assert np.array_equal(oracle.scatter_rows(dst, [], np.zeros((0, 3), np.uint32)), dst)
    with pytest.raises(IndexError):
        oracle.scatter_rows(dst, [4], upd[:1])


# -- the operators around the products: transpose=false, Softmax, Mean, Scalar ------------

@pytest.mark.parametrize("rows,n,k,gs,bits", [(1, 64, 256, 64, 4), (3, 40, 64, 16, 2), (2, 32, 128, 32, 8),
                                              (2, 8, 16, 8, 4)])
def test_matmul_dequant_matches_float64(oracle, rows, n, k, gs, bits):
    """MatMul(x, Dequantize(w)) (cpu/cpu_misc.go:233-236) against the float64
    product with the exactly dequantized matrix: x [rows, n] . W [n, k]."""
    q = synth.quant_linear(3100 + n, n, k, gs, bits=bits)
    _, x = synth.activations(3101 + rows, (rows, n))
    got = oracle.matmul_dequant(x, q.w, q.s, q.b, gs, bits)
    wd = oracle.dequantize(q.w, q.s, q.b, gs, bits).astype(np.float64)
    ok, d, sc = rel_ok(got, x.astype(np.float64) @ wd, 1e-5)
    assert ok, (d, sc)


def test_matmul_dequant_catches_transposed_operand(oracle):
    """A planted mistake -- the matrix used transposed, as the transpose=true
    path reads it -- fails the float64 check on a square matrix."""
    q = synth.quant_linear(3110, 64, 64, 32)
    _, x = synth.activations(3111, (2, 64))
    wd = oracle.dequantize(q.w, q.s, q.b, 32).astype(np.float64)
    wrong = oracle.quant_matmul(x, q.w, q.s, q.b, 32)  # x . W^T
    assert not rel_ok(wrong, x.astype(np.float64) @ wd, 1e-2)[0]
    assert rel_ok(oracle.matmul_dequant(x, q.w, q.s, q.b, 32), x.astype(np.float64) @ wd, 1e-5)[0]


def test_matmul_dequant_skips_zero_inputs(oracle):
    """cpu/cpu_ops.go:41-43 skips a zero x term, so a NaN weight row met only by
    x == 0 leaves the result finite (the float64 product would be NaN)."""
    q = synth.quant_linear(3120, 16, 64, 64)
    q.s_bits[5, 0] = 0x7FC0
    _, x = synth.activations(3121, (2, 16))
    x[:, 5] = 0
    got = oracle.matmul_dequant(x, q.w, q.s, q.b, 64)
    assert np.isfinite(got).all()
    x[1, 5] = 1.0
    assert np.isnan(oracle.matmul_dequant(x, q.w, q.s, q.b, 64)[1, :64]).all()


def test_gather_matmul_dequant_is_per_slot(oracle):
    q = synth.quant_linear(3130, 48, 64, 32, lead=(4,))
    idx = np.array([[0, 3, 3], [2, 1, 0]], np.int32)
    _, x = synth.activations(3131, (2, 3, 48))
    got = oracle.gather_matmul_dequant(x, q.w, q.s, q.b, idx, 32)
    for l in range(2):
        for k in range(3):
            e = idx[l, k]
            assert np.array_equal(got[l, k], oracle.matmul_dequant(x[l, k][None], q.w[e], q.s[e], q.b[e], 32)[0])
    with pytest.raises(IndexError):
        oracle.gather_matmul_dequant(x, q.w, q.s, q.b, np.array([[0, 4, 1], [0, 0, 0]], np.int32), 32)


@pytest.mark.parametrize("shape,axis", [((6, 128), -1), ((3, 7, 5), 1), ((4, 3), 0)])
def test_softmax_along_axis_float64(oracle, shape, axis):
    _, x = synth.activations(3140 + len(shape), shape)
    got = oracle.softmax(x, axis)
    e = np.exp(x.astype(np.float64) - x.max(axis=axis, keepdims=True))
    ok, d, sc = rel_ok(got, e / e.sum(axis=axis, keepdims=True), 1e-6)
    assert ok, (d, sc)
    # each line through the pinned softmax_row
    assert np.array_equal(np.moveaxis(got, axis, -1)[0, ...].reshape(-1, shape[axis])[0],
                          oracle.softmax_row(np.moveaxis(x, axis, -1)[0, ...].reshape(-1, shape[axis])[0]))


def test_mean_sequential_order_known_answer(oracle):
    """cpu/cpu_ops.go:136-140 sums in index order in fp32: 1e8 + 1 rounds back
    to 1e8, so [1e8, 1, -1e8, 1] averages to 0.25 (the exact mean is 0.5, a
    pairwise sum gives 0)."""
    assert oracle.mean(np.array([1e8, 1, -1e8, 1], np.float32), 0) == np.float32(0.25)
    _, x = synth.activations(3150, (4, 9, 33))
    for ax in (0, 1, 2):
        ok, d, sc = rel_ok(oracle.mean(x, ax), x.astype(np.float64).mean(axis=ax), 1e-6)
        assert ok, (ax, d, sc)


def test_scalar_ops_closed_form(oracle):
    x = np.array([1.5, -2.0, 3.0e38, 0.1], np.float32)
    assert np.array_equal(oracle.scalar_mul(x, 2.0), np.array([3.0, -4.0, np.inf, 0.2], np.float32))
    assert np.array_equal(oracle.scalar_add(x, 1.0), np.array([2.5, -1.0, 3.0e38, 1.1], np.float32))
