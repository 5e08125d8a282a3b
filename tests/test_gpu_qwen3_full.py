"""BASELINE config 4 at its stated size: the full Qwen3-8B-architecture decode
step (36 layers, hidden 4096, 32 query / 8 KV heads, head_dim 128, SwiGLU
intermediate 12288, vocab 151936, RMSNorm eps 1e-6, RoPE theta 1e6) on seeded
random 4-bit weights, with the bf16 KV caches filled with seeded N(0,1) to
context 512 and 8192, one new token decoded on the GPU and compared with the
same step composed from the oracle's operators (qwen/model.go:294-303,
qwen/block.go:58-61, qwen/attention.go:98-128, qwen/mlp.go:32-36).

The weights are generated once on the device and copied to the host for the
oracle (4.3 GB), so both sides read the same bits. The GPU feeds bf16 inputs
to the products (fp32 activations rounded in registers) and keeps bf16 or f16
caches; the oracle is fp32 throughout. The logits are held to TOL of
max|logit| and the GPU's greedy token must be one the oracle scores within
TOL * max|logit| of its best. The unfused case is the reference's own call
sequence and dtype flow: F32 activations from Dequantize on, and the f16
caches KVCache.Update's cast makes on this backend (qwen/cache.go:90-93).
"""
import numpy as np
import pytest

from janis_amd.engine import F16
from janis_amd.qwen3_decode import Qwen3Config, decode_step, random_model
from tests.conftest import rel_ok, step

pytestmark = pytest.mark.gpu

# the north star's bar (relOK, ggml/ggml_test.go:56-65)
TOL = 1e-2


class _Q:
    def __init__(self, w, s, b):
        self.w, self.s, self.b = w, s, b


def _host_quant(t3):
    w, s, b = (t._keep for t in t3)
    return _Q(w.cpu().numpy().view(np.uint32), s.float().cpu().numpy(), b.float().cpu().numpy())


@pytest.fixture(scope="module")
def full_model(hip):
    import torch

    cfg = Qwen3Config()
    dev = torch.device("cuda:0")
    cap = 8192 + 1
    step("building the full Qwen3-8B-shape model on the device (seeded)")
    torch.manual_seed(2024)
    m, _ = random_model(hip, cfg, cap, seed=11, torch=torch, dev=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(2025)
    for L in m.layers:
        L.k_cache._keep.normal_(generator=g)
        L.v_cache._keep.normal_(generator=g)
    torch.cuda.synchronize()
    step("copying the weights to the host for the oracle")
    host = {"embed": _host_quant(m.embed), "lm_head": _host_quant(m.lm_head),
            "norm": m.norm._keep.float().cpu().numpy()}
    for l, L in enumerate(m.layers):
        for name in ("qkv", "o", "gate_up", "down"):
            host[f"l{l}.{name}"] = _host_quant(getattr(L, name))
        for name in ("in_norm", "post_norm", "q_norm", "k_norm"):
            host[f"l{l}.{name}"] = getattr(L, name)._keep.float().cpu().numpy()
    yield cfg, m, host
    del m, host
    torch.cuda.empty_cache()


def _with_f16_caches(hip, m, ctx):
    """The same model with f16 caches of ctx + 8 rows holding the bf16 caches'
    first ctx rows (converted), as a copy of the model's layer list."""
    import copy

    import torch

    m2 = copy.copy(m)
    m2.layers = []
    for L in m.layers:
        L2 = copy.copy(L)
        for name in ("k_cache", "v_cache"):
            src = getattr(L, name)._keep
            t = torch.zeros((1, src.shape[1], ctx + 8, src.shape[3]), dtype=torch.float16, device=src.device)
            t[:, :, :ctx] = src[:, :, :ctx].to(torch.float16)
            setattr(L2, name, hip.Wrap(t.data_ptr(), tuple(t.shape), F16, keep=t))
        m2.layers.append(L2)
    torch.cuda.synchronize()
    return m2


def _oracle_step(o, cfg, host, m, token, pos):
    """The step composed from the pinned oracle operators; the cache rows
    before pos are read from the GPU's caches, the row at pos is the
    oracle's own key and value."""
    gs, eps = cfg.group_size, cfg.eps
    Hq, Hk, Dh, I = cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.inter
    e = host["embed"]
    h = o.dequantize(e.w[[token]], e.s[[token]], e.b[[token]], gs)  # [1, H]
    for l in range(cfg.layers):
        q_ = lambda n: host[f"l{l}.{n}"]
        L = m.layers[l]
        xn = o.rms_norm(h, q_("in_norm"), eps)
        w = q_("qkv")
        qkv = o.quant_matmul(xn, w.w, w.s, w.b, gs)[0]
        q = o.rms_norm(qkv[:Hq * Dh].reshape(1, Hq, 1, Dh), q_("q_norm"), eps)
        k = o.rms_norm(qkv[Hq * Dh:(Hq + Hk) * Dh].reshape(1, Hk, 1, Dh), q_("k_norm"), eps)
        v = qkv[(Hq + Hk) * Dh:].reshape(1, Hk, 1, Dh)
        q = o.rope(q, Dh, False, cfg.theta, 1.0, pos)
        k = o.rope(k, Dh, False, cfg.theta, 1.0, pos)
        kc = np.concatenate([L.k_cache._keep[:, :, :pos].float().cpu().numpy(), k], axis=2)
        vc = np.concatenate([L.v_cache._keep[:, :, :pos].float().cpu().numpy(), v], axis=2)
        att = o.sdpa(q, kc, vc, Dh ** -0.5, False).reshape(1, Hq * Dh)
        w = q_("o")
        h = (h + o.quant_matmul(att, w.w, w.s, w.b, gs)).astype(np.float32)
        xn = o.rms_norm(h, q_("post_norm"), eps)
        w = q_("gate_up")
        gu = o.quant_matmul(xn, w.w, w.s, w.b, gs)[0]
        act = (o.silu(gu[:I]) * gu[I:]).astype(np.float32)[None]
        w = q_("down")
        h = (h + o.quant_matmul(act, w.w, w.s, w.b, gs)).astype(np.float32)
    hn = o.rms_norm(h, host["norm"], eps)
    w = host["lm_head"]
    return o.quant_matmul(hn, w.w, w.s, w.b, gs)[0]


@pytest.mark.parametrize("ctx,fused,cache", [(512, True, "bf16"), (512, False, "bf16"), (512, False, "f16"),
                                             (512, True, "f16"), (8192, True, "bf16")])
def test_qwen3_8b_full_decode_step(hip, oracle, full_model, ctx, fused, cache):
    cfg, m, host = full_model
    token = 1234
    if cache == "f16":
        step(f"f16 copies of the caches' first {ctx} rows")
        m = _with_f16_caches(hip, m, ctx)
    step(f"oracle: full Qwen3-8B step at ctx {ctx} (cache {cache})")
    want = _oracle_step(oracle, cfg, host, m, token, ctx)
    step(f"GPU: full Qwen3-8B decode step at ctx {ctx} fused={fused} cache={cache}")
    logits, nxt = decode_step(hip, m, hip.FromInt32(np.array([token], np.int32)), ctx, fused=fused)
    got = hip.Floats(logits).reshape(-1)
    assert got.shape == (cfg.vocab,) and np.isfinite(got).all()
    ok, d, sc = rel_ok(got, want, TOL)
    print(f"  ctx {ctx} fused={fused} cache={cache}: max|diff| {d:.4g} of max|logit| {sc:.4g} ({d / sc:.2e})",
          flush=True)
    assert ok, (d, sc)
    g = int(hip.Ints(nxt).reshape(-1)[0])
    assert g == int(np.argmax(got))
    # the GPU's greedy token is one the oracle scores within TOL of its best
    assert want[g] >= want.max() - TOL * sc, (g, int(np.argmax(want)), float(want.max() - want[g]))
