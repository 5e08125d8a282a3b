"""One Qwen3 decode step on the HIP backend, written against the engine mirror
the way the reference's model code is written against engine.Backend:
forwardCachedT (qwen/model.go:294-303) -> Block.ForwardCached
(qwen/block.go:58-61) -> Attention.ForwardCached (qwen/attention.go:98-128) and
MLP.Forward (qwen/mlp.go:32-36). It is the caller above the boundary, kept here
only to drive the decode-step operators for tests and measurement.

Two layout choices, both exact: q/k/v rows are stacked into one quantized matrix
and gate/up into another at load time (QuantMatmul rows are independent, so one
launch gives the same numbers as three or two), and the residual stream stays
fp32 while the inputs of the quantized products are bf16.
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .engine import BF16, F16, F32, I32, HipBackend, Tensor


@dataclass
class Qwen3Config:
    hidden: int = 4096
    inter: int = 12288
    n_heads: int = 32
    n_kv: int = 8
    head_dim: int = 128
    vocab: int = 151936
    layers: int = 36
    eps: float = 1e-6
    theta: float = 1e6
    group_size: int = 64
    bits: int = 4
    tie: bool = False   # lm_head tied to the embedding (QuantEmbedding.AsLinear)


@dataclass
class Qwen3Layer:
    qkv: tuple          # (W, S, B) [(Hq+2Hk)*Dh, hidden/8]
    o: tuple            # [hidden, Hq*Dh/8]
    gate_up: tuple      # [2*inter, hidden/8]: the gate rows, then the up rows
    down: tuple         # [hidden, inter/8]
    in_norm: Tensor     # [hidden]
    post_norm: Tensor   # [hidden]
    q_norm: Tensor      # [head_dim]
    k_norm: Tensor      # [head_dim]
    k_cache: Tensor     # [1, Hk, capacity, Dh] bf16
    v_cache: Tensor


@dataclass
class Qwen3Model:
    cfg: Qwen3Config
    embed: tuple        # QuantEmbedding (W, S, B) [vocab, hidden/8]
    layers: list = field(default_factory=list)
    norm: Tensor = None
    lm_head: tuple = None  # None: tied to the embedding (QuantEmbedding.AsLinear)


def decode_step(b: HipBackend, m: Qwen3Model, token: Tensor, pos: int, fused: bool = True) -> tuple:
    """Runs token (I32 [1], device) at position pos through every layer, appends
    its keys/values to the caches, returns (logits F32 [1, vocab], next token I32 [1]).
    fused=True takes the backend's fused operators: each RMSNorm split between
    the product that makes the residual stream (its epilogue writes bf16(h*w)
    and the sum of h^2) and the product that reads it (which applies the
    1/rms factor to its output), SiLU*mul in the gate/up product's epilogue,
    the residual adds in the o/down products' epilogues, and the q/k norms,
    RoPE, KV append and SDPA in the q/k/v product's launch, whose split
    partials are merged inside it (4 launches per layer; on GPUs that do not
    deal workgroups to their XCDs round-robin the product and the attention
    are separate launches, with a merge launch), and the embedding row, the
    first norm's producer half and the RoPE factors in one launch.
    fused=False makes the reference's calls one for one (qwen/block.go,
    qwen/attention.go, qwen/mlp.go, qwen/cache.go), with engine.Backend's own
    parameters only: separate q/k/v and gate/up products on row views of the
    stacked matrices, Reshape/Transpose views, KVCache.Update's F16 cast and the
    KVAppender, SDPA over the cache views. Its activations are F32 (Dequantize's
    dtype, kept by every operator), as unchanged janis model code makes them."""
    c = m.cfg
    gs, bits = c.group_size, c.bits
    H, Hq, Hk, Dh, I = c.hidden, c.n_heads, c.n_kv, c.head_dim, c.inter
    NORMED, SWIGLU, RESID_NORM = _lib.JH_PRO_NORMED, _lib.JH_EPI_SWIGLU, _lib.JH_EPI_RESID_NORM
    ew, es, eb = m.embed
    head = m.lm_head if m.lm_head is not None else m.embed
    if fused:
        # QuantEmbedding.Forward (qwen/embed.go:78-83), the first block's
        # InputNorm (producer half) and the RoPE factors shared by every layer,
        # in one launch
        h, u, st, cs = b.EmbedNormPrepare(token, ew, es, eb, gs, bits, m.layers[0].in_norm,
                                          rope=(Dh, c.theta, 1.0, pos))
        qkv_buf = b.empty(F32, 1, (Hq + 2 * Hk) * Dh)
        for li, L in enumerate(m.layers):
            nxt = m.layers[li + 1].in_norm if li + 1 < len(m.layers) else m.norm
            att = b.QkvAttentionDecode(u, st, c.eps, *L.qkv, gs, bits, qkv_buf, Hq, Hk, L.q_norm, L.k_norm, c.eps,
                                       c.theta, 1.0, pos, L.k_cache, L.v_cache, Dh ** -0.5, rope_cs=cs,
                                       out_dtype=BF16)
            b.QuantMatvecFused(att, *L.o, gs, bits, norm=L.post_norm, epilogue=RESID_NORM, resid=h, out=h,
                               stats=st, norm_out=u)
            act = b.QuantMatvecFused(u, *L.gate_up, gs, bits, NORMED, eps=c.eps, stats=st, epilogue=SWIGLU,
                                     out_dtype=BF16)
            b.QuantMatvecFused(act, *L.down, gs, bits, norm=nxt, epilogue=RESID_NORM, resid=h, out=h, stats=st,
                               norm_out=u)
        logits = b.QuantMatvecFused(u, *head, gs, bits, NORMED, eps=c.eps, stats=st, out_dtype=F32)
        return logits, b.Argmax(logits)
    # The reference's operator sequence, call for call, with the dtype flow its
    # unchanged model code produces on this backend: every result takes its
    # input's dtype, so the F32 row Dequantize returns keeps the activations
    # F32 throughout (the products' fp32 x takes the same decode tiles, rounded
    # to bf16 in registers), and KVCache.Update casts the F32 keys and values to
    # F16 because this backend is a RawReader (qwen/cache.go:90-93).
    # QuantEmbedding.Forward (qwen/embed.go:78-83), forwardCachedT's reshape
    # (qwen/model.go:294-303)
    B, T = 1, 1
    h = b.Reshape(b.Dequantize(b.TakeAxis(ew, token, 0), b.TakeAxis(es, token, 0), b.TakeAxis(eb, token, 0), gs,
                               bits), B, T, H)
    for L in m.layers:
        # Block.ForwardCached (qwen/block.go:58-61): h = x + Attn(InputNorm(x))
        x = h
        xn = b.RMSNorm(x, L.in_norm, c.eps)
        # Attention.ForwardCached (qwen/attention.go:98-128)
        wq, wk, wv = (_linear_rows(b, L.qkv, r0, n) for r0, n in ((0, Hq * Dh), (Hq * Dh, Hk * Dh),
                                                                    ((Hq + Hk) * Dh, Hk * Dh)))
        q = b.Reshape(b.QuantMatmul(xn, *wq, True, gs, bits), B, T, Hq, Dh)
        k = b.Reshape(b.QuantMatmul(xn, *wk, True, gs, bits), B, T, Hk, Dh)
        q, k = b.RMSNorm(q, L.q_norm, c.eps), b.RMSNorm(k, L.k_norm, c.eps)
        q, k = b.Transpose(q, 0, 2, 1, 3), b.Transpose(k, 0, 2, 1, 3)
        v = b.Transpose(b.Reshape(b.QuantMatmul(xn, *wv, True, gs, bits), B, T, Hk, Dh), 0, 2, 1, 3)
        q = b.RoPE(q, Dh, False, c.theta, 1.0, pos)
        k = b.RoPE(k, Dh, False, c.theta, 1.0, pos)
        k, v = kv_cache_update(b, L, pos, k, v)
        att = b.SDPA(q, k, v, Dh ** -0.5, T > 1)
        att = b.Reshape(b.Transpose(att, 0, 2, 1, 3), B, T, Hq * Dh)
        h = b.Add(x, b.QuantMatmul(att, *_linear_rows(b, L.o, 0, H), True, gs, bits))
        # MLP.Forward (qwen/mlp.go:32-36) on PostNorm(h), and the second residual add
        xn = b.RMSNorm(h, L.post_norm, c.eps)
        gate = b.SiLU(b.QuantMatmul(xn, *_linear_rows(b, L.gate_up, 0, I), True, gs, bits))
        up = b.QuantMatmul(xn, *_linear_rows(b, L.gate_up, I, I), True, gs, bits)
        h = b.Add(h, b.QuantMatmul(b.Mul(gate, up), *_linear_rows(b, L.down, 0, H), True, gs, bits))
    # forwardCachedT's final norm, last position, head (qwen/model.go:294-303, 271-276)
    h = b.Slice(b.RMSNorm(h, m.norm, c.eps), 1, T - 1, T)
    logits = b.QuantMatmul(h, *head, True, gs, bits)
    return b.Reshape(logits, 1, -1), b.Argmax(logits, -1)


def kv_cache_update(b: HipBackend, L: Qwen3Layer, n: int, k: Tensor, v: Tensor) -> tuple:
    """KVCache.Update (qwen/cache.go:90-98) on this backend: it is an
    engine.RawReader, so F32 keys and values are cast to F16 first; then
    KVAppender.AppendKV writes them at token n of the layer's spare-room buffers
    (the model's caches; their first n tokens are the current views) and the
    views of the first n + L tokens come back."""
    if b.DTypeOf(k) == F32:
        k, v = b.Cast(k, F16), b.Cast(v, F16)
    _, kview = b.AppendKV(L.k_cache, b.Slice(L.k_cache, 2, 0, n), n, k)
    _, vview = b.AppendKV(L.v_cache, b.Slice(L.v_cache, 2, 0, n), n, v)
    return kview, vview


def _linear_rows(b: HipBackend, lin: tuple, r0: int, n: int) -> tuple:
    """Rows r0..r0+n of a stacked quantized matrix (W, S, B): one of the
    reference's separate QuantLinears (q/k/v or gate/up) as Slice views."""
    return tuple(b.Slice(t, 0, r0, r0 + n) for t in lin)


def random_model(b: HipBackend, cfg: Qwen3Config, capacity: int, seed: int = 0, torch=None, dev=None,
                 cache_dtype: int = BF16):
    """Random-init weights of the architecture (codes uniform 0..15, scales
    |N(0,1)|*0.02, biases -8*scale + N(0, 1e-3), norm weights 1 + N(0, 0.05))
    and zeroed caches of `capacity` rows (bf16, or f16: the dtype
    KVCache.Update's cast gives F32 keys on this backend). With torch given, everything is
    generated on the device (the 8B model in seconds); otherwise with numpy from
    janis_amd.synth and uploaded (small models). Returns (model, host copies or
    None)."""
    from . import synth
    from .engine import U32
    gs = cfg.group_size
    H, Hq, Hk, Dh, I = cfg.hidden, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.inter
    host = {} if torch is None else None

    def qlin(name, n, k):
        if torch is not None:
            shape = (n, k // 8)
            w = torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev)
            s = (torch.randn((n, k // gs), device=dev).abs() * 0.02).to(torch.bfloat16)
            bb = (-8.0 * s.float() + torch.randn((n, k // gs), device=dev) * 1e-3).to(torch.bfloat16)
            return (b.Wrap(w.data_ptr(), shape, U32, keep=w), b.Wrap(s.data_ptr(), s.shape, BF16, keep=s),
                    b.Wrap(bb.data_ptr(), bb.shape, BF16, keep=bb))
        q = synth.quant_linear(synth.stream_seed(seed, zlib.crc32(name.encode())), n, k, gs)
        host[name] = q
        return (b.FromRaw(U32, q.w, *q.w.shape), b.FromBF16Bits(q.s_bits, *q.s_bits.shape),
                b.FromBF16Bits(q.b_bits, *q.b_bits.shape))

    def normw(name, n):
        if torch is not None:
            t = (1.0 + 0.05 * torch.randn(n, device=dev)).to(torch.bfloat16)
            return b.Wrap(t.data_ptr(), (n,), BF16, keep=t)
        rng = np.random.default_rng(synth.stream_seed(seed, zlib.crc32(name.encode())))
        bits = synth.f32_to_bf16_bits((1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32))
        host[name] = synth.bf16_bits_to_f32(bits)
        return b.FromBF16Bits(bits, n)

    def cache():
        if torch is not None:
            t = torch.zeros((1, Hk, capacity, Dh), dtype=torch.bfloat16 if cache_dtype == BF16 else torch.float16,
                            device=dev)
            return b.Wrap(t.data_ptr(), tuple(t.shape), cache_dtype, keep=t)
        return b.FromRaw(cache_dtype, np.zeros((1, Hk, capacity, Dh), np.uint16), 1, Hk, capacity, Dh)

    m = Qwen3Model(cfg, qlin("embed", cfg.vocab, H))
    for l in range(cfg.layers):
        m.layers.append(Qwen3Layer(
            qkv=qlin(f"l{l}.qkv", (Hq + 2 * Hk) * Dh, H), o=qlin(f"l{l}.o", H, Hq * Dh),
            gate_up=qlin(f"l{l}.gate_up", 2 * I, H), down=qlin(f"l{l}.down", H, I),
            in_norm=normw(f"l{l}.in_norm", H), post_norm=normw(f"l{l}.post_norm", H),
            q_norm=normw(f"l{l}.q_norm", Dh), k_norm=normw(f"l{l}.k_norm", Dh),
            k_cache=cache(), v_cache=cache()))
    m.norm = normw("norm", H)
    m.lm_head = qlin("lm_head", cfg.vocab, H)
    return m, host
