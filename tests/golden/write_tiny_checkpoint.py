"""Writes a small random Qwen3 checkpoint in the MLX on-disk format
(config.json + model.safetensors: U32 packed 4-bit weights, BF16 scales,
biases and norm weights, names as mlx-community publishes them), for the
loader tests. The tensors come from janis_amd.synth, so tests can rebuild
them on the host; nothing here is the reference's."""
from __future__ import annotations

import json
import os
import struct
import zlib

import numpy as np

from janis_amd import synth


def write_safetensors(path: str, tensors: dict) -> None:
    """tensors: name -> (dtype string, shape, numpy array of the raw elements)."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode("utf-8")
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)


def tiny_qwen3(model_dir: str, hidden=512, inter=1024, heads=4, kv=2, head_dim=128, vocab=1000, layers=2,
               gs=64, seed=11, tie=False) -> dict:
    """Writes the checkpoint; returns the host tensors (synth.QuantLinear per
    linear, float32 norm weights) keyed by their checkpoint prefix."""
    os.makedirs(model_dir, exist_ok=True)
    host, st = {}, {}

    def qlin(name, n, k):
        q = synth.quant_linear(synth.stream_seed(seed, zlib.crc32(name.encode())), n, k, gs)
        host[name] = q
        st[name + ".weight"] = ("U32", q.w.shape, q.w)
        st[name + ".scales"] = ("BF16", q.s_bits.shape, q.s_bits)
        st[name + ".biases"] = ("BF16", q.b_bits.shape, q.b_bits)

    def normw(name, n):
        rng = np.random.default_rng(synth.stream_seed(seed, zlib.crc32(name.encode())))
        bits = synth.f32_to_bf16_bits((1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32))
        host[name] = synth.bf16_bits_to_f32(bits)
        st[name + ".weight"] = ("BF16", (n,), bits)

    qlin("model.embed_tokens", vocab, hidden)
    for i in range(layers):
        p = f"model.layers.{i}"
        qlin(f"{p}.self_attn.q_proj", heads * head_dim, hidden)
        qlin(f"{p}.self_attn.k_proj", kv * head_dim, hidden)
        qlin(f"{p}.self_attn.v_proj", kv * head_dim, hidden)
        qlin(f"{p}.self_attn.o_proj", hidden, heads * head_dim)
        qlin(f"{p}.mlp.gate_proj", inter, hidden)
        qlin(f"{p}.mlp.up_proj", inter, hidden)
        qlin(f"{p}.mlp.down_proj", hidden, inter)
        normw(f"{p}.input_layernorm", hidden)
        normw(f"{p}.post_attention_layernorm", hidden)
        normw(f"{p}.self_attn.q_norm", head_dim)
        normw(f"{p}.self_attn.k_norm", head_dim)
    normw("model.norm", hidden)
    if not tie:
        qlin("lm_head", vocab, hidden)
    write_safetensors(os.path.join(model_dir, "model.safetensors"), st)
    cfg = {"model_type": "qwen3", "hidden_size": hidden, "intermediate_size": inter,
           "num_attention_heads": heads, "num_key_value_heads": kv, "head_dim": head_dim, "vocab_size": vocab,
           "num_hidden_layers": layers, "rms_norm_eps": 1e-6, "rope_theta": 1000000.0,
           "tie_word_embeddings": tie, "quantization": {"group_size": gs, "bits": 4}}
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(cfg, f)
    return host
