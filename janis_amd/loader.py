"""Loading an MLX-format Qwen3 checkpoint (config.json + *.safetensors, 4-bit
affine-quantized as mlx-community publishes them) onto the HIP backend, the way
the reference's loaders do (qwen/config.go LoadConfig, qwen/model.go:240-268
LoadModel, qwen/linear.go:20-40 LoadQuantLinear): every tensor goes to the
device in its on-disk layout through FromRaw -- no repack. Two layout choices
of this backend's decode step are made here, both row concatenations of the
same MLX layout: q/k/v and gate/up become one matrix each (their rows are
independent, so one product gives the same numbers as two or three).

The safetensors reader is a small one of its own: the format is an 8-byte
little-endian header length, a JSON header of {name: {dtype, shape,
data_offsets}}, then the raw bytes; files are memory-mapped, nothing in them is
executed.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from .engine import BF16, F16, F32, I32, U32, U8, HipBackend, JanisHipError
from .qwen3_decode import Qwen3Config, Qwen3Layer, Qwen3Model

_ST_DTYPES = {"F32": (F32, 4), "F16": (F16, 2), "BF16": (BF16, 2), "I32": (I32, 4), "U32": (U32, 4),
              "U8": (U8, 1)}


class SafeTensors:
    """One .safetensors file, memory-mapped: names -> (dtype, shape, raw bytes)."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            if n > 100 << 20:
                raise ValueError(f"{path}: implausible safetensors header of {n} bytes")
            header = json.loads(f.read(n).decode("utf-8"))
        self.meta = {k: v for k, v in header.items() if k != "__metadata__"}
        self._base = 8 + n
        self._mm = np.memmap(path, dtype=np.uint8, mode="r")

    def names(self):
        return list(self.meta)

    def raw(self, name: str):
        """(dtype string, shape, uint8 view of the bytes)."""
        m = self.meta[name]
        a, b = m["data_offsets"]
        shape = tuple(int(d) for d in m["shape"])
        size = _ST_DTYPES[m["dtype"]][1] * (int(np.prod(shape, dtype=np.int64)) if shape else 1)
        if b - a != size:
            raise ValueError(f"{self.path}: {name} holds {b - a} bytes for {m['dtype']} {list(shape)}")
        return m["dtype"], shape, self._mm[self._base + a:self._base + b]


class Checkpoint:
    """The tensors of a model directory: one model.safetensors, or the shards a
    model.safetensors.index.json maps."""

    def __init__(self, model_dir: str):
        idx = os.path.join(model_dir, "model.safetensors.index.json")
        self.files = {}
        self.where = {}
        if os.path.exists(idx):
            with open(idx) as f:
                wm = json.load(f)["weight_map"]
            for name, fn in wm.items():
                if fn not in self.files:
                    self.files[fn] = SafeTensors(os.path.join(model_dir, fn))
                self.where[name] = self.files[fn]
        else:
            names = sorted(x for x in os.listdir(model_dir) if x.endswith(".safetensors"))
            if not names:
                raise FileNotFoundError(f"{model_dir}: no .safetensors files")
            for fn in names:
                st = SafeTensors(os.path.join(model_dir, fn))
                self.files[fn] = st
                for name in st.names():
                    self.where[name] = st

    def has(self, name: str) -> bool:
        return name in self.where

    def upload(self, b: HipBackend, name: str):
        """FromRaw of the tensor's bytes (engine/backend.go:152-154)."""
        if name not in self.where:
            raise KeyError(f"checkpoint has no tensor {name}")
        dt, shape, raw = self.where[name].raw(name)
        return b.FromRaw(_ST_DTYPES[dt][0], np.ascontiguousarray(raw), *shape)


def load_config(model_dir: str) -> Qwen3Config:
    """The config.json fields a Qwen3 dense model needs (qwen/config.go), with
    the same defaults: head_dim = hidden / heads, kv heads = heads, tied
    embeddings unless stated, the global quantization group size and bits."""
    with open(os.path.join(model_dir, "config.json")) as f:
        r = json.load(f)
    if r.get("model_type") not in ("qwen3",):
        raise JanisHipError(2, f"{model_dir}: model_type {r.get('model_type')!r}; this loader reads dense qwen3")
    heads, hidden = int(r.get("num_attention_heads", 0)), int(r.get("hidden_size", 0))
    if heads == 0 or hidden == 0:
        raise JanisHipError(1, f"{model_dir}: config has no attention heads / hidden size")
    q = r.get("quantization") or r.get("quantization_config") or {}
    cfg = Qwen3Config(hidden=hidden, inter=int(r["intermediate_size"]), n_heads=heads,
                      n_kv=int(r.get("num_key_value_heads") or heads),
                      head_dim=int(r.get("head_dim") or hidden // heads), vocab=int(r["vocab_size"]),
                      layers=int(r["num_hidden_layers"]), eps=float(r.get("rms_norm_eps", 1e-6)),
                      theta=float(r.get("rope_theta", 1e6)), group_size=int(q.get("group_size", 64)),
                      bits=int(q.get("bits", 4)), tie=r.get("tie_word_embeddings", True) is not False)
    return cfg


def load_qwen3(b: HipBackend, model_dir: str, capacity: int) -> Qwen3Model:
    """A Qwen3 dense checkpoint on the device, with bf16 KV caches of
    `capacity` tokens per layer."""
    cfg = load_config(model_dir)
    ck = Checkpoint(model_dir)
    Hk, Dh = cfg.n_kv, cfg.head_dim

    def lin(prefix):
        return tuple(ck.upload(b, f"{prefix}.{part}") for part in ("weight", "scales", "biases"))

    def stacked(prefixes):
        parts = [lin(p) for p in prefixes]
        out = []
        for j in range(3):
            t = parts[0][j]
            for p in parts[1:]:
                t = b.Concat(t, p[j], 0)
            out.append(t)
        return tuple(out)

    def cache():
        return b.empty(BF16, 1, Hk, capacity, Dh)

    m = Qwen3Model(cfg, lin("model.embed_tokens"))
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        m.layers.append(Qwen3Layer(
            qkv=stacked([f"{p}.self_attn.{x}_proj" for x in ("q", "k", "v")]),
            o=lin(f"{p}.self_attn.o_proj"),
            gate_up=stacked([f"{p}.mlp.gate_proj", f"{p}.mlp.up_proj"]),
            down=lin(f"{p}.mlp.down_proj"),
            in_norm=ck.upload(b, f"{p}.input_layernorm.weight"),
            post_norm=ck.upload(b, f"{p}.post_attention_layernorm.weight"),
            q_norm=ck.upload(b, f"{p}.self_attn.q_norm.weight"),
            k_norm=ck.upload(b, f"{p}.self_attn.k_norm.weight"),
            k_cache=cache(), v_cache=cache()))
    m.norm = ck.upload(b, "model.norm.weight")
    m.lm_head = None if cfg.tie and not ck.has("lm_head.weight") else lin("lm_head")
    b.Sync()
    return m
