"""Seeded synthetic inputs for the MLX affine-quantized matrix products.

One counter-based generator (splitmix64) feeds every tensor, so a test and the
CPU oracle it checks against see the same bytes, and any element can be
regenerated on its own from (seed, stream, index).

Distributions follow the benchmark configurations of this backend:
  codes   uniform 0..15, packed 8 per little-endian uint32, lowest nibble first
          (the MLX layout, cpu/cpu_misc.go:124-130 in the reference)
  scale   bf16(|N(0,1)| * 0.02)                      per group of `group_size`
  bias    bf16(-8 * scale + N(0,1) * 1e-3)           from the bf16-rounded scale
  x       bf16(N(0,1))

Normals come from Box-Muller on two 53-bit uniforms; bf16 values are rounded
from float32 to nearest-even. bf16 tensors are carried as their uint16 bit
patterns (numpy has no bfloat16) together with an exact float32 widening.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset+1 .. offset+n of the splitmix64 sequence started at seed."""
    out = np.empty(n, dtype=np.uint64)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        for lo in range(0, n, _CHUNK):
            hi = min(n, lo + _CHUNK)
            i = np.arange(offset + lo + 1, offset + hi + 1, dtype=np.uint64)
            out[lo:hi] = _mix(s + i * _GAMMA)
    return out


def stream_seed(seed: int, stream: int) -> int:
    """Seed of an independent sub-stream (one per tensor)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + np.uint64(stream + 1) * _GAMMA
        return int(_mix(np.array([z], dtype=np.uint64))[0] ^ np.uint64(0xA5A5A5A5A5A5A5A5))


def uniform_u32(seed: int, n: int) -> np.ndarray:
    return (splitmix64(seed, n) >> np.uint64(32)).astype(np.uint32)


def normal(seed: int, n: int) -> np.ndarray:
    """n standard normals (float64) by Box-Muller, consuming two outputs each."""
    r = splitmix64(seed, 2 * n)
    u1 = ((r[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (r[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest-even); returns the uint16 patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """Exact widening, as the reference's FromRaw does (cpu/cpu.go:186-190)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


class QuantLinear:
    """A 4-bit affine-quantized weight triplet in MLX layout plus its fp32 view.

    w       uint32 [N, K/8]
    s_bits  uint16 [N, K/group_size]   bf16 scales
    b_bits  uint16 [N, K/group_size]   bf16 biases
    """

    def __init__(self, w: np.ndarray, s_bits: np.ndarray, b_bits: np.ndarray, group_size: int, bits: int = 4):
        self.w = np.ascontiguousarray(w, dtype=np.uint32)
        self.s_bits = np.ascontiguousarray(s_bits, dtype=np.uint16)
        self.b_bits = np.ascontiguousarray(b_bits, dtype=np.uint16)
        self.group_size = group_size
        self.bits = bits

    @property
    def out_features(self) -> int:
        return self.w.shape[-2]

    @property
    def in_features(self) -> int:
        return self.w.shape[-1] * (32 // self.bits)

    @property
    def s(self) -> np.ndarray:
        return bf16_bits_to_f32(self.s_bits)

    @property
    def b(self) -> np.ndarray:
        return bf16_bits_to_f32(self.b_bits)


def quant_linear(seed: int, n: int, k: int, group_size: int = 64, lead: tuple = (), bits: int = 4) -> QuantLinear:
    """Random `bits`-wide weights [*lead, n, k] (uniform words: uniform codes of
    any width) with the scale/bias distributions above; the bias centres the
    codes, -2^(bits-1) * scale."""
    vpw = 32 // bits
    if bits not in (2, 4, 8) or k % group_size or group_size % vpw:
        raise ValueError("bits 2/4/8, in_features a multiple of group_size, group_size of 32/bits")
    rows = int(np.prod(lead, dtype=np.int64)) * n
    g = k // group_size
    w = uniform_u32(stream_seed(seed, 0), rows * (k // vpw)).reshape(*lead, n, k // vpw)
    s32 = (np.abs(normal(stream_seed(seed, 1), rows * g)) * 0.02).astype(np.float32)
    s_bits = f32_to_bf16_bits(s32)
    s = bf16_bits_to_f32(s_bits).astype(np.float64)
    b64 = -float(1 << (bits - 1)) * s + normal(stream_seed(seed, 2), rows * g) * 1e-3
    b_bits = f32_to_bf16_bits(b64.astype(np.float32))
    return QuantLinear(w, s_bits.reshape(*lead, n, g), b_bits.reshape(*lead, n, g), group_size, bits)


def activations(seed: int, shape: tuple) -> tuple[np.ndarray, np.ndarray]:
    """bf16(N(0,1)) of the given shape: (uint16 bits, exact float32 view)."""
    n = int(np.prod(shape, dtype=np.int64))
    bits = f32_to_bf16_bits(normal(stream_seed(seed, 3), n).astype(np.float32)).reshape(shape)
    return bits, bf16_bits_to_f32(bits)


def topk_rows(probs: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-row top-k by k passes of selection sort with strict '>' and a swap,
    the tie behaviour of the reference router (qwen/moe.go:420-444)."""
    probs = np.asarray(probs, dtype=np.float32)
    t, n = probs.shape
    order = np.tile(np.arange(n), (t, 1))
    rows = np.arange(t)
    for i in range(min(k, n)):
        vals = probs[rows[:, None], order[:, i:]]
        # first maximum over the remaining positions == the strict '>' scan
        best = i + np.argmax(vals, axis=1)
        a = order[rows, i].copy()
        order[rows, i] = order[rows, best]
        order[rows, best] = a
    idx = order[:, :k].astype(np.int32)
    return idx, probs[rows[:, None], idx]


def route(seed: int, n_tok: int, n_experts: int, k: int, norm_topk: bool = True):
    """Seeded router: logits N(0,1) -> softmax -> top-k -> renormalised scores.

    Returns (expert indices int32 [n_tok, k], scores float32 [n_tok, k])."""
    logits = normal(stream_seed(seed, 4), n_tok * n_experts).astype(np.float32).reshape(n_tok, n_experts)
    m = logits.max(axis=1, keepdims=True)
    e = np.exp((logits - m).astype(np.float64)).astype(np.float32)
    probs = (e / e.sum(axis=1, dtype=np.float32, keepdims=True)).astype(np.float32)
    idx, sc = topk_rows(probs, k)
    if norm_topk:
        sc = (sc / sc.sum(axis=1, dtype=np.float32, keepdims=True)).astype(np.float32)
    return idx, sc
