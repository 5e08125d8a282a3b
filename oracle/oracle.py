"""ctypes view of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, always as the checker or the CPU baseline, never as the product.
It restates janis's CPU quantized-linear arithmetic; see janis_oracle.h for the
reference file:line each function follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int

_lib = None


def build() -> None:
    """Compile liboracle.so from the C sources next to this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.or_dequantize.argtypes = [_u32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _int, _int]
        L.or_dequantize.restype = None
        for name in ("or_qchannel4_ref", "or_qchannel4_avx2_order", "or_qchannel4_avx2"):
            fn = getattr(L, name)
            fn.argtypes = [_u32p, _f32p, _f32p, _f32p, _int, _int]
            fn.restype = ctypes.c_float
        L.or_have_avx2_fma.argtypes = []
        L.or_have_avx2_fma.restype = _int
        L.or_qmv_blocked_go.argtypes = [_f32p, _u32p, _f32p, _f32p, _f32p, _i64, _i64, _int, _int]
        L.or_qmv_blocked_go.restype = None
        L.or_qmv_generic.argtypes = [_f32p, _u32p, _f32p, _f32p, _f32p, _i64, _i64, _int, _int]
        L.or_qmv_generic.restype = None
        L.or_qmm_wbuf.argtypes = [_f32p, _i64, _u32p, _f32p, _f32p, _f32p, _i64, _i64, _int, _int]
        L.or_qmm_wbuf.restype = None
        L.or_quant_matmul.argtypes = [_f32p, _i64, _u32p, _f32p, _f32p, _f32p, _i64, _i64, _int, _int, _int]
        L.or_quant_matmul.restype = None
        L.or_gather_quant_matmul.argtypes = [_f32p, _i64, _i64, _u32p, _f32p, _f32p, _i64, _i32p, _i64,
                                             _f32p, _i64, _i64, _int, _int, _int]
        L.or_gather_quant_matmul.restype = _int
        L.or_qmv_avx2_parallel.argtypes = [_f32p, _u32p, _f32p, _f32p, _f32p, _i64, _i64, _int, _int]
        L.or_qmv_avx2_parallel.restype = _int
        L.or_moe_apply.argtypes = [_f32p, _i64, _u32p, _f32p, _f32p, _u32p, _f32p, _f32p, _u32p, _f32p, _f32p,
                                   _i64, _i64, _i64, _i32p, _f32p, _i64, _f32p, _int, _int]
        L.or_moe_apply.restype = _int
        L.or_topk.argtypes = [_f32p, _int, _int, _i32p, _f32p]
        L.or_topk.restype = None
        L.or_softmax_row.argtypes = [_f32p, _f32p, _int]
        L.or_softmax_row.restype = None
        _f = ctypes.c_float
        L.or_rms_norm.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _f]
        L.or_rms_norm.restype = None
        L.or_rope.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _int, _int, _f, _f, _i64, ctypes.c_void_p]
        L.or_rope.restype = None
        L.or_sdpa.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _i64, _f, _int]
        L.or_sdpa.restype = None
        L.or_silu.argtypes = [_f32p, _f32p, _i64]
        L.or_silu.restype = None
        L.or_argmax.argtypes = [_f32p, _i64, _i64, _i32p]
        L.or_argmax.restype = None
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def dequantize(w, s, b, group_size: int, bits: int = 4) -> np.ndarray:
    """cpu/cpu_misc.go:134-161. w [..., P] -> [..., P*32/bits] float32."""
    w, s, b = _u32(w), _f32(s), _f32(b)
    P = w.shape[-1]
    rows = w.size // P
    out = np.empty(w.shape[:-1] + (P * (32 // bits),), dtype=np.float32)
    lib().or_dequantize(w, s, b, out, rows, P, s.shape[-1], group_size, bits)
    return out


def qchannel4(kind: str, w, x, s, b, groups: int, wpg: int) -> float:
    fn = {"ref": lib().or_qchannel4_ref, "avx2_order": lib().or_qchannel4_avx2_order,
          "avx2": lib().or_qchannel4_avx2}[kind]
    return float(fn(_u32(w), _f32(x), _f32(s), _f32(b), groups, wpg))


def have_avx2_fma() -> bool:
    return bool(lib().or_have_avx2_fma())


def quant_matmul(x, w, s, b, group_size: int, bits: int = 4, simd: bool = True) -> np.ndarray:
    """cpu/cpu_misc.go:232-400 (transpose=true). x [..., K] -> [..., N]."""
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    N, P = w.shape[-2], w.shape[-1]
    K = P * (32 // bits)
    assert x.shape[-1] == K, (x.shape, K)
    rows = x.size // K
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    lib().or_quant_matmul(x, rows, w, s, b, y, N, K, group_size, bits, int(simd))
    return y


def qmv_blocked_go(x, w, s, b, group_size: int, workers: int = 1) -> np.ndarray:
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    N, K = w.shape[-2], w.shape[-1] * 8
    y = np.empty((N,), dtype=np.float32)
    lib().or_qmv_blocked_go(x, w, s, b, y, N, K, group_size, workers)
    return y


def qmv_generic(x, w, s, b, group_size: int, bits: int) -> np.ndarray:
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    N, K = w.shape[-2], w.shape[-1] * (32 // bits)
    y = np.empty((N,), dtype=np.float32)
    lib().or_qmv_generic(x, w, s, b, y, N, K, group_size, bits)
    return y


def qmm_wbuf(x, w, s, b, group_size: int, bits: int = 4) -> np.ndarray:
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    N, K = w.shape[-2], w.shape[-1] * (32 // bits)
    rows = x.size // K
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    lib().or_qmm_wbuf(x, rows, w, s, b, y, N, K, group_size, bits)
    return y


def gather_quant_matmul(x, w, s, b, idx, group_size: int, bits: int = 4, simd: bool = True) -> np.ndarray:
    """cpu/cpu_misc.go:178-230. x [n_lead, A, 1, K] (or [n_lead, A, K]),
    w [E, N, P], idx [n_lead, k] -> y [n_lead, k, 1, N]."""
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    E, N, P = w.shape
    K = P * (32 // bits)
    n_lead = int(np.prod(idx.shape[:-1], dtype=np.int64))
    k_slots = idx.shape[-1]
    A = x.size // (n_lead * K)
    y = np.zeros(idx.shape + (1, N), dtype=np.float32)
    rc = lib().or_gather_quant_matmul(x, n_lead, A, w, s, b, E, idx, k_slots, y, N, K,
                                      group_size, bits, int(simd))
    if rc != 0:
        raise IndexError("expert index out of range")
    return y


def moe_apply(x, gate, up, down, idx, scores, group_size: int = 64, simd: bool = True) -> np.ndarray:
    """qwen/moe.go:501-511 over resident stacks. gate/up/down are (w, s, b)
    triples of float32 scales/biases; x [n_tok, H]; idx, scores [n_tok, K]."""
    x = _f32(x)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    scores = _f32(scores)
    n_tok, k = idx.shape
    (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = gate, up, down
    E, I, _ = wg.shape
    H = x.shape[-1]
    out = np.zeros((n_tok, H), dtype=np.float32)
    rc = lib().or_moe_apply(x, n_tok, _u32(wg), _f32(sg), _f32(bg), _u32(wu), _f32(su), _f32(bu),
                            _u32(wd), _f32(sd), _f32(bd), E, H, I, idx, scores, k, out, group_size, int(simd))
    if rc != 0:
        raise IndexError("expert index out of range")
    return out


def qmv_avx2_parallel(x, w, s, b, group_size: int, workers: int) -> tuple[np.ndarray, int]:
    x, w, s, b = _f32(x), _u32(w), _f32(s), _f32(b)
    N, K = w.shape[-2], w.shape[-1] * 8
    y = np.empty((N,), dtype=np.float32)
    used = lib().or_qmv_avx2_parallel(x, w, s, b, y, N, K, group_size, workers)
    return y, used


def topk(row, k: int) -> tuple[np.ndarray, np.ndarray]:
    row = _f32(row)
    idx = np.empty(k, dtype=np.int32)
    val = np.empty(k, dtype=np.float32)
    lib().or_topk(row, row.size, k, idx, val)
    return idx, val


def softmax_row(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_softmax_row(x, out, x.size)
    return out


# -- decode-step operators ------------------------------------------------------------

def rms_norm(x, w, eps: float) -> np.ndarray:
    """cpu/cpu_ops.go:144-162 over the last axis."""
    x, w = _f32(x), _f32(w)
    d = x.shape[-1]
    out = np.empty_like(x)
    lib().or_rms_norm(x, w, out, x.size // d, d, ctypes.c_float(eps))
    return out


def rope(x, dims: int, traditional: bool, base: float, scale: float, offset: int, freqs=None) -> np.ndarray:
    """cpu/cpu_attn.go:13-62; x [..., L, D]."""
    x = _f32(x)
    D, L = x.shape[-1], x.shape[-2]
    out = np.empty_like(x)
    fr = None if freqs is None else _f32(freqs)
    lib().or_rope(x, out, x.size // D, L, D, dims, int(traditional), ctypes.c_float(base), ctypes.c_float(scale),
                  offset, None if fr is None else fr.ctypes.data_as(ctypes.c_void_p))
    return out


def sdpa(q, k, v, scale: float, causal: bool) -> np.ndarray:
    """cpu/cpu_attn.go:64-119; q [B, Hq, Lq, Dh], k/v [B, Hk, Lk, Dh]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Lq, Dh = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    lib().or_sdpa(q, k, v, out, B, Hq, Hk, Lq, Lk, Dh, ctypes.c_float(scale), int(causal))
    return out


def silu(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_silu(x, out, x.size)
    return out


def argmax(x) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    out = np.empty(x.shape[:-1], dtype=np.int32)
    lib().or_argmax(x, x.size // n, n, out)
    return out


def scatter_rows(dst, indices, updates) -> np.ndarray:
    """cpu/cpu_ops.go:215-233 (RowScatterer.ScatterRows): a copy of dst whose
    row indices[i] (axis 0) is replaced by updates[i], applied in index order
    (so a repeated index keeps its last update); any dtype, rows compared as
    bytes. Raises IndexError for an index outside [0, rows), where the
    reference's slice copy panics."""
    dst = np.asarray(dst)
    out = dst.copy()
    upd = np.asarray(updates).reshape((len(indices),) + dst.shape[1:])
    for i, r in enumerate(np.asarray(indices, dtype=np.int64).reshape(-1)):
        if r < 0 or r >= dst.shape[0]:
            raise IndexError(f"scatter_rows: index {r} outside [0, {dst.shape[0]})")
        out[r] = upd[i]
    return out


# -- engine operators around the products ---------------------------------------------

def matmul_dequant(x, w, s, b, group_size: int, bits: int = 4) -> np.ndarray:
    """QuantMatmul with transpose=false: MatMul(x, Dequantize(w))
    (cpu/cpu_misc.go:233-236). Dequantize is cpu/cpu_misc.go:154-156; the
    product follows cpu/cpu_ops.go:33-48 -- per output row, over k in
    increasing order, a zero x[i, k] skipped, the term x[i, k] * W[k, :]
    rounded to fp32 and then added in fp32. x [..., N] with N the rows of w;
    returns [..., K]."""
    wd = dequantize(w, s, b, group_size, bits)  # [N, K]
    x = _f32(x)
    N, K = wd.shape
    assert x.shape[-1] == N, (x.shape, wd.shape)
    xr = x.reshape(-1, N)
    out = np.zeros((xr.shape[0], K), dtype=np.float32)
    for i in range(xr.shape[0]):
        o = out[i]
        for k in range(N):
            a = xr[i, k]
            if a == 0:
                continue
            o += (np.float32(a) * wd[k]).astype(np.float32)  # float32 * float32 -> rounded, then added
    return out.reshape(x.shape[:-1] + (K,))


def gather_matmul_dequant(x, w, s, b, idx, group_size: int, bits: int = 4) -> np.ndarray:
    """GatherQuantMatmul with transpose=false (cpu/cpu_misc.go:178-230 with
    :233-236): slot (l, k) is MatMul(x[l, a], Dequantize(W[idx[l, k]])) with a
    = 0 when x has one vector per lead (A = 1), else k. x [n_lead, A, N];
    returns [n_lead, K, Kin]. Raises IndexError for an index outside the stack."""
    x = _f32(x)
    idx = np.asarray(idx, dtype=np.int64)
    n_lead, kk = idx.shape
    A = x.shape[1]
    E = w.shape[0]
    kin = w.shape[-1] * (32 // bits)
    out = np.empty((n_lead, kk, kin), dtype=np.float32)
    for l in range(n_lead):
        for k in range(kk):
            e = int(idx[l, k])
            if e < 0 or e >= E:
                raise IndexError(f"expert index {e} outside [0, {E})")
            out[l, k] = matmul_dequant(x[l, 0 if A == 1 else k][None], w[e], s[e], b[e], group_size, bits)[0]
    return out


def softmax(x, axis: int) -> np.ndarray:
    """Backend.Softmax (cpu/cpu.go:461-499) along any axis: each line through
    softmax_row (max, fp32(exp(double(x - max))), the sequential fp32 sum, then
    the fp32 division)."""
    x = _f32(x)
    xm = np.moveaxis(x, axis, -1)
    flat = np.ascontiguousarray(xm.reshape(-1, xm.shape[-1]))
    out = np.stack([softmax_row(r) for r in flat]) if flat.shape[0] else flat.copy()
    return np.ascontiguousarray(np.moveaxis(out.reshape(xm.shape), -1, axis))


def mean(x, axis: int) -> np.ndarray:
    """Backend.Mean (cpu/cpu_ops.go:113-142): per output the fp32 sum along
    the axis in increasing index order, then divided by the axis length in
    fp32. (numpy's own reductions sum pairwise; this loop keeps the order.)"""
    x = _f32(x)
    xm = np.moveaxis(x, axis, -1)
    n = xm.shape[-1]
    s = np.zeros(xm.shape[:-1], dtype=np.float32)
    for i in range(n):
        s = (s + xm[..., i]).astype(np.float32)
    return (s / np.float32(n)).astype(np.float32)


def scalar_mul(x, v: float) -> np.ndarray:
    """Backend.ScalarMul (cpu/cpu_misc.go:24-26): x * v in fp32."""
    return (_f32(x) * np.float32(v)).astype(np.float32)


def scalar_add(x, v: float) -> np.ndarray:
    """Backend.ScalarAdd (cpu/cpu_misc.go:28-30): x + v in fp32."""
    return (_f32(x) + np.float32(v)).astype(np.float32)
