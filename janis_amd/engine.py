"""Host-side mirror of janis's engine.Backend for the quantized-linear path.

HipBackend offers the methods of engine.Backend (engine/backend.go:142-287)
that this backend implements -- FromRaw, FromFloats, FromInt32, Dequantize,
QuantMatmul, GatherQuantMatmul, Floats, Ints, Bytes/DTypeOf (RawReader),
Version, Close -- with the reference's names, argument meaning and result
shapes, each a thin call into the C ABI of libjanis_hip.so (include/janis_hip.h).
It is what a Go `hip` package would do over cgo, written in Python so the parity
tests read like the reference's own backend tests. Bad input raises
JanisHipError where the reference panics.

Tensors live in device memory owned by the backend (jh_alloc) and are freed
when the handle is collected, like the Go finalizers of the ggml backend
(ggml/ggml.go:451-465).
"""
from __future__ import annotations

import contextlib
import ctypes

import numpy as np

from . import _lib
from ._lib import BF16, F16, F32, I32, U32, U8, JanisHipError, check

DTYPE_SIZE = {F32: 4, F16: 2, BF16: 2, I32: 4, U32: 4, U8: 1}
DTYPE_NAME = {F32: "F32", F16: "F16", BF16: "BF16", I32: "I32", U32: "U32", U8: "U8"}


class Tensor:
    """Device tensor: shape, dtype, device pointer. engine.Tensor (engine/backend.go:24-26)."""

    def __init__(self, backend: "HipBackend", ptr: int, shape, dtype: int, owned: bool = True, keep=None):
        self._b = backend
        self.ptr = int(ptr) if ptr else 0
        self.shape = tuple(int(d) for d in shape)
        self.dtype = dtype
        self._owned = owned
        self._keep = keep  # an object whose lifetime covers the memory (non-owned views)

    def Shape(self) -> list:
        return list(self.shape)

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * DTYPE_SIZE[self.dtype]

    def __del__(self):
        try:
            if self._owned and self.ptr and self._b._ctx:
                _lib.load().jh_free(self._b._ctx, ctypes.c_void_p(self.ptr))
        except Exception:
            pass
        self.ptr = 0

    def __repr__(self):
        return f"Tensor({DTYPE_NAME[self.dtype]}, {list(self.shape)})"


class HipBackend:
    """engine.Backend subset on one MI355X (gfx950)."""

    def __init__(self, device: int = 0):
        L = _lib.load()
        ctx = ctypes.c_void_p()
        rc = L.jh_create(device, ctypes.byref(ctx))
        if rc != 0:
            raise JanisHipError(rc, (L.jh_last_error(None) or b"").decode())
        self._L = L
        self._ctx = ctx
        self._arena = None  # [base tensor, offset] while an arena is in use

    # -- lifecycle / info ------------------------------------------------------
    def Version(self) -> str:
        return self._L.jh_version().decode()

    def EngineInfo(self) -> str:
        buf = ctypes.create_string_buffer(256)
        cus = ctypes.c_int()
        check(self._ctx, self._L.jh_device_info(self._ctx, buf, 256, ctypes.byref(cus)))
        return f"HIP backend on {buf.value.decode()}"

    def Close(self) -> None:
        if self._ctx:
            self._L.jh_destroy(self._ctx)
            self._ctx = None

    def Sync(self) -> None:
        check(self._ctx, self._L.jh_sync(self._ctx))

    def SetStream(self, stream_handle: int | None) -> None:
        """Enqueue on a caller's hipStream_t (e.g. torch.cuda.current_stream().cuda_stream)."""
        check(self._ctx, self._L.jh_set_stream(self._ctx, ctypes.c_void_p(stream_handle or 0)))

    def SetChecks(self, on: bool) -> None:
        check(self._ctx, self._L.jh_set_checks(self._ctx, int(bool(on))))

    # -- creation ----------------------------------------------------------------
    def make_arena(self, nbytes: int) -> Tensor:
        """One device allocation that `use_arena` carves results from."""
        return self.empty(U8, int(nbytes))

    @contextlib.contextmanager
    def use_arena(self, arena: Tensor):
        """While active, every result tensor is carved from `arena` (256-byte
        aligned, from its start) instead of allocated: no jh_alloc/jh_free inside,
        so the operator sequence can be captured into a HIP graph, and two runs of
        the same sequence get the same addresses. Results stay valid while the
        arena lives and until the next use_arena on it."""
        prev = self._arena
        self._arena = [arena, 0]
        try:
            yield arena
        finally:
            self._arena = prev

    def empty(self, dtype: int, *shape) -> Tensor:
        n = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if self._arena is not None:
            base, off = self._arena
            need = max(1, n * DTYPE_SIZE[dtype])
            if off + need > base.nbytes:
                raise JanisHipError(_lib.JH_ERR_OOM, f"arena of {base.nbytes} bytes exhausted")
            self._arena[1] = (off + need + 255) & ~255
            return Tensor(self, base.ptr + off, shape, dtype, owned=False, keep=base)
        p = ctypes.c_void_p()
        check(self._ctx, self._L.jh_alloc(self._ctx, max(1, n * DTYPE_SIZE[dtype]), ctypes.byref(p)))
        return Tensor(self, p.value, shape, dtype)

    def FromRaw(self, dt: int, raw, *shape) -> Tensor:
        """Copies packed little-endian bytes of dtype dt (engine/backend.go:152-154)."""
        buf = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) \
            else np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        t = self.empty(dt, *shape)
        if buf.size != t.nbytes:
            raise JanisHipError(_lib.JH_ERR_INVALID,
                                f"FromRaw: {buf.size} bytes for shape {list(shape)} of {DTYPE_NAME[dt]}")
        check(self._ctx, self._L.jh_h2d(self._ctx, ctypes.c_void_p(t.ptr),
                                        buf.ctypes.data_as(ctypes.c_void_p), buf.size))
        return t

    def FromFloats(self, data, *shape) -> Tensor:
        a = np.ascontiguousarray(data, dtype=np.float32)
        return self.FromRaw(F32, a, *(shape or a.shape))

    def FromInt32(self, data, *shape) -> Tensor:
        a = np.ascontiguousarray(data, dtype=np.int32)
        return self.FromRaw(I32, a, *(shape or a.shape))

    def FromBF16Bits(self, bits, *shape) -> Tensor:
        a = np.ascontiguousarray(bits, dtype=np.uint16)
        return self.FromRaw(BF16, a, *(shape or a.shape))

    def Wrap(self, ptr: int, shape, dtype: int, keep=None) -> Tensor:
        """A non-owning handle over existing device memory (e.g. a torch tensor)."""
        return Tensor(self, ptr, shape, dtype, owned=False, keep=keep)

    # -- read back -------------------------------------------------------------------
    def Bytes(self, t: Tensor) -> bytes:
        out = np.empty(t.nbytes, dtype=np.uint8)
        check(self._ctx, self._L.jh_d2h(self._ctx, out.ctypes.data_as(ctypes.c_void_p),
                                        ctypes.c_void_p(t.ptr), t.nbytes))
        return out.tobytes()

    def DTypeOf(self, t: Tensor) -> int:
        return t.dtype

    def Floats(self, t: Tensor) -> np.ndarray:
        """engine/backend.go:276-277: evaluates and copies out as float32."""
        raw = np.frombuffer(self.Bytes(t), dtype=np.uint8)
        if t.dtype == F32:
            a = raw.view(np.float32)
        elif t.dtype == BF16:
            a = (raw.view(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
        elif t.dtype == F16:
            a = raw.view(np.float16).astype(np.float32)
        elif t.dtype in (I32,):
            a = raw.view(np.int32).astype(np.float32)
        else:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Floats: unsupported dtype {DTYPE_NAME[t.dtype]}")
        return a.reshape(t.shape).copy()

    def Ints(self, t: Tensor) -> np.ndarray:
        raw = np.frombuffer(self.Bytes(t), dtype=np.uint8)
        if t.dtype not in (I32, U32):
            raise JanisHipError(_lib.JH_ERR_INVALID, "Ints: tensor is not I32/U32")
        return raw.view(np.int32).reshape(t.shape).copy()

    # -- quantized operators ------------------------------------------------------------
    @staticmethod
    def _sb_dtype(scales: Tensor, biases: Tensor) -> int:
        if scales.dtype != biases.dtype:
            raise JanisHipError(_lib.JH_ERR_INVALID, "scales and biases differ in dtype")
        return scales.dtype

    def Dequantize(self, w: Tensor, scales: Tensor, biases: Tensor, groupSize: int, bits: int,
                   out_dtype: int = F32) -> Tensor:
        """engine/backend.go:261-263: w [..., P] U32 -> [..., P*32/bits] (cpu/cpu_misc.go:134-161)."""
        if w.dtype != U32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "Dequantize: weight tensor is not packed U32")
        P = w.shape[-1]
        k = P * (32 // bits)
        rows = w.numel // P
        out = self.empty(out_dtype, *w.shape[:-1], k)
        check(self._ctx, self._L.jh_dequantize(self._ctx, w.ptr, scales.ptr, biases.ptr,
                                               self._sb_dtype(scales, biases), rows, k, groupSize,
                                               bits, out.ptr, out_dtype))
        return out

    def QuantMatmul(self, x: Tensor, w: Tensor, scales: Tensor, biases: Tensor, transpose: bool,
                    groupSize: int, bits: int, out: Tensor | None = None, out_dtype: int | None = None) -> Tensor:
        """engine/backend.go:265-267: x [..., in] -> [..., out] with W [out, P]
        (transpose=true, cpu/cpu_misc.go:232-400). The result has x's dtype
        unless out_dtype says otherwise; `out` may supply the result buffer."""
        if w.dtype != U32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatmul: weight tensor is not packed U32")
        n, P = w.shape[-2], w.shape[-1]
        k = P * (32 // bits)
        if x.shape[-1] != k:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"QuantMatmul: x has {x.shape[-1]} features, W has {k}")
        rows = x.numel // k
        yd = out_dtype if out_dtype is not None else (out.dtype if out is not None else x.dtype)
        y = out if out is not None else self.empty(yd, *x.shape[:-1], n)
        check(self._ctx, self._L.jh_quant_matmul(self._ctx, x.ptr, x.dtype, rows, w.ptr, scales.ptr,
                                                 biases.ptr, self._sb_dtype(scales, biases), n, k,
                                                 int(bool(transpose)), groupSize, bits, y.ptr, y.dtype))
        return y

    def GatherQuantMatmul(self, x: Tensor, w: Tensor, scales: Tensor, biases: Tensor, rhsIndices: Tensor,
                          transpose: bool, groupSize: int, bits: int, out: Tensor | None = None,
                          out_dtype: int | None = None) -> Tensor:
        """engine/backend.go:269-274: x [lead.., A, 1, in], stacks [E, out, .],
        rhsIndices [lead.., K] -> [lead.., K, 1, out] (cpu/cpu_misc.go:178-230)."""
        if w.dtype != U32 or len(w.shape) != 3:
            raise JanisHipError(_lib.JH_ERR_INVALID, "GatherQuantMatmul: w must be U32 [E, out, P]")
        if rhsIndices.dtype != I32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "GatherQuantMatmul: indices must be I32")
        E, n, P = w.shape
        k = P * (32 // bits)
        rs = rhsIndices.shape
        K = rs[-1]
        n_lead = int(np.prod(rs[:-1], dtype=np.int64)) if len(rs) > 1 else 1
        if x.shape[-1] != k or len(x.shape) < 3:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"GatherQuantMatmul: x {list(x.shape)} vs in={k}")
        A = x.shape[-3]
        if x.numel != n_lead * A * k:
            raise JanisHipError(_lib.JH_ERR_INVALID, "GatherQuantMatmul: x lead dims do not match indices")
        yd = out_dtype if out_dtype is not None else (out.dtype if out is not None else x.dtype)
        y = out if out is not None else self.empty(yd, *rs, 1, n)
        check(self._ctx, self._L.jh_gather_quant_matmul(
            self._ctx, x.ptr, x.dtype, n_lead, A, w.ptr, scales.ptr, biases.ptr,
            self._sb_dtype(scales, biases), E, n, k, rhsIndices.ptr, K, int(bool(transpose)),
            groupSize, bits, y.ptr, y.dtype))
        return y

    # -- the other operators of a decode step ----------------------------------------
    def Reshape(self, x: Tensor, *shape) -> Tensor:
        """engine.Backend.Reshape: a view over the same memory (one -1 allowed)."""
        shape = list(shape)
        if shape.count(-1) == 1:
            known = int(np.prod([d for d in shape if d != -1], dtype=np.int64))
            shape[shape.index(-1)] = x.numel // known if known else 0
        if int(np.prod(shape, dtype=np.int64)) != x.numel:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Reshape: {list(x.shape)} -> {shape}")
        return Tensor(self, x.ptr, shape, x.dtype, owned=False, keep=x)

    def Transpose(self, x: Tensor, *perm) -> Tensor:
        """engine.Backend.Transpose where it moves only length-1 axes (a view);
        other permutations are not implemented here."""
        kept = [a for a in perm if x.shape[a] != 1]
        if kept != sorted(kept):
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "Transpose: only layout-preserving permutations")
        return Tensor(self, x.ptr, [x.shape[a] for a in perm], x.dtype, owned=False, keep=x)

    def RMSNorm(self, x: Tensor, weight: Tensor, eps: float, out_dtype: int | None = None) -> Tensor:
        """cpu/cpu_ops.go:144-162 over the last axis."""
        d = x.shape[-1]
        out = self.empty(out_dtype if out_dtype is not None else x.dtype, *x.shape)
        check(self._ctx, self._L.jh_rms_norm(self._ctx, x.ptr, x.dtype, x.numel // d, d, weight.ptr, weight.dtype,
                                             float(eps), out.ptr, out.dtype))
        return out

    def _rope(self, x, dims, traditional, base, scale, offset, freqs, out_dtype):
        D, L = x.shape[-1], x.shape[-2]
        out = self.empty(out_dtype if out_dtype is not None else x.dtype, *x.shape)
        check(self._ctx, self._L.jh_rope(self._ctx, x.ptr, x.dtype, x.numel // D, L, D, dims, int(bool(traditional)),
                                         float(base), float(scale), int(offset), freqs.ptr if freqs else None,
                                         out.ptr, out.dtype))
        return out

    def RoPE(self, x: Tensor, dims: int, traditional: bool, base: float, scale: float, offset: int,
             out_dtype: int | None = None) -> Tensor:
        """cpu/cpu_attn.go:13-20; x [..., L, D]."""
        return self._rope(x, dims, traditional, base, scale, offset, None, out_dtype)

    def RoPEFreqs(self, x: Tensor, dims: int, traditional: bool, scale: float, offset: int, freqs: Tensor,
                  out_dtype: int | None = None) -> Tensor:
        """cpu/cpu_attn.go:22-34 (freqs fp32 [dims/2])."""
        if freqs.dtype != F32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "RoPEFreqs: freqs must be F32")
        return self._rope(x, dims, traditional, 1.0, scale, offset, freqs, out_dtype)

    def SDPA(self, q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool, kv_len: int | None = None,
             out_dtype: int | None = None) -> Tensor:
        """cpu/cpu_attn.go:64-119: q [B, Hq, Lq, Dh]; k/v [B, Hk, cap, Dh] whose first
        kv_len rows are valid (all of them when kv_len is None)."""
        B, Hq, Lq, Dh = q.shape
        Hk, cap = k.shape[1], k.shape[2]
        if k.shape != v.shape or k.dtype != v.dtype or k.shape[0] != B or k.shape[3] != Dh:
            raise JanisHipError(_lib.JH_ERR_INVALID, "SDPA: k/v shapes do not match q")
        Lk = cap if kv_len is None else kv_len
        out = self.empty(out_dtype if out_dtype is not None else q.dtype, B, Hq, Lq, Dh)
        check(self._ctx, self._L.jh_sdpa(self._ctx, q.ptr, q.dtype, k.ptr, v.ptr, k.dtype, B, Hq, Hk, Lq, Lk, cap,
                                         Dh, float(scale), int(bool(causal)), out.ptr, out.dtype))
        return out

    def _elementwise(self, op, a, b, out_dtype):
        if b is not None and b.numel != a.numel:
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "elementwise: operands must have the same size")
        out = self.empty(out_dtype if out_dtype is not None else a.dtype, *a.shape)
        check(self._ctx, self._L.jh_elementwise(self._ctx, op, a.ptr, a.dtype, b.ptr if b is not None else None,
                                                b.dtype if b is not None else a.dtype, a.numel, out.ptr, out.dtype))
        return out

    def Add(self, a: Tensor, b: Tensor, out_dtype: int | None = None) -> Tensor:
        return self._elementwise(_lib.JH_OP_ADD, a, b, out_dtype)

    def Mul(self, a: Tensor, b: Tensor, out_dtype: int | None = None) -> Tensor:
        return self._elementwise(_lib.JH_OP_MUL, a, b, out_dtype)

    def SiLU(self, x: Tensor, out_dtype: int | None = None) -> Tensor:
        return self._elementwise(_lib.JH_OP_SILU, x, None, out_dtype)

    def SiLUMul(self, gate: Tensor, up: Tensor, out_dtype: int | None = None) -> Tensor:
        """Mul(SiLU(gate), up) in one pass (qwen/mlp.go:33-35)."""
        return self._elementwise(_lib.JH_OP_SILU_MUL, gate, up, out_dtype)

    def Argmax(self, x: Tensor, axis: int = -1) -> Tensor:
        """cpu/cpu_misc.go:91-121, last axis only."""
        if axis not in (-1, len(x.shape) - 1):
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "Argmax: last axis only")
        n = x.shape[-1]
        out = self.empty(I32, *x.shape[:-1])
        check(self._ctx, self._L.jh_argmax(self._ctx, x.ptr, x.dtype, x.numel // n, n, out.ptr))
        return out

    def TakeAxis(self, a: Tensor, indices: Tensor, axis: int = 0) -> Tensor:
        """cpu/cpu_misc.go:48-89 on axis 0 (rows of any dtype, packed words included)."""
        if axis != 0 or indices.dtype != I32:
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "TakeAxis: axis 0 with I32 indices only")
        rows = a.shape[0]
        row_bytes = a.nbytes // rows if rows else 0
        out = self.empty(a.dtype, *indices.shape, *a.shape[1:])
        check(self._ctx, self._L.jh_take_rows(self._ctx, a.ptr, row_bytes, rows, indices.ptr, indices.numel, out.ptr))
        return out

    def AppendKV(self, k_cache: Tensor, v_cache: Tensor, pos: int, k_new: Tensor, v_new: Tensor) -> None:
        """KV-cache append: caches [B, Hk, cap, Dh], new rows [B, Hk, L, Dh] at pos."""
        B, Hk, cap, Dh = k_cache.shape
        L = k_new.shape[-2]
        if k_new.shape != v_new.shape or k_new.dtype != v_new.dtype or k_new.numel != B * Hk * L * Dh:
            raise JanisHipError(_lib.JH_ERR_INVALID, "AppendKV: new rows do not match the cache")
        check(self._ctx, self._L.jh_kv_append(self._ctx, k_cache.ptr, v_cache.ptr, k_cache.dtype, B * Hk, cap,
                                              int(pos), k_new.ptr, v_new.ptr, k_new.dtype, L, Dh))

    def QKNormRoPEAppend(self, qkv: Tensor, n_heads: int, n_kv_heads: int, q_norm: Tensor, k_norm: Tensor,
                         eps: float, base: float, scale: float, pos: int, k_cache: Tensor, v_cache: Tensor,
                         out_dtype: int | None = None) -> Tensor:
        """qwen/attention.go:101-122 for one token: per-head q/k RMSNorm, RoPE and
        the KV append in one launch. qkv [.., (Hq+2Hk)*128]; caches [1, Hk, cap, 128].
        Returns q [1, Hq, 1, 128]."""
        if q_norm.dtype != k_norm.dtype:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QKNormRoPEAppend: norm weights differ in dtype")
        Dh = 128
        cap = k_cache.shape[-2]
        q = self.empty(out_dtype if out_dtype is not None else qkv.dtype, 1, n_heads, 1, Dh)
        check(self._ctx, self._L.jh_qk_norm_rope_append(
            self._ctx, qkv.ptr, qkv.dtype, n_heads, n_kv_heads, Dh, q_norm.ptr, k_norm.ptr, q_norm.dtype,
            float(eps), float(base), float(scale), int(pos), k_cache.ptr, v_cache.ptr, k_cache.dtype, cap,
            q.ptr, q.dtype))
        return q

    def QuantMatvecFused(self, x: Tensor, w: Tensor, scales: Tensor, biases: Tensor, groupSize: int, bits: int,
                         prologue: int = _lib.JH_PRO_NONE, norm: Tensor | None = None, eps: float = 0.0,
                         epilogue: int | None = None, resid: Tensor | None = None, out: Tensor | None = None,
                         out_dtype: int | None = None, stats: Tensor | None = None,
                         norm_out: Tensor | None = None) -> Tensor:
        """One-token QuantMatmul (transpose=true) with the operator before it
        fused in (JH_PRO_RMSNORM: RMSNorm(x, norm, eps), the norm feeding q/k/v,
        gate/up and the LM head; JH_PRO_SILU_MUL: x = [gate | up] -> SiLU(gate)*up)
        and the one after it (JH_EPI_RESID, the default when resid is given: the
        residual Add of qwen/block.go:59-60 into an fp32 result, out may be resid;
        JH_EPI_SWIGLU: w stacks the Gate rows then the Up rows and the result is
        SiLU(gate)*up, qwen/mlp.go:33-35). The split norm: JH_EPI_RESID_NORM
        also writes norm_out = bf16(y * norm) (norm = the NEXT norm's weight)
        and its statistics into `stats`; the product that consumes them takes
        JH_PRO_NORMED with x = that norm_out and the same `stats`."""
        if w.dtype != U32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatvecFused: weight tensor is not packed U32")
        if epilogue is None:
            epilogue = _lib.JH_EPI_RESID if resid is not None else _lib.JH_EPI_STORE
        rows, P = w.shape[-2], w.shape[-1]
        if epilogue == _lib.JH_EPI_SWIGLU and rows % 2:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatvecFused: SwiGLU needs gate and up rows")
        n = rows // 2 if epilogue == _lib.JH_EPI_SWIGLU else rows
        k = P * (32 // bits)
        want = 2 * k if prologue == _lib.JH_PRO_SILU_MUL else k
        if x.numel != want:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"QuantMatvecFused: x has {x.numel} elements, needs {want}")
        residual = epilogue in (_lib.JH_EPI_RESID, _lib.JH_EPI_RESID_NORM)
        if residual and (resid is None or resid.dtype != F32 or resid.numel != n):
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatvecFused: resid must be F32 [out_features]")
        if prologue == _lib.JH_PRO_RMSNORM and (norm is None or norm.numel != k):
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatvecFused: RMSNorm needs a weight of in_features")
        if epilogue == _lib.JH_EPI_RESID_NORM and (norm is None or norm.numel != n or norm_out is None
                                                   or norm_out.dtype != BF16 or norm_out.numel != n):
            raise JanisHipError(_lib.JH_ERR_INVALID,
                                "QuantMatvecFused: the split norm needs norm [out] and a BF16 norm_out [out]")
        if (prologue == _lib.JH_PRO_NORMED or epilogue == _lib.JH_EPI_RESID_NORM) and (
                stats is None or stats.dtype != F32 or stats.numel != _lib.JH_NORM_STATS):
            raise JanisHipError(_lib.JH_ERR_INVALID, "QuantMatvecFused: stats must be F32 [JH_NORM_STATS]")
        yd = F32 if residual else (
            out_dtype if out_dtype is not None else (out.dtype if out is not None else x.dtype))
        y = out if out is not None else self.empty(yd, 1, n)
        check(self._ctx, self._L.jh_quant_matvec_fused(
            self._ctx, int(prologue), x.ptr, x.dtype, norm.ptr if norm is not None else None,
            norm.dtype if norm is not None else BF16, float(eps), w.ptr, scales.ptr, biases.ptr,
            self._sb_dtype(scales, biases), n, k, groupSize, bits, int(epilogue),
            resid.ptr if resid is not None else None, y.ptr, y.dtype,
            stats.ptr if stats is not None else None, norm_out.ptr if norm_out is not None else None))
        return y

    def NormPrepare(self, x: Tensor, norm: Tensor, norm_out: Tensor | None = None,
                    stats: Tensor | None = None) -> tuple:
        """The producer half of a split RMSNorm for a row already at hand (the
        embedding row): (bf16(x * norm) [1, d], F32 statistics [JH_NORM_STATS]),
        for a QuantMatvecFused with JH_PRO_NORMED."""
        d = x.shape[-1]
        if x.numel != d or norm.numel != d:
            raise JanisHipError(_lib.JH_ERR_INVALID, "NormPrepare: one row and a weight of its length")
        u = norm_out if norm_out is not None else self.empty(BF16, 1, d)
        st = stats if stats is not None else self.empty(F32, _lib.JH_NORM_STATS)
        check(self._ctx, self._L.jh_norm_prepare(self._ctx, x.ptr, x.dtype, d, norm.ptr, norm.dtype, u.ptr, st.ptr))
        return u, st

    def RoPETable(self, dims: int, base: float, scale: float, pos: int, freqs: Tensor | None = None) -> Tensor:
        """cos and sin of the RoPE angles at pos (cpu/cpu_attn.go:13-34): F32
        [dims] = [cos(theta_0..), sin(theta_0..)]."""
        out = self.empty(F32, dims)
        check(self._ctx, self._L.jh_rope_table(self._ctx, int(dims), float(base), float(scale), int(pos),
                                               freqs.ptr if freqs is not None else None, out.ptr))
        return out

    def AttentionDecode(self, qkv: Tensor, n_heads: int, n_kv_heads: int, q_norm: Tensor | None,
                        k_norm: Tensor | None, eps: float, base: float, rope_scale: float, pos: int,
                        k_cache: Tensor, v_cache: Tensor, scale: float, out_dtype: int | None = None,
                        rope_cs: Tensor | None = None) -> Tensor:
        """Attention.ForwardCached for one token after the q/k/v product
        (qwen/attention.go:98-128) in one launch: q/k RMSNorm (when the weights
        are given), RoPE at pos, the KV append at row pos, and SDPA over keys
        0..pos. qkv [.., (Hq+2Hk)*128]; caches bf16 [1, Hk, cap, 128]; rope_cs
        optionally RoPETable(128, base, rope_scale, pos). Returns [1, Hq*128]."""
        if q_norm is not None and k_norm is not None and q_norm.dtype != k_norm.dtype:
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: norm weights differ in dtype")
        if k_cache.dtype != v_cache.dtype or k_cache.shape != v_cache.shape:
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: caches differ")
        Dh = 128
        cap = k_cache.shape[-2]
        out = self.empty(out_dtype if out_dtype is not None else qkv.dtype, 1, n_heads * Dh)
        wd = q_norm.dtype if q_norm is not None else (k_norm.dtype if k_norm is not None else BF16)
        check(self._ctx, self._L.jh_attention_decode(
            self._ctx, qkv.ptr, qkv.dtype, n_heads, n_kv_heads, Dh, q_norm.ptr if q_norm is not None else None,
            k_norm.ptr if k_norm is not None else None, wd, float(eps), float(base), float(rope_scale),
            rope_cs.ptr if rope_cs is not None else None, int(pos),
            k_cache.ptr, v_cache.ptr, k_cache.dtype, cap, float(scale), out.ptr, out.dtype))
        return out

    def MoeRoute(self, logits: Tensor, k: int, normTopk: bool = True) -> tuple:
        """The router of MoEBlock.Forward (qwen/moe.go:455-491) on the device:
        softmax over the last axis, top-k (selection-sort ties), optional
        renormalisation. Returns (indices I32 [lead.., k], scores F32 [lead.., k])."""
        E = logits.shape[-1]
        n_tok = logits.numel // E if E else 0
        lead = logits.shape[:-1]
        idx = self.empty(I32, *lead, k)
        sc = self.empty(F32, *lead, k)
        check(self._ctx, self._L.jh_moe_route(self._ctx, logits.ptr, logits.dtype, n_tok, E, k,
                                              int(bool(normTopk)), idx.ptr, sc.ptr))
        return idx, sc

    def MoeSwiGLU(self, x: Tensor, gate: tuple, up: tuple, down: tuple, rhsIndices: Tensor,
                  scores: Tensor, groupSize: int, bits: int, out: Tensor | None = None,
                  out_dtype: int | None = None) -> Tensor:
        """The expert MLP of moeApply (qwen/moe.go:501-511) as one operator:
        sum_k scores[t, k] * down(SiLU(gate x_t) * up x_t) over the routed
        experts. x [lead.., H] bf16; gate/up/down are (W, S, B) stacks
        [E, I, H/8], [E, I, H/8], [E, H, I/8]; rhsIndices I32 and scores F32
        [lead.., K]. Returns [lead.., H] (F32 unless out_dtype says BF16)."""
        (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = gate, up, down
        for w in (wg, wu, wd):
            if w.dtype != U32 or len(w.shape) != 3:
                raise JanisHipError(_lib.JH_ERR_INVALID, "MoeSwiGLU: stacks must be U32 [E, out, P]")
        if rhsIndices.dtype != I32 or scores.dtype != F32 or rhsIndices.shape != scores.shape:
            raise JanisHipError(_lib.JH_ERR_INVALID, "MoeSwiGLU: indices I32 and scores F32 of one shape")
        E, I, Pg = wg.shape
        H = Pg * (32 // bits)
        if wu.shape != wg.shape or wd.shape != (E, H, I * bits // 32):
            raise JanisHipError(_lib.JH_ERR_INVALID, "MoeSwiGLU: stack shapes do not match")
        rs = rhsIndices.shape
        K = rs[-1]
        n_tok = int(np.prod(rs[:-1], dtype=np.int64)) if len(rs) > 1 else 1
        if x.shape[-1] != H or x.numel != n_tok * H:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"MoeSwiGLU: x {list(x.shape)} vs hidden={H}")
        od = out_dtype if out_dtype is not None else (out.dtype if out is not None else F32)
        y = out if out is not None else self.empty(od, *rs[:-1], H)
        check(self._ctx, self._L.jh_moe_swiglu(
            self._ctx, x.ptr, x.dtype, n_tok, wg.ptr, sg.ptr, bg.ptr, wu.ptr, su.ptr, bu.ptr,
            wd.ptr, sd.ptr, bd.ptr, self._sb_dtype(sg, bg), E, H, I, rhsIndices.ptr, scores.ptr, K,
            groupSize, bits, y.ptr, y.dtype))
        return y

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass
