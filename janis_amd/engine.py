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


def _dense_strides(shape) -> tuple:
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= int(d)
    return tuple(reversed(st))


class Tensor:
    """Device tensor: shape, dtype, device pointer, element strides (views from
    Slice/Transpose/ExpandDims are strided, as MLX's are). engine.Tensor
    (engine/backend.go:24-26)."""

    def __init__(self, backend: "HipBackend", ptr: int, shape, dtype: int, owned: bool = True, keep=None,
                 strides=None):
        self._b = backend
        self.ptr = int(ptr) if ptr else 0
        self.shape = tuple(int(d) for d in shape)
        self.dtype = dtype
        self._owned = owned
        self._keep = keep  # an object whose lifetime covers the memory (non-owned views)
        self.strides = tuple(int(x) for x in strides) if strides is not None else _dense_strides(self.shape)
        if backend is not None and owned and backend._sweeper is not None:
            backend._sweeper.track(self)

    @property
    def contiguous(self) -> bool:
        """Row-major dense (strides of length-1 axes do not matter)."""
        dense = _dense_strides(self.shape)
        return all(n == 1 or a == b for n, a, b in zip(self.shape, self.strides, dense))

    def Shape(self) -> list:
        return list(self.shape)

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * DTYPE_SIZE[self.dtype]

    def free(self) -> None:
        """Releases an owned allocation now (Freer.Free / Sweeper.Sweep)."""
        try:
            if self._owned and self.ptr and self._b._ctx:
                _lib.load().jh_free(self._b._ctx, ctypes.c_void_p(self.ptr))
        except Exception:
            pass
        self.ptr = 0

    def __del__(self):
        self.free()

    def __repr__(self):
        return f"Tensor({DTYPE_NAME[self.dtype]}, {list(self.shape)})"


class _Sweeper:
    """engine.Sweeper bookkeeping (engine/backend.go:43-51): owned tensors made
    while it is active are tracked; Sweep frees the unpinned ones still alive."""

    def __init__(self):
        import weakref
        self._live = weakref.WeakValueDictionary()  # id -> Tensor
        self._pinned = set()

    def track(self, t: "Tensor") -> None:
        self._live[id(t)] = t

    def pin_all(self) -> None:
        self._pinned.update(self._live.keys())

    def pin(self, ts) -> None:
        for t in ts:
            if t is not None:
                self._pinned.add(id(t))
                keep = getattr(t, "_keep", None)  # a view pins the memory it views
                if isinstance(keep, Tensor):
                    self.pin([keep])

    def unpin(self, ts) -> None:
        for t in ts:
            if t is not None:
                self._pinned.discard(id(t))
                keep = getattr(t, "_keep", None)
                if isinstance(keep, Tensor):
                    self.unpin([keep])

    def sweep(self) -> int:
        freed = 0
        for key, t in list(self._live.items()):
            if key not in self._pinned:
                t.free()
                del self._live[key]
                freed += 1
        self._pinned &= set(self._live.keys())
        return freed


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
        self._sweeper = None  # set by PinAll (engine.Sweeper)
        self._kv_reserve = 0  # CacheReserver.ReserveCache

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

    def Eval(self, *ts) -> None:
        """engine.Backend.Eval (engine/backend.go:168): operators run as they are
        called, so forcing evaluation is waiting for the stream (the Qwen session
        and the MoE block call it, qwen/session.go:319, qwen/moe.go:632, 652)."""
        self.Sync()

    def SetWaitLimit(self, polls: int) -> None:
        """jh_set_wait_limit: polls of the fused q/k/v + attention launch's
        in-kernel wait before it gives up (0: at once, for tests of the failure
        path, reported as JH_ERR_TIMEOUT by the next Sync)."""
        check(self._ctx, self._L.jh_set_wait_limit(self._ctx, int(polls)))

    # -- engine.Backend methods off this backend's path ------------------------------
    # The interface's other operators (engine/backend.go:180-248) serve models
    # outside the Qwen3 decode path (Gemma, Whisper, Qwen3.5's GatedDeltaNet);
    # they exist so the type satisfies the interface and fail loudly, as the
    # ggml backend does for its own gaps.
    def _unsupported(self, name: str):
        raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, f"{name}: not in this backend (engine/backend.go; "
                                                     f"off the quantized-linear decode path)")

    def MatMul(self, a: Tensor, b: Tensor) -> Tensor:
        self._unsupported("MatMul")

    def LayerNorm(self, x: Tensor, weight: Tensor, bias: Tensor, eps: float) -> Tensor:
        self._unsupported("LayerNorm")

    def Erf(self, x: Tensor) -> Tensor:
        self._unsupported("Erf")

    def Tanh(self, x: Tensor) -> Tensor:
        self._unsupported("Tanh")

    def Exp(self, x: Tensor) -> Tensor:
        self._unsupported("Exp")

    def Sigmoid(self, x: Tensor) -> Tensor:
        self._unsupported("Sigmoid")

    def Softplus(self, x: Tensor) -> Tensor:
        self._unsupported("Softplus")

    def Conv1dDepthwise(self, x: Tensor, w: Tensor) -> Tensor:
        self._unsupported("Conv1dDepthwise")

    def GatedDeltaScan(self, q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor) -> tuple:
        self._unsupported("GatedDeltaScan")

    def Gelu(self, x: Tensor) -> Tensor:
        self._unsupported("Gelu")

    def SetStream(self, stream_handle: int | None) -> None:
        """Enqueue on a caller's hipStream_t (e.g. torch.cuda.current_stream().cuda_stream)."""
        check(self._ctx, self._L.jh_set_stream(self._ctx, ctypes.c_void_p(stream_handle or 0)))

    # -- engine.Sweeper / engine.Freer ---------------------------------------------------
    def PinAll(self) -> None:
        """Pins everything made so far (after weight load) and starts tracking:
        tensors made from now on are freed by Sweep unless pinned."""
        if self._sweeper is None:
            self._sweeper = _Sweeper()
        self._sweeper.pin_all()

    def Pin(self, *ts) -> None:
        if self._sweeper is not None:
            self._sweeper.pin(ts)

    def Unpin(self, *ts) -> None:
        if self._sweeper is not None:
            self._sweeper.unpin(ts)

    def Sweep(self) -> int:
        """Frees every tracked, unpinned tensor (after the queued work that may
        read it). Returns how many were freed."""
        if self._sweeper is None:
            return 0
        self.Sync()
        return self._sweeper.sweep()

    def Free(self, *ts) -> None:
        """engine.Freer: releases the given tensors now (pinned ones are kept)."""
        self.Sync()
        for t in ts:
            if t is None or (self._sweeper is not None and id(t) in self._sweeper._pinned):
                continue
            t.free()

    def SetChecks(self, on) -> None:
        """Read-back checks like JANIS_GGML_CHECK (ggml/ggml.go:622-677): True or
        JH_CHECK_INDICES range-checks device indices, JH_CHECK_VALUES counts
        every float result for NaN/Inf (JH_ERR_NONFINITE); flags combine."""
        flags = _lib.JH_CHECK_INDICES if on is True else int(on)
        check(self._ctx, self._L.jh_set_checks(self._ctx, flags))

    def CheckFinite(self, t: Tensor) -> tuple:
        """(count of NaN/Inf values in t, index of the first, or numel when none)."""
        t = self._c(t)
        cnt, first = ctypes.c_int64(), ctypes.c_int64()
        check(self._ctx, self._L.jh_check_finite(self._ctx, t.ptr, t.dtype, t.numel, ctypes.byref(cnt),
                                                 ctypes.byref(first)))
        return cnt.value, first.value

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
        t = self._c(t)
        out = np.empty(t.nbytes, dtype=np.uint8)
        check(self._ctx, self._L.jh_d2h(self._ctx, out.ctypes.data_as(ctypes.c_void_p),
                                        ctypes.c_void_p(t.ptr), t.nbytes))
        return out.tobytes()

    def DTypeOf(self, t: Tensor) -> int:
        return t.dtype

    def Floats(self, t: Tensor) -> np.ndarray:
        """engine/backend.go:276-277: evaluates and copies out as float32."""
        t = self._c(t)
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
        """engine/backend.go:282-283: I32/U32 copied out as they are; a float
        tensor rounded half away from zero, as the CPU backend rounds its fp32
        data (cpu/cpu_misc.go:15-22)."""
        t = self._c(t)
        if t.dtype not in (I32, U32):
            f = self.Floats(t).astype(np.float64)
            return (np.sign(f) * np.floor(np.abs(f) + 0.5)).astype(np.int32)
        raw = np.frombuffer(self.Bytes(t), dtype=np.uint8)
        return raw.view(np.int32).reshape(t.shape).copy()

    def _result(self, op: str, out: Tensor | None, out_dtype: int | None, default_dtype: int, shape,
                dtypes=(F32, BF16)) -> Tensor:
        """The result buffer of an operator: `out` when given (checked: dense,
        exactly the result's element count, a dtype the operator writes and, when
        out_dtype is also given, that dtype), else a new tensor of `shape`."""
        n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
        if out is None:
            dt = out_dtype if out_dtype is not None else default_dtype
            if dt not in dtypes:
                raise JanisHipError(_lib.JH_ERR_INVALID, f"{op}: result dtype {DTYPE_NAME.get(dt, dt)} not in "
                                                         f"{[DTYPE_NAME[d] for d in dtypes]}")
            return self.empty(dt, *shape)
        self._live(out)
        if out.numel != n or not out.contiguous:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"{op}: out {list(out.shape)} must be a dense buffer of "
                                                     f"{n} elements ({list(shape)})")
        if out.dtype not in dtypes or (out_dtype is not None and out_dtype != out.dtype):
            raise JanisHipError(_lib.JH_ERR_INVALID, f"{op}: out is {DTYPE_NAME[out.dtype]}, needs "
                                                     f"{DTYPE_NAME.get(out_dtype, out_dtype) if out_dtype is not None else [DTYPE_NAME[d] for d in dtypes]}")
        return out

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
        w, scales, biases = self._c(w), self._c(scales), self._c(biases)
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
        x, w, scales, biases = self._c(x), self._c(w), self._c(scales), self._c(biases)
        n, P = w.shape[-2], w.shape[-1]
        k = P * (32 // bits)
        # transpose=false is MatMul(x, Dequantize(w)) (cpu/cpu_misc.go:233-236):
        # x [..., n] -> [..., k]
        x_feat, y_feat = (k, n) if transpose else (n, k)
        if x.shape[-1] != x_feat:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"QuantMatmul: x has {x.shape[-1]} features, needs {x_feat}")
        rows = x.numel // x_feat
        y = self._result("QuantMatmul", out, out_dtype, x.dtype, (*x.shape[:-1], y_feat))
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
        x, w, scales, biases, rhsIndices = (self._c(t) for t in (x, w, scales, biases, rhsIndices))
        E, n, P = w.shape
        k = P * (32 // bits)
        rs = rhsIndices.shape
        K = rs[-1]
        n_lead = int(np.prod(rs[:-1], dtype=np.int64)) if len(rs) > 1 else 1
        # transpose=false: each slot's MatMul(x, Dequantize(W_e)), x features = n
        x_feat, y_feat = (k, n) if transpose else (n, k)
        if x.shape[-1] != x_feat or len(x.shape) < 3:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"GatherQuantMatmul: x {list(x.shape)} vs {x_feat} features")
        A = x.shape[-3]
        if x.numel != n_lead * A * x_feat:
            raise JanisHipError(_lib.JH_ERR_INVALID, "GatherQuantMatmul: x lead dims do not match indices")
        y = self._result("GatherQuantMatmul", out, out_dtype, x.dtype, (*rs, 1, y_feat))
        check(self._ctx, self._L.jh_gather_quant_matmul(
            self._ctx, x.ptr, x.dtype, n_lead, A, w.ptr, scales.ptr, biases.ptr,
            self._sb_dtype(scales, biases), E, n, k, rhsIndices.ptr, K, int(bool(transpose)),
            groupSize, bits, y.ptr, y.dtype))
        return y

    # -- the other operators of a decode step ----------------------------------------
    # -- layout: views and copies (engine/backend.go: Reshape, Transpose, Slice, ...) --
    def _copy(self, x: Tensor, dst: Tensor, dst_strides=None) -> None:
        self._live(x), self._live(dst)
        nd = len(x.shape)
        sh = (ctypes.c_int64 * max(1, nd))(*x.shape)
        st = (ctypes.c_int64 * max(1, nd))(*x.strides)
        ds = (ctypes.c_int64 * max(1, nd))(*dst_strides) if dst_strides is not None else None
        check(self._ctx, self._L.jh_copy_strided(self._ctx, x.ptr, x.dtype, nd, sh, st, dst.ptr, dst.dtype, ds))

    @staticmethod
    def _live(x: Tensor) -> Tensor:
        """x, after checking that neither it nor the memory it views was freed
        (Sweep / Free): a freed tensor's address must never reach a kernel."""
        t = x
        while isinstance(t, Tensor):
            if t.ptr == 0 and (t._owned or t is x) and t.numel:
                raise JanisHipError(_lib.JH_ERR_INVALID, "tensor used after it was freed (Sweep / Free)")
            t = t._keep
        return x

    def _c(self, x: Tensor) -> Tensor:
        """x itself when dense, else a dense copy (what an op that reads memory
        linearly needs)."""
        self._live(x)
        if x.contiguous:
            return x
        out = self.empty(x.dtype, *x.shape)
        self._copy(x, out)
        return out

    def _view(self, x: Tensor, shape, strides, offset: int = 0) -> Tensor:
        return Tensor(self, x.ptr + offset * DTYPE_SIZE[x.dtype], shape, x.dtype, owned=False, keep=x,
                      strides=strides)

    def Reshape(self, x: Tensor, *shape) -> Tensor:
        """engine.Backend.Reshape: a view of the same memory when x is dense (one
        -1 allowed), else of a dense copy."""
        shape = list(shape)
        if shape.count(-1) == 1:
            known = int(np.prod([d for d in shape if d != -1], dtype=np.int64))
            shape[shape.index(-1)] = x.numel // known if known else 0
        if int(np.prod(shape, dtype=np.int64)) != x.numel:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Reshape: {list(x.shape)} -> {shape}")
        x = self._c(x)
        return Tensor(self, x.ptr, shape, x.dtype, owned=False, keep=x)

    def Transpose(self, x: Tensor, *perm) -> Tensor:
        """engine.Backend.Transpose: x's axes permuted, as a strided view."""
        if sorted(perm) != list(range(len(x.shape))):
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Transpose: {perm} is not a permutation of {len(x.shape)} axes")
        return self._view(x, [x.shape[a] for a in perm], [x.strides[a] for a in perm])

    def Slice(self, x: Tensor, axis: int, start: int, end: int) -> Tensor:
        """engine.Backend.Slice: [start:end] along axis, a view (full extent elsewhere)."""
        axis = axis % len(x.shape)
        if not 0 <= start <= end <= x.shape[axis]:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Slice: [{start}:{end}] of axis {axis} sized {x.shape[axis]}")
        shape = list(x.shape)
        shape[axis] = end - start
        return self._view(x, shape, x.strides, offset=start * x.strides[axis])

    def ExpandDims(self, x: Tensor, axis: int) -> Tensor:
        """engine.Backend.ExpandDims: a length-1 axis inserted, a view."""
        axis = axis % (len(x.shape) + 1)
        shape = list(x.shape)
        strides = list(x.strides)
        shape.insert(axis, 1)
        strides.insert(axis, strides[axis] * x.shape[axis] if axis < len(x.shape) else 1)
        return self._view(x, shape, strides)

    def Concat(self, a: Tensor, b: Tensor, axis: int) -> Tensor:
        """engine.Backend.Concat along axis (two strided copies into a new tensor)."""
        axis = axis % len(a.shape)
        if a.dtype != b.dtype or len(a.shape) != len(b.shape) or any(
                i != axis and x != y for i, (x, y) in enumerate(zip(a.shape, b.shape))):
            raise JanisHipError(_lib.JH_ERR_INVALID, f"Concat: {list(a.shape)} and {list(b.shape)} on axis {axis}")
        shape = list(a.shape)
        shape[axis] = a.shape[axis] + b.shape[axis]
        out = self.empty(a.dtype, *shape)
        self._copy(a, out, out.strides)
        tail = self._view(out, b.shape, out.strides, offset=a.shape[axis] * out.strides[axis])
        self._copy(b, tail, tail.strides)
        return out

    def Cast(self, x: Tensor, dt: int) -> Tensor:
        """engine.Backend.Cast between F32/F16/BF16 (round to nearest even)."""
        out = self.empty(dt, *x.shape)
        self._copy(x, out)
        return out

    def Contiguous(self, x: Tensor) -> Tensor:
        return self._c(x)

    def RMSNorm(self, x: Tensor, weight: Tensor, eps: float, out_dtype: int | None = None) -> Tensor:
        """cpu/cpu_ops.go:144-162 over the last axis."""
        x, weight = self._c(x), self._c(weight)
        d = x.shape[-1]
        out = self.empty(out_dtype if out_dtype is not None else x.dtype, *x.shape)
        check(self._ctx, self._L.jh_rms_norm(self._ctx, x.ptr, x.dtype, x.numel // d, d, weight.ptr, weight.dtype,
                                             float(eps), out.ptr, out.dtype))
        return out

    def _rope(self, x, dims, traditional, base, scale, offset, freqs, out_dtype):
        x = self._c(x)
        freqs = self._c(freqs) if freqs is not None else None
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
        """cpu/cpu_attn.go:64-119: q [B, Hq, Lq, Dh]; k/v [B, Hk, Lk, Dh], which may be
        views of the first Lk rows of caches [B, Hk, cap, Dh] (AppendKV's views:
        read in place), or whole caches of which the first kv_len rows count."""
        q = self._c(q)
        B, Hq, Lq, Dh = q.shape
        if k.shape != v.shape or k.dtype != v.dtype or k.shape[0] != B or k.shape[3] != Dh:
            raise JanisHipError(_lib.JH_ERR_INVALID, "SDPA: k/v shapes do not match q")
        Hk = k.shape[1]
        k, cap = self._kv_rows(k)
        v, vcap = self._kv_rows(v)
        if vcap != cap:  # one row stride for both
            k, v = self._c(k), self._c(v)
            cap = k.shape[2]
        Lk = k.shape[2] if kv_len is None else kv_len
        out = self.empty(out_dtype if out_dtype is not None else q.dtype, B, Hq, Lq, Dh)
        check(self._ctx, self._L.jh_sdpa(self._ctx, q.ptr, q.dtype, k.ptr, v.ptr, k.dtype, B, Hq, Hk, Lq, Lk, cap,
                                         Dh, float(scale), int(bool(causal)), out.ptr, out.dtype))
        return out

    def _kv_rows(self, t: Tensor) -> tuple:
        """(t, row capacity) when t's rows sit in a [B, H, cap, D] buffer with
        dense rows (a cache view), else (dense copy, its row count)."""
        B, H, L, D = t.shape
        st = t.strides
        if st[3] == 1 and st[2] == D and st[1] % D == 0 and st[1] // D >= L and (B == 1 or st[0] == H * st[1]):
            return t, st[1] // D
        t = self._c(t)
        return t, L


    def _broadcast(self, x: Tensor, shape) -> Tensor:
        """x expanded to `shape` by numpy broadcasting (length-1 or missing
        leading axes repeat), as the CPU backend's elementwise ops read their
        operands (cpu/cpu.go:290-298): a zero-stride view copied dense."""
        shape = tuple(shape)
        if tuple(x.shape) == shape:
            return x
        lead = len(shape) - len(x.shape)
        if lead < 0:
            raise JanisHipError(_lib.JH_ERR_INVALID, f"broadcast: {list(x.shape)} to {list(shape)}")
        st = []
        for ax, n in enumerate(shape):
            if ax < lead:
                st.append(0)
                continue
            d, s_ = x.shape[ax - lead], x.strides[ax - lead]
            if d == n:
                st.append(s_)
            elif d == 1:
                st.append(0)
            else:
                raise JanisHipError(_lib.JH_ERR_INVALID, f"broadcast: {list(x.shape)} to {list(shape)}")
        out = self.empty(x.dtype, *shape)
        self._copy(self._view(x, shape, st), out)
        return out

    @staticmethod
    def _broadcast_shape(a, b) -> tuple:
        n = max(len(a), len(b))
        a, b = (1,) * (n - len(a)) + tuple(a), (1,) * (n - len(b)) + tuple(b)
        out = []
        for x, y in zip(a, b):
            if x != y and x != 1 and y != 1:
                raise JanisHipError(_lib.JH_ERR_INVALID, f"shapes {list(a)} and {list(b)} do not broadcast")
            out.append(max(x, y) if x and y else 0)
        return tuple(out)

    def _elementwise(self, op, a, b, out_dtype):
        if b is not None and tuple(a.shape) != tuple(b.shape):
            shape = self._broadcast_shape(a.shape, b.shape)
            a, b = self._broadcast(a, shape), self._broadcast(b, shape)
        a = self._c(a)
        b = self._c(b) if b is not None else None
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

    @staticmethod
    def _axis_view(x: Tensor, axis: int) -> tuple:
        axis = axis % len(x.shape)
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        return axis, outer, x.shape[axis], inner

    def Softmax(self, x: Tensor, axis: int) -> Tensor:
        """engine.Backend.Softmax (cpu/cpu.go:461-499): F32 of x's shape."""
        x = self._c(x)
        _, outer, n, inner = self._axis_view(x, axis)
        out = self.empty(F32, *x.shape)
        check(self._ctx, self._L.jh_softmax(self._ctx, x.ptr, x.dtype, outer, n, inner, out.ptr))
        return out

    def Mean(self, x: Tensor, axis: int) -> Tensor:
        """engine.Backend.Mean (cpu/cpu_ops.go:113-142): the axis removed, F32."""
        x = self._c(x)
        ax, outer, n, inner = self._axis_view(x, axis)
        out = self.empty(F32, *x.shape[:ax], *x.shape[ax + 1:])
        check(self._ctx, self._L.jh_mean(self._ctx, x.ptr, x.dtype, outer, n, inner, out.ptr))
        return out

    def _scalar(self, op, x, v, out_dtype):
        x = self._c(x)
        out = self.empty(out_dtype if out_dtype is not None else x.dtype, *x.shape)
        check(self._ctx, self._L.jh_scalar(self._ctx, op, x.ptr, x.dtype, x.numel, float(v), out.ptr, out.dtype))
        return out

    def ScalarMul(self, x: Tensor, v: float, out_dtype: int | None = None) -> Tensor:
        """engine.Backend.ScalarMul (cpu/cpu_misc.go:24-26): x * v."""
        return self._scalar(_lib.JH_SCALAR_MUL, x, v, out_dtype)

    def ScalarAdd(self, x: Tensor, v: float, out_dtype: int | None = None) -> Tensor:
        """engine.Backend.ScalarAdd (cpu/cpu_misc.go:28-30): x + v."""
        return self._scalar(_lib.JH_SCALAR_ADD, x, v, out_dtype)

    def Argmax(self, x: Tensor, axis: int = -1) -> Tensor:
        """cpu/cpu_misc.go:91-121, last axis only."""
        if axis not in (-1, len(x.shape) - 1):
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "Argmax: last axis only")
        x = self._c(x)
        n = x.shape[-1]
        out = self.empty(I32, *x.shape[:-1])
        check(self._ctx, self._L.jh_argmax(self._ctx, x.ptr, x.dtype, x.numel // n, n, out.ptr))
        return out

    def TakeAxis(self, a: Tensor, indices: Tensor, axis: int = 0) -> Tensor:
        """cpu/cpu_misc.go:48-89 on axis 0 (rows of any dtype, packed words included)."""
        if axis != 0 or indices.dtype != I32:
            raise JanisHipError(_lib.JH_ERR_UNSUPPORTED, "TakeAxis: axis 0 with I32 indices only")
        a, indices = self._c(a), self._c(indices)
        rows = a.shape[0]
        row_bytes = a.nbytes // rows if rows else 0
        out = self.empty(a.dtype, *indices.shape, *a.shape[1:])
        check(self._ctx, self._L.jh_take_rows(self._ctx, a.ptr, row_bytes, rows, indices.ptr, indices.numel, out.ptr))
        return out

    def ScatterRows(self, dst: Tensor, indices, updates: Tensor) -> Tensor:
        """engine.RowScatterer (engine/backend.go:95-105; CPU semantics
        cpu/cpu_ops.go:215-233): a new tensor equal to dst with row indices[i]
        (axis 0) replaced by updates[i]; updates is [len(indices), *dst.shape[1:]]
        of dst's dtype, indices host int32 as the interface passes them. A
        repeated index keeps its last update; one outside [0, rows) raises."""
        idx = np.ascontiguousarray(np.asarray(indices, dtype=np.int32).reshape(-1))
        if updates.dtype != dst.dtype or tuple(updates.shape) != (idx.size, *dst.shape[1:]):
            raise JanisHipError(_lib.JH_ERR_INVALID,
                                f"ScatterRows: updates {DTYPE_NAME[updates.dtype]}{list(updates.shape)} for dst "
                                f"{DTYPE_NAME[dst.dtype]}{list(dst.shape)} and {idx.size} indices")
        dst, updates = self._c(dst), self._c(updates)
        rows = dst.shape[0]
        out = self.empty(dst.dtype, *dst.shape)
        check(self._ctx, self._L.jh_scatter_rows(self._ctx, dst.ptr, out.ptr, rows, dst.nbytes // rows if rows else 0,
                                                 idx.ctypes.data, idx.size, updates.ptr))
        return out

    KV_STEP = 256  # cache capacity granularity (tokens)
    KV_AHEAD = 2048  # at most this many tokens of room beyond what a request needs now

    def ReserveCache(self, tokens: int) -> None:
        """engine.CacheReserver: size the caches made from now on for `tokens`."""
        self._kv_reserve = int(tokens)

    def AppendKV(self, buf: Tensor | None, view: Tensor | None, n: int, x: Tensor) -> tuple:
        """engine.KVAppender (engine/backend.go:56-61): writes x [B, H, L, D] into buf
        at token n (axis 2) in place, growing buf when it has no room (buf None: a
        new one; view's first n tokens are copied in first), and returns (buf, the
        view of its first n+L tokens). A new buffer holds max(need, min(reserve,
        need + KV_AHEAD)) tokens rounded up to KV_STEP, as the MLX backend sizes
        them (mlxc/mlxc.go:283-306); rows past the view are never read."""
        B, H, L, D = x.shape
        need = n + L
        if buf is None or buf.shape[2] < need or buf.shape[:2] != (B, H) or buf.shape[3] != D:
            cap = max(need, min(self._kv_reserve, need + self.KV_AHEAD))
            cap = (cap + self.KV_STEP - 1) // self.KV_STEP * self.KV_STEP
            grown = self.empty(x.dtype if buf is None else buf.dtype, B, H, cap, D)
            if n > 0 and view is not None:
                src = self.Slice(view, 2, 0, n)
                self._copy(src, self._view(grown, src.shape, grown.strides), grown.strides)
            buf = grown
        dst = self._view(buf, x.shape, buf.strides, offset=n * buf.strides[2])
        self._copy(x, dst, buf.strides)
        return buf, self.Slice(buf, 2, 0, need)

    def AppendKVRows(self, k_cache: Tensor, v_cache: Tensor, pos: int, k_new: Tensor, v_new: Tensor) -> None:
        """Both caches at once with one launch: caches [B, Hk, cap, Dh], new rows
        [B, Hk, L, Dh] at pos (jh_kv_append)."""
        k_new, v_new = self._c(k_new), self._c(v_new)
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
        qkv, q_norm, k_norm = self._c(qkv), self._c(q_norm), self._c(k_norm)
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
        x, w, scales, biases = self._c(x), self._c(w), self._c(scales), self._c(biases)
        norm = self._c(norm) if norm is not None else None
        resid = self._c(resid) if resid is not None else None
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
        if residual:
            y = self._result("QuantMatvecFused", out, out_dtype, F32, (1, n), dtypes=(F32,))
        else:
            y = self._result("QuantMatvecFused", out, out_dtype, x.dtype, (1, n))
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
        x, norm = self._c(x), self._c(norm)
        d = x.shape[-1]
        if x.numel != d or norm.numel != d:
            raise JanisHipError(_lib.JH_ERR_INVALID, "NormPrepare: one row and a weight of its length")
        u = norm_out if norm_out is not None else self.empty(BF16, 1, d)
        st = stats if stats is not None else self.empty(F32, _lib.JH_NORM_STATS)
        check(self._ctx, self._L.jh_norm_prepare(self._ctx, x.ptr, x.dtype, d, norm.ptr, norm.dtype, u.ptr, st.ptr))
        return u, st

    def EmbedNormPrepare(self, ids: Tensor, w: Tensor, scales: Tensor, biases: Tensor, groupSize: int, bits: int,
                         norm: Tensor, rope: tuple | None = None) -> tuple:
        """The decode step's first launch: the embedding row of token ids[0]
        (QuantEmbedding.Forward, qwen/embed.go:78-83: Dequantize of the TakeAxis
        rows), NormPrepare on it with norm, and with rope = (dims, base, scale,
        pos) the RoPETable at pos. Returns (h F32 [1, d], u BF16 [1, d], stats,
        cs or None), each bit-identical to the separate calls."""
        if w.dtype != U32 or len(w.shape) != 2:
            raise JanisHipError(_lib.JH_ERR_INVALID, "EmbedNormPrepare: table is not packed U32 [vocab, P]")
        ids, w, scales, biases, norm = (self._c(t) for t in (ids, w, scales, biases, norm))
        if ids.dtype != I32 or ids.numel != 1:
            raise JanisHipError(_lib.JH_ERR_INVALID, "EmbedNormPrepare: one I32 token id")
        vocab, d = w.shape[0], w.shape[-1] * 32 // bits
        if norm.numel != d:
            raise JanisHipError(_lib.JH_ERR_INVALID, "EmbedNormPrepare: norm weight of the row's length")
        h, u, st = self.empty(F32, 1, d), self.empty(BF16, 1, d), self.empty(F32, _lib.JH_NORM_STATS)
        cs = self.empty(F32, int(rope[0])) if rope is not None else None
        rd, rb, rs, rp = rope if rope is not None else (0, 0.0, 0.0, 0)
        check(self._ctx, self._L.jh_embed_norm_prepare(
            self._ctx, ids.ptr, w.ptr, scales.ptr, biases.ptr, self._sb_dtype(scales, biases), vocab, d, groupSize,
            bits, norm.ptr, norm.dtype, h.ptr, u.ptr, st.ptr, int(rd), float(rb), float(rs), int(rp),
            cs.ptr if cs is not None else None))
        return h, u, st, cs

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
                        rope_cs: Tensor | None = None, out: Tensor | None = None, noalloc: bool = False) -> Tensor:
        """Attention.ForwardCached for one token after the q/k/v product
        (qwen/attention.go:98-128) in one launch: q/k RMSNorm (when the weights
        are given), RoPE at pos, the KV append at row pos, and SDPA over keys
        0..pos. qkv [.., (Hq+2Hk)*128]; caches bf16 [1, Hk, cap, 128]; rope_cs
        optionally RoPETable(128, base, rope_scale, pos). Returns [1, Hq*128].
        noalloc=True takes jh_attention_decode_noalloc (partials in the
        library's fixed device scratch instead of the context's workspace)."""
        if q_norm is not None and k_norm is not None and q_norm.dtype != k_norm.dtype:
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: norm weights differ in dtype")
        if k_cache.dtype != v_cache.dtype or k_cache.shape != v_cache.shape:
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: caches differ")
        if not (k_cache.contiguous and v_cache.contiguous):
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: the caches must be whole buffers")
        qkv = self._c(qkv)
        q_norm = self._c(q_norm) if q_norm is not None else None
        k_norm = self._c(k_norm) if k_norm is not None else None
        Dh = 128
        cap = k_cache.shape[-2]
        if out is None:
            out = self.empty(out_dtype if out_dtype is not None else qkv.dtype, 1, n_heads * Dh)
        elif out.numel != n_heads * Dh or out.dtype not in (F32, BF16):
            raise JanisHipError(_lib.JH_ERR_INVALID, "AttentionDecode: out must be F32/BF16 [1, Hq*128]")
        wd = q_norm.dtype if q_norm is not None else (k_norm.dtype if k_norm is not None else BF16)
        fn = self._L.jh_attention_decode_noalloc if noalloc else self._L.jh_attention_decode
        check(self._ctx, fn(
            self._ctx, qkv.ptr, qkv.dtype, n_heads, n_kv_heads, Dh, q_norm.ptr if q_norm is not None else None,
            k_norm.ptr if k_norm is not None else None, wd, float(eps), float(base), float(rope_scale),
            rope_cs.ptr if rope_cs is not None else None, int(pos),
            k_cache.ptr, v_cache.ptr, k_cache.dtype, cap, float(scale), out.ptr, out.dtype))
        return out

    def QkvAttentionDecode(self, x: Tensor, stats: Tensor, norm_eps: float, w: Tensor, scales: Tensor,
                           biases: Tensor, groupSize: int, bits: int, qkv: Tensor, n_heads: int, n_kv_heads: int,
                           q_norm: Tensor | None, k_norm: Tensor | None, eps: float, base: float, rope_scale: float,
                           pos: int, k_cache: Tensor, v_cache: Tensor, scale: float,
                           rope_cs: Tensor | None = None, out: Tensor | None = None,
                           out_dtype: int | None = None) -> Tensor:
        """The q/k/v product of one token (JH_PRO_NORMED: x = the bf16 norm_out of
        a split RMSNorm and `stats` its statistics; w stacks the q, k and v rows)
        written to `qkv` (F32 or BF16 [1, (Hq+2Hk)*128]) and its attention (as
        AttentionDecode) in one launch when the backend has it: the same results
        as QuantMatvecFused(PRO_NORMED) then AttentionDecode, bit for bit
        (qwen/attention.go:98-128 after qwen/block.go:59). Returns [1, Hq*128]."""
        if w.dtype != U32:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: weight tensor is not packed U32")
        if k_cache.dtype != v_cache.dtype or k_cache.shape != v_cache.shape:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: caches differ")
        if not (k_cache.contiguous and v_cache.contiguous):
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: the caches must be whole buffers")
        if q_norm is not None and k_norm is not None and q_norm.dtype != k_norm.dtype:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: norm weights differ in dtype")
        x, w, scales, biases = self._c(x), self._c(w), self._c(scales), self._c(biases)
        Dh = 128
        rows, P = w.shape[-2], w.shape[-1]
        k = P * (32 // bits)
        if rows != (n_heads + 2 * n_kv_heads) * Dh:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: w must hold (Hq + 2 Hk) * 128 rows")
        if x.dtype != BF16 or x.numel != k:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: x must be the BF16 norm_out [in_features]")
        if stats.dtype != F32 or stats.numel != _lib.JH_NORM_STATS:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: stats must be F32 [JH_NORM_STATS]")
        if qkv.dtype not in (F32, BF16) or qkv.numel != rows:
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: qkv must be F32/BF16 [1, (Hq + 2 Hk) * 128]")
        if out is None:
            out = self.empty(out_dtype if out_dtype is not None else BF16, 1, n_heads * Dh)
        elif out.numel != n_heads * Dh or out.dtype not in (F32, BF16):
            raise JanisHipError(_lib.JH_ERR_INVALID, "QkvAttentionDecode: out must be F32/BF16 [1, Hq*128]")
        q_norm = self._c(q_norm) if q_norm is not None else None
        k_norm = self._c(k_norm) if k_norm is not None else None
        wd = q_norm.dtype if q_norm is not None else (k_norm.dtype if k_norm is not None else BF16)
        check(self._ctx, self._L.jh_qkv_attention_decode(
            self._ctx, x.ptr, stats.ptr, float(norm_eps), w.ptr, scales.ptr, biases.ptr, scales.dtype, k,
            int(groupSize), int(bits), qkv.ptr, qkv.dtype, n_heads, n_kv_heads, Dh,
            q_norm.ptr if q_norm is not None else None, k_norm.ptr if k_norm is not None else None, wd, float(eps),
            float(base), float(rope_scale), rope_cs.ptr if rope_cs is not None else None, int(pos),
            k_cache.ptr, v_cache.ptr, k_cache.dtype, k_cache.shape[-2], float(scale), out.ptr, out.dtype))
        return out

    def MoeRoute(self, logits: Tensor, k: int, normTopk: bool = True) -> tuple:
        """The router of MoEBlock.Forward (qwen/moe.go:455-491) on the device:
        softmax over the last axis, top-k (selection-sort ties), optional
        renormalisation. Returns (indices I32 [lead.., k], scores F32 [lead.., k])."""
        logits = self._c(logits)
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
        (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = ((self._c(t) for t in m) for m in (gate, up, down))
        x, rhsIndices, scores = self._c(x), self._c(rhsIndices), self._c(scores)
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
        y = self._result("MoeSwiGLU", out, out_dtype, F32, (*rs[:-1], H))
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
