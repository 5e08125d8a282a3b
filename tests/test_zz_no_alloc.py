"""jh_attention_decode_noalloc through the C ABI against jh_attention_decode:
two calls in a row on the same context, the second with a smaller input
(fewer heads, a shorter cache), each on its own copy of the same caches. The
output and the cache rows written are bit-identical to the allocating entry
point's, so sharing the attention kernels and putting the split partials in
the library's fixed device scratch changes nothing."""
import ctypes

import numpy as np
import pytest

from janis_amd import _lib, synth
from janis_amd.engine import BF16, F32, HipBackend
from tests.conftest import step

pytestmark = pytest.mark.gpu


def _case(hip, seed, Hq, Hk, cap, pos):
    """qkv, norm weights, and two identical pairs of bf16 caches filled with
    seeded N(0,1) rows."""
    Dh = 128
    qkv = hip.FromBF16Bits(synth.activations(seed, ((Hq + 2 * Hk) * Dh,))[0], (Hq + 2 * Hk) * Dh)
    qn = hip.FromBF16Bits(synth.f32_to_bf16_bits(1 + 0.05 * synth.normal(seed + 1, Dh).astype(np.float32)), Dh)
    kn = hip.FromBF16Bits(synth.f32_to_bf16_bits(1 + 0.05 * synth.normal(seed + 2, Dh).astype(np.float32)), Dh)
    kv = [synth.f32_to_bf16_bits(synth.normal(seed + 3 + i, Hk * cap * Dh).astype(np.float32)) for i in range(2)]
    caches = [[hip.FromBF16Bits(a, 1, Hk, cap, Dh) for a in kv] for _ in range(2)]
    return qkv, qn, kn, caches


def _call(hip, fn, qkv, qn, kn, Hq, Hk, pos, kc, vc, cap, out):
    return fn(hip._ctx, qkv.ptr, BF16, Hq, Hk, 128, qn.ptr, kn.ptr, BF16, ctypes.c_float(1e-6),
              ctypes.c_float(1e6), ctypes.c_float(1.0), None, pos, kc.ptr, vc.ptr, BF16, cap,
              ctypes.c_float(128 ** -0.5), out.ptr, F32)


@pytest.mark.parametrize("fresh", [True, False])
def test_attention_noalloc_matches_allocating_entry(hip, fresh):
    b = HipBackend(0) if fresh else hip  # a new context, or the session's (after the other tests)
    try:
        L = b._L
        for Hq, Hk, cap, pos in ((32, 8, 8200, 8192), (16, 4, 700, 600)):
            qkv, qn, kn, caches = _case(b, 900 + pos, Hq, Hk, cap, pos)
            outs = [b.empty(F32, 1, Hq * 128) for _ in range(2)]
            step(f"jh_attention_decode vs _noalloc Hq={Hq} Hk={Hk} pos={pos} fresh={fresh}")
            assert _call(b, L.jh_attention_decode, qkv, qn, kn, Hq, Hk, pos, *caches[0], cap, outs[0]) == _lib.JH_OK
            rc = _call(b, L.jh_attention_decode_noalloc, qkv, qn, kn, Hq, Hk, pos, *caches[1], cap, outs[1])
            assert rc == _lib.JH_OK, L.jh_last_error(b._ctx)
            want, got = b.Floats(outs[0]), b.Floats(outs[1])
            assert np.isfinite(want).all()
            assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
            for t0, t1 in zip(caches[0], caches[1]):
                assert b.Bytes(t0) == b.Bytes(t1)
    finally:
        if fresh:
            b.Close()
