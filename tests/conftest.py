import os
import sys

import pytest

try:
    # torch first: a test that makes device buffers with torch needs torch's HIP
    # runtime to be the one the process loaded, before libjanis_hip.so is
    # loaded by the first fixture (the library then binds to it, as bench.py does)
    import torch  # noqa: F401
except Exception:  # torch is optional for every other test
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def rel_ok(got, want, rel):
    """relOK of the reference tests (ggml/ggml_test.go:56-65): every element
    within rel * max|want| of the oracle. Returns (ok, max_abs_diff, scale)."""
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    d = float(np.max(np.abs(got - want))) if want.size else 0.0
    return (d <= rel * scale and not np.isnan(d)), d, scale


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def hip():
    """The backend under test on cuda:0 (the HIP path; there is no fallback)."""
    from janis_amd.engine import HipBackend

    b = HipBackend(0)
    print(f"\n[hip] {b.Version()} | {b.EngineInfo()}", flush=True)
    yield b
    b.Close()


def upload_quant(b, q):
    """Uploads a synth.QuantLinear as (W U32, scales BF16, biases BF16)."""
    from janis_amd.engine import U32

    w = b.FromRaw(U32, q.w, *q.w.shape)
    s = b.FromBF16Bits(q.s_bits, *q.s_bits.shape)
    bb = b.FromBF16Bits(q.b_bits, *q.b_bits.shape)
    return w, s, bb


def step(msg):
    """Names the GPU case about to run, flushed before the launch."""
    print(f"  [gpu] {msg}", flush=True)


_RT = None


def hip_runtime():
    """libamdhip64 (the one libjanis_hip.so links) through ctypes, for tests
    that capture and replay HIP graphs on a stream of their own."""
    global _RT
    if _RT is None:
        import ctypes
        import subprocess

        from janis_amd import _lib as jl

        jl.load()
        # the HIP runtime this process already loaded (torch's when torch came
        # first, else the one the library links); a second copy would not resolve
        path = None
        with open("/proc/self/maps") as f:
            for ln in f:
                if "libamdhip64" in ln:
                    path = ln.split()[-1]
                    break
        if path is None:
            out = subprocess.run(["ldd", jl.LIB_PATH], capture_output=True, text=True).stdout
            path = next(ln.split("=>")[1].split()[0] for ln in out.splitlines() if "libamdhip64" in ln)
        rt = ctypes.CDLL(path)
        for name in ("hipStreamCreate", "hipStreamSynchronize", "hipStreamBeginCapture", "hipStreamEndCapture",
                     "hipGraphInstantiate", "hipGraphLaunch", "hipGraphExecDestroy", "hipGraphDestroy",
                     "hipStreamDestroy"):
            getattr(rt, name).restype = ctypes.c_int
        _RT = rt
    return _RT


class Graph:
    """One HIP graph captured from `fn` on a stream of its own (the backend
    enqueues on that stream meanwhile); replay() launches it and waits."""

    def __init__(self, hip, fn):
        import ctypes

        self.rt, self.hip = hip_runtime(), hip
        self.stream, self.graph, self.exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        assert self.rt.hipStreamCreate(ctypes.byref(self.stream)) == 0
        hip.SetStream(self.stream.value)
        assert self.rt.hipStreamBeginCapture(self.stream, 0) == 0
        try:
            fn()
        finally:
            rc = self.rt.hipStreamEndCapture(self.stream, ctypes.byref(self.graph))
            hip.SetStream(None)
        assert rc == 0
        assert self.rt.hipGraphInstantiate(ctypes.byref(self.exe), self.graph, None, None, 0) == 0

    def replay(self):
        assert self.rt.hipGraphLaunch(self.exe, self.stream) == 0
        assert self.rt.hipStreamSynchronize(self.stream) == 0

    def close(self):
        if self.exe.value:
            self.rt.hipGraphExecDestroy(self.exe)
        if self.graph.value:
            self.rt.hipGraphDestroy(self.graph)
        if self.stream.value:
            self.rt.hipStreamDestroy(self.stream)
        self.exe = self.graph = self.stream = type(self.stream)()


def put(hip, t, a):
    """Host array a written over device tensor t (same bytes), synchronously."""
    import ctypes

    import numpy as np

    a = np.ascontiguousarray(a)
    assert a.nbytes == t.nbytes, (a.nbytes, t.nbytes)
    hip.Sync()
    hip._L.jh_h2d(hip._ctx, ctypes.c_void_p(t.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
    hip.Sync()
