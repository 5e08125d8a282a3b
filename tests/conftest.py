import os
import sys

import pytest

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
