"""janis_amd: an MI355X (gfx950) backend for janis's MLX affine-quantized
matrix products (decode GEMV, prefill GEMM, MoE expert gather).

The product is libjanis_hip.so (HIP kernels + the C ABI of include/janis_hip.h);
`engine.HipBackend` mirrors the reference's engine.Backend methods over it.
"""
from . import _lib  # noqa: F401

__all__ = ["engine", "synth", "build"]
