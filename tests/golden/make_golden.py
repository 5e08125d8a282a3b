"""Writes the golden fixtures under tests/golden/ from data files that janis's
own tests hold. Run once in a container where /root/reference is mounted:

    python tests/golden/make_golden.py /root/reference

Fixtures written (all data, no code):

inkling2_embed_{f32,bf16}.npz
    From inkling2/testdata/tiny-{f32,bf16}/ (produced by mlx-lm, see
    inkling2/testdata/gen_fixture.py:330-340 in the reference): the MLX
    4-bit group-64 quantized embedding table (weight uint32 [128, 8], scales and
    biases [128, 1]), embed_norm.weight [64], the token ids [20] and the
    expected embedding output [20, 64] = RMSNorm(Dequantize(rows), eps 1e-6),
    which inkling2/reference_test.go:100-122 checks at 2e-4 (f32) and 5e-2
    (bf16) of the largest value. bf16 tensors are stored as uint16 bit patterns.

The safetensors files are parsed as a JSON header plus raw little-endian
buffers; nothing in them is executed.
"""
from __future__ import annotations

import json
import os
import struct
import sys

import numpy as np

_DT = {"F32": np.float32, "U32": np.uint32, "I32": np.int32, "BF16": np.uint16, "F16": np.float16,
       "U8": np.uint8, "I8": np.int8, "I64": np.int64, "F64": np.float64, "BOOL": np.uint8}


def read_safetensors(path: str) -> dict:
    with open(path, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen))
        base = 8 + hlen
        out = {}
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            lo, hi = meta["data_offsets"]
            f.seek(base + lo)
            buf = f.read(hi - lo)
            arr = np.frombuffer(buf, dtype=_DT[meta["dtype"]]).reshape(meta["shape"])
            out[name] = (meta["dtype"], arr.copy())
        return out


def main(ref_root: str) -> None:
    here = os.path.dirname(os.path.abspath(__file__))
    for name in ("f32", "bf16"):
        d = os.path.join(ref_root, "inkling2", "testdata", f"tiny-{name}")
        model = read_safetensors(os.path.join(d, "model.safetensors"))
        expected = read_safetensors(os.path.join(d, "expected.safetensors"))
        pre = "model.language_model."
        fx = {}
        for key, short in (("embed_tokens.weight", "w"), ("embed_tokens.scales", "s"),
                           ("embed_tokens.biases", "b"), ("embed_norm.weight", "norm")):
            dt, arr = model[pre + key]
            fx[short] = arr
            fx[short + "_dtype"] = np.array(dt)
        fx["tokens"] = expected["tokens"][1]
        fx["embed"] = expected["embed"][1]
        cfg = json.load(open(os.path.join(d, "config.json")))
        fx["group_size"] = np.array(cfg["quantization"]["group_size"])
        fx["bits"] = np.array(cfg["quantization"]["bits"])
        fx["eps"] = np.array(cfg["text_config"]["rms_norm_eps"], dtype=np.float64)
        np.savez(os.path.join(here, f"inkling2_embed_{name}.npz"), **fx)
        print(name, {k: (v.dtype, v.shape) for k, v in fx.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
