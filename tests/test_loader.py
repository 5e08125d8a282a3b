"""The MLX-checkpoint loader: the safetensors reader against an independent
implementation (the safetensors package) and against what was written; the
config defaults of qwen/config.go. CPU only."""
import json
import os

import numpy as np
import pytest

from janis_amd import loader
from tests.golden.write_tiny_checkpoint import tiny_qwen3, write_safetensors


def test_reader_matches_the_safetensors_package(tmp_path):
    st_np = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(1)
    t = {"a": rng.integers(0, 2**32, (7, 5), dtype=np.uint32), "b": rng.standard_normal((3, 4)).astype(np.float32),
         "c": rng.standard_normal(9).astype(np.float16), "d": np.arange(6, dtype=np.int32).reshape(2, 3)}
    path = str(tmp_path / "x.safetensors")
    st_np.save_file(t, path)
    r = loader.SafeTensors(path)
    for name, arr in t.items():
        dt, shape, raw = r.raw(name)
        assert shape == arr.shape
        assert np.array_equal(np.frombuffer(raw.tobytes(), dtype=arr.dtype).reshape(shape), arr)
    # and the package reads what this repository's writer writes
    path2 = str(tmp_path / "y.safetensors")
    write_safetensors(path2, {k: ({np.uint32: "U32", np.float32: "F32", np.float16: "F16", np.int32: "I32"}[
        v.dtype.type], v.shape, v) for k, v in t.items()})
    back = st_np.load_file(path2)
    for name, arr in t.items():
        assert np.array_equal(back[name], arr)


def test_tiny_checkpoint_tensors_and_config(tmp_path):
    d = str(tmp_path / "m")
    host = tiny_qwen3(d, layers=1)
    ck = loader.Checkpoint(d)
    dt, shape, raw = ck.where["model.layers.0.mlp.up_proj.weight"].raw("model.layers.0.mlp.up_proj.weight")
    q = host["model.layers.0.mlp.up_proj"]
    assert dt == "U32" and shape == q.w.shape
    assert np.array_equal(np.frombuffer(raw.tobytes(), np.uint32).reshape(shape), q.w)
    dt, shape, raw = ck.where["model.norm.weight"].raw("model.norm.weight")
    assert dt == "BF16" and shape == (512,)
    cfg = loader.load_config(d)
    assert (cfg.hidden, cfg.inter, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.vocab, cfg.layers) == \
        (512, 1024, 4, 2, 128, 1000, 1)
    assert cfg.group_size == 64 and cfg.bits == 4 and not cfg.tie
    # qwen/config.go defaults: head_dim = hidden / heads, kv heads = heads, tied unless stated
    with open(os.path.join(d, "config.json")) as f:
        c = json.load(f)
    for k in ("head_dim", "num_key_value_heads", "tie_word_embeddings"):
        del c[k]
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(c, f)
    cfg = loader.load_config(d)
    assert cfg.head_dim == 128 and cfg.n_kv == 4 and cfg.tie


def test_sharded_index(tmp_path):
    d = tmp_path / "s"
    d.mkdir()
    write_safetensors(str(d / "a.safetensors"), {"x": ("F32", (2,), np.array([1, 2], np.float32))})
    write_safetensors(str(d / "b.safetensors"), {"y": ("I32", (1,), np.array([7], np.int32))})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "a.safetensors",
                                                                               "y": "b.safetensors"}}))
    ck = loader.Checkpoint(str(d))
    assert ck.has("x") and ck.has("y") and not ck.has("z")
    assert np.frombuffer(ck.where["y"].raw("y")[2].tobytes(), np.int32)[0] == 7
