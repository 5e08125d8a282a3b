"""CPU-side checks of the drop-in boundary: the HIP library is built for gfx950,
loads, exports exactly the entry points include/janis_hip.h declares, and the
product package never reaches the oracle. No compute call is made here."""
import ast
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "janis_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^JH_API[^(]*?\b(jh_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from janis_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from janis_amd import build

        build.build()
    return _lib.load()


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("jh_quant_matmul", "jh_gather_quant_matmul", "jh_dequantize", "jh_create"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    from janis_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r"\bT (jh_\w+)", out)))
    assert exported == declared_symbols()
    assert sorted(_lib.EXPORTS) == declared_symbols()
    for s in declared_symbols():
        assert hasattr(lib, s)


def test_library_carries_gfx950_code():
    from janis_amd import _lib

    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_version_and_no_device_error(lib):
    assert lib.jh_version().startswith(b"janis-hip-gfx950")
    try:
        import torch

        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except Exception:
        pass
    ctx = ctypes.c_void_p()
    rc = lib.jh_create(0, ctypes.byref(ctx))
    assert rc != 0 and not ctx.value
    assert lib.jh_last_error(None)


def test_null_context_is_rejected(lib):
    assert lib.jh_sync(None) != 0


def test_product_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "janis_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                tree = ast.parse(open(os.path.join(dirpath, f)).read())
                for node in ast.walk(tree):
                    if isinstance(node, ast.Import):
                        assert not any(a.name.split(".")[0] == "oracle" for a in node.names), f
                    if isinstance(node, ast.ImportFrom):
                        assert (node.module or "").split(".")[0] != "oracle", f
            if f.endswith((".hip", ".hpp", ".cpp", ".h")):
                assert "janis_oracle" not in open(os.path.join(dirpath, f)).read(), f
