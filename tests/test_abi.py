"""The C-ABI library: loads, exports every symbol include/jfh.h declares, and
its host-only runtime (prompt lookup, acceptance/rollback loop, payload codecs)
passes the C++ tests in tests/cpp. No GPU is touched here.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

import jetsonfabric_amd as jf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "jfh.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(jfh_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("jfh_model_open", "jfh_engine_create", "jfh_session_create", "jfh_session_prefill",
                     "jfh_session_decode", "jfh_session_verify", "jfh_session_rollback", "jfh_engine_step_batch",
                     "jfh_prompt_lookup_propose", "jfh_generate"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(jf.LIBRARY_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_bindings_cover_the_header():
    from jetsonfabric_amd import _capi

    assert set(declared_functions()) == set(_capi.SIGNATURES)


def test_product_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "jetsonfabric_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text and "jfo.h" not in text, f
    nm = subprocess.run(["nm", "-D", jf.LIBRARY_PATH], capture_output=True, text=True).stdout
    assert "jfo_" not in nm


def test_host_runtime_cpp_tests():
    exe = os.path.join(ROOT, "tests", "cpp", "runtime_test")
    # up to date with the library's headers (the tests use its C++ classes)
    subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout


def test_weight_tile_layout_cpp_tests():
    """Packs random GGML blocks into the gfx950 tiles and decodes them with
    the device tile decoder compiled for the host: bit-exact with the oracle."""
    exe = os.path.join(ROOT, "tests", "cpp", "tile_test")
    # up to date with the library's headers (the tests use its C++ classes)
    subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "tile tests passed" in r.stdout


def test_engine_creation_fails_loudly_without_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    cfg = jf.ModelConfig(n_layer=1, n_embd=256, n_ff=256, n_head=2, n_head_kv=1, n_vocab=256, n_ctx=64)
    m = jf.Model.synthesize(cfg, seed=1)
    with pytest.raises(jf.JfhError):
        jf.NativeEngine(m)
