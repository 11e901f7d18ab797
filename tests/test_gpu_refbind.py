"""The engine behind the reference runtime's own compiled Executor contract.

tests/refbind/refbind_test.cpp, in this process: the C-ABI HipStageExecutor
of tests/refbind compiled against the reference's runtime/inference
contract sources (stage.cpp, token_payload.cpp, executor.hpp) and wrapped in
the reference's ContinuousBatchingExecutor
(runtime/pipeline_parallel/continuous_batching_executor.cpp), built from
those sources by tests/refbind/Makefile. It runs the serving and
distributed cases of native_stage_executor_test.cpp:72-230 on the reference's
two-layer fixture package, verify and execute_batch against serial decode,
and continuous_batching_executor_test.cpp's coalescing case with concurrent
generations checked against direct decode loops.
"""
from __future__ import annotations

import ctypes
import os

import pytest

import jetsonfabric_amd as jf
from tests.golden import tiny_fixture

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tests", "refbind", "_ref", "librefbind.so")


def _inputs():
    yield jf.LIBRARY_PATH
    yield os.path.join(ROOT, "include", "jfh.h")
    for name in ("hip_stage_executor.cpp", "hip_stage_executor.hpp", "refbind_test.cpp"):
        yield os.path.join(ROOT, "tests", "refbind", name)


def test_reference_executor_contract_drives_the_engine(tmp_path, capfd):
    if not os.path.exists(LIB):
        pytest.skip("tests/refbind/_ref/librefbind.so is built only where the reference checkout is present "
                    "(make -C tests/refbind)")
    newest = max(os.path.getmtime(p) for p in _inputs())
    assert os.path.getmtime(LIB) >= newest, "tests/refbind/_ref/librefbind.so is stale: make -C tests/refbind"
    model = jf.Model.build(jf.ModelConfig(**tiny_fixture.CONFIG), tiny_fixture.tensors())
    package = tmp_path / "fixture.jfm"
    model.write_package(str(package))
    model.close()
    jf.library()  # the engine library first, so the test binds to the loaded copy
    main = ctypes.CDLL(LIB).jfh_refbind_test_main
    main.argtypes = [ctypes.c_char_p]
    main.restype = ctypes.c_int
    rc = main(str(package).encode())
    out = capfd.readouterr().out
    assert rc == 0, out
    assert "refbind tests passed" in out


def test_reference_executor_serves_text_with_the_tokenizer(tmp_path, capfd):
    """The text path of the reference contract: tests/refbind's CAbiTokenizer
    (the reference's Tokenizer over the C ABI, in place of LlamaCppTokenizer)
    tokenizes a ChatML prompt for the executor on a two-layer model imported
    from a GGUF file with a byte-level BPE vocabulary; prompt ids, sampled
    tokens, pieces and end flags equal the tokenizer's and a direct session's."""
    if not os.path.exists(LIB):
        pytest.skip("tests/refbind/_ref/librefbind.so is built only where the reference checkout is present "
                    "(make -C tests/refbind)")
    newest = max(os.path.getmtime(p) for p in _inputs())
    assert os.path.getmtime(LIB) >= newest, "tests/refbind/_ref/librefbind.so is stale: make -C tests/refbind"
    pytest.importorskip("tokenizers")
    from tests.test_tokenizer import gguf_with_vocab, train_vocab
    hf = train_vocab()
    cfg = jf.ModelConfig(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=hf.get_vocab_size(), n_ctx=128)
    model = jf.Model.synthesize(cfg, seed=9)
    path = tmp_path / "vocab.gguf"
    gguf_with_vocab(model, hf, str(path))
    model.close()
    imported = jf.Model.open_gguf(str(path))
    package = tmp_path / "vocab.jfm"
    imported.write_package(str(package))
    imported.close()
    jf.library()
    main = ctypes.CDLL(LIB).jfh_refbind_text_main
    main.argtypes = [ctypes.c_char_p]
    main.restype = ctypes.c_int
    rc = main(str(package).encode())
    out = capfd.readouterr().out
    assert rc == 0, out
    assert "refbind text tests passed" in out
