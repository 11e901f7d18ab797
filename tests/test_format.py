"""JFM v2 package reading/writing and the host model (CPU only).

Pinned against the reference's frozen golden package
(runtime/engines/native/tests/fixtures/jfm-v2-golden, asserted counts in
runtime/engines/native/tests/engine_test.cpp:95-113 and residency figures
247-317), its SHA-256 known answer (444-455), its rejection cases (319-442)
and, where oracle/_ref is built, the reference loader itself
(runtime/engines/native/src/engine.c) reading the same files.
"""
from __future__ import annotations

import os
import shutil
import struct

import pytest

import jetsonfabric_amd as jf
import oracle as jo

ALL = 0xFFFFFFFF


def test_sha256_known_answer():
    expected = bytes.fromhex("ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad")
    assert jf.sha256(b"abc") == expected
    assert jf.sha256(b"") == bytes.fromhex("e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855")
    import hashlib

    blob = bytes(range(256)) * 300
    assert jf.sha256(blob) == hashlib.sha256(blob).digest()


def test_type_layout_table():
    for t, layout in {jf.F32: (1, 4), jf.F16: (1, 2), jf.Q8_0: (32, 34), jf.Q2_K: (256, 84), jf.Q4_K: (256, 144),
                      jf.Q6_K: (256, 210)}.items():
        assert jf.type_layout(t) == layout
    with pytest.raises(jf.JfhError) as e:
        jf.type_layout(12345)
    assert e.value.code == 3  # format error, as jf_tensor_type_layout (engine.c:305-307)


@pytest.mark.skipif(not jo.ref_loader.available(), reason="reference loader not built (oracle/_ref)")
def test_type_layout_table_equals_reference_for_every_id():
    for t in range(0, 64):
        ref = jo.ref_loader.type_layout(t)
        if ref is None:
            with pytest.raises(jf.JfhError):
                jf.type_layout(t)
        else:
            assert jf.type_layout(t) == ref, t


def test_golden_package_stage_selection(golden_package):
    # engine_test.cpp:107-112: first stage 3 tensors, last stage 4
    with jf.Package(golden_package, 0, 1) as p:
        assert p.stats()["selected_tensor_count"] == 3
    with jf.Package(golden_package, 1, 2) as p:
        assert p.stats()["selected_tensor_count"] == 4
    with jf.Package(golden_package, 0, ALL) as p:
        s = p.stats()
        assert s["layer_end"] == 2 and s["layer_count"] == 2
        assert s["selected_tensor_count"] == s["total_tensor_count"]
        names = list(p.tensors())
        assert names == sorted(names)
        assert p.gguf_metadata()[:4] == b"GGUF"


@pytest.mark.skipif(not jo.ref_loader.available(), reason="reference loader not built (oracle/_ref)")
@pytest.mark.parametrize("rng", [(0, 1), (1, 2), (0, 2), (0, ALL)])
def test_golden_package_agrees_with_reference_loader(golden_package, rng):
    code, msg, ref_stats, ref_tensors = jo.ref_loader.open(golden_package, *rng)
    assert code == 0, msg
    with jf.Package(golden_package, *rng) as p:
        s = p.stats()
        for key in ("layer_start", "layer_end", "layer_count", "selected_weight_bytes", "total_weight_bytes",
                    "selected_tensor_count", "total_tensor_count"):
            assert s[key] == ref_stats[key], key
        assert p.tensors() == ref_tensors


def test_empty_layer_range_is_rejected(golden_package):
    with pytest.raises(jf.InvalidArgument):
        jf.Package(golden_package, 1, 1)


def test_corrupted_segment_fails_hash_verification(golden_package, tmp_path):
    bad = tmp_path / "bad"
    shutil.copytree(golden_package, bad)
    seg = bad / "layer-00000.jfs"
    data = bytearray(seg.read_bytes())
    data[-1] ^= 0xFF
    seg.write_bytes(bytes(data))
    with pytest.raises(jf.JfhError) as e:
        jf.Package(str(bad), 0, 1, verify_hashes=True)
    assert e.value.code == 3  # format error
    with jf.Package(str(bad), 0, 1, verify_hashes=False):
        pass
    if jo.ref_loader.available():
        assert jo.ref_loader.open(str(bad), 0, 1, True)[0] == 3


def test_manifest_reserved_field_and_missing_files(golden_package, tmp_path):
    bad = tmp_path / "reserved"
    shutil.copytree(golden_package, bad)
    man = bad / "manifest.jfm"
    data = bytearray(man.read_bytes())
    data[60:64] = struct.pack("<I", 1)  # engine_test.cpp:411-414
    man.write_bytes(bytes(data))
    with pytest.raises(jf.JfhError) as e:
        jf.Package(str(bad))
    assert e.value.code == 3
    missing = tmp_path / "missing"
    shutil.copytree(golden_package, missing)
    os.remove(missing / "output.jfs")
    with pytest.raises(jf.JfhError):
        jf.Package(str(missing), 1, 2)


def _small_model(seed=4, tied=False):
    cfg = jf.ModelConfig(n_layer=3, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=320, n_ctx=128)
    embd = jf.Q8_0 if tied else jf.Q4_K
    return jf.Model.synthesize(cfg, type_linear=jf.Q4_K, type_embd=embd, type_output=jf.Q8_0 if tied else jf.Q6_K,
                               tied_output=tied, seed=seed)


def test_synthesis_is_deterministic_and_seeded():
    a, b, c = _small_model(4), _small_model(4), _small_model(5)
    name = "blk.1.ffn_down.weight"
    assert a.tensor_bytes(name) == b.tensor_bytes(name)
    assert a.tensor_bytes(name) != c.tensor_bytes(name)
    assert a.tensor_bytes("blk.0.attn_q.weight") != a.tensor_bytes("blk.1.attn_q.weight")
    assert a.tensor("blk.0.ffn_up.weight")["shape"] == (256, 512)
    assert a.tensor("blk.0.ffn_down.weight")["shape"] == (512, 256)


def test_tied_output_is_a_byte_copy_of_the_embedding():
    m = _small_model(tied=True)
    assert m.tensor_bytes("output.weight") == m.tensor_bytes("token_embd.weight")


@pytest.mark.parametrize("tied", [False, True])
def test_write_package_round_trip(tmp_path, tied):
    m = _small_model(tied=tied)
    out = tmp_path / "model.jfm"
    m.write_package(str(out))
    names = m.tensor_names()
    with jf.Package(str(out)) as p:
        tensors = p.tensors()
        assert sorted(tensors) == sorted(names)
        for n in names:
            assert tensors[n][2] == m.tensor_bytes(n), n
    back = jf.Model.open(str(out))
    assert back.config == m.config
    assert back.source_sha256() == m.source_sha256()
    if jo.ref_loader.available():
        code, msg, stats, ref_tensors = jo.ref_loader.open(str(out), 0, ALL)
        assert code == 0, msg
        assert stats["total_tensor_count"] == len(names)
        for n in names:
            assert ref_tensors[n][2] == m.tensor_bytes(n), n
        # stage selection: layers [1, 2) carry only that layer's tensors
        code, msg, stats, ref_tensors = jo.ref_loader.open(str(out), 1, 2)
        assert code == 0 and all(n.startswith("blk.1.") or n.startswith("output") for n in ref_tensors)


def test_model_validation_rejects_missing_and_misshapen_tensors():
    cfg = jf.ModelConfig(n_layer=1, n_embd=4, n_ff=8, n_head=1, n_head_kv=1, n_vocab=8, n_ctx=16)
    from tests.golden import tiny_fixture

    tensors = [t for t in tiny_fixture.tensors() if not t[0].startswith("blk.1.")]
    jf.Model.build(cfg, tensors)  # one layer of the fixture is complete
    with pytest.raises(jf.JfhError):
        jf.Model.build(cfg, [t for t in tensors if t[0] != "output.weight"])  # qwen2_architecture.cpp:96-101
    with pytest.raises(jf.JfhError):
        jf.Model.build(cfg, [t for t in tensors if t[0] != "blk.0.attn_q.bias"])  # biases are required
    bad = [(n, ty, (8, 4) if n == "blk.0.attn_q.weight" else s, b) for n, ty, s, b in tensors]
    with pytest.raises(jf.JfhError):
        jf.Model.build(cfg, bad)


def test_stage_model_stats_count_the_whole_model(tmp_path):
    """A model opened or sliced for a layer range reports its own weights as
    selected and the whole model's as total (jf_model_stats, engine.h:74-83)."""
    cfg = jf.ModelConfig(n_layer=4, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=512, n_ctx=64)
    whole = jf.Model.synthesize(cfg, seed=5)
    whole.write_package(str(tmp_path / "m.jfm"))
    total = whole.stats()["total_weight_bytes"]
    assert total == whole.stats()["selected_weight_bytes"]
    parts = []
    for a, b in ((0, 2), (2, 4)):
        for stage in (jf.Model.open(str(tmp_path / "m.jfm"), a, b), whole.slice(a, b)):
            s = stage.stats()
            assert s["total_weight_bytes"] == total and s["selected_weight_bytes"] < total
            assert s["total_tensor_count"] == whole.stats()["total_tensor_count"]
            parts.append(s["selected_weight_bytes"])
            stage.close()
    assert parts[0] + parts[2] == total and parts[1] + parts[3] == total
    whole.close()
