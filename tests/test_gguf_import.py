"""GGUF -> JFM v2 import (jf_model_compile.cpp:549-645), on the CPU.

The GGUF file layout the test writes (header, then every tensor's payload at
data start + its recorded offset, offsets 32-byte aligned) is pinned by the
reference's frozen golden package: its metadata.gguf plus its tensors laid
out that way hash to the source SHA-256 its manifest records. Imports of
qwen2 files in that layout must then give back every tensor byte for byte,
the same segments as the package written from the in-memory model, and the
file's own SHA-256 as the manifest's source digest.
"""
from __future__ import annotations

import hashlib
import os
import struct

import pytest

import jetsonfabric_amd as jf

GGML_IDS = {jf.F32: 0, jf.F16: 1, jf.Q8_0: 8, jf.Q2_K: 10, jf.Q4_K: 12, jf.Q6_K: 14}


def tensor_infos(header: bytes):
    """(name, ggml type, offset) of a GGUF header's tensor infos, and the data start."""
    n_tensors, n_kv = struct.unpack_from("<QQ", header, 8)
    c = 24

    def string():
        nonlocal c
        (n,) = struct.unpack_from("<Q", header, c)
        c += 8 + n
        return header[c - n:c].decode()

    widths = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
    for _ in range(n_kv):
        string()
        (t,) = struct.unpack_from("<I", header, c)
        c += 4
        if t == 8:
            string()
        elif t == 9:
            et, n = struct.unpack_from("<IQ", header, c)
            c += 12
            for _ in range(n):
                if et == 8:
                    string()
                else:
                    c += widths[et]
        else:
            c += widths[t]
    infos = []
    for _ in range(n_tensors):
        name = string()
        (rank,) = struct.unpack_from("<I", header, c)
        c += 4 + 8 * rank
        ty, off = struct.unpack_from("<IQ", header, c)
        c += 12
        infos.append((name, ty, off, c - 12))
    return infos, (c + 31) // 32 * 32


def gguf_file(header: bytes, payload) -> bytearray:
    infos, start = tensor_infos(header)
    out = bytearray(header)
    for name, _, off, _ in infos:
        data = payload(name)
        end = start + off + len(data)
        if len(out) < end:
            out.extend(b"\0" * (end - len(out)))
        out[start + off:end] = data
    return out


def test_golden_source_digest_pins_the_layout(golden_package):
    with jf.Package(golden_package) as pkg:
        header = pkg.gguf_metadata()
        tensors = pkg.tensors()
        want = pkg.source_sha256()
    blob = gguf_file(header, lambda name: tensors[name][2])
    assert hashlib.sha256(bytes(blob)).digest() == want
    infos, _ = tensor_infos(header)
    # the reference's metadata carries GGML type ids (F32 = 0)
    assert {ty for _, ty, _, _ in infos} == {0}


CFG = jf.ModelConfig(n_layer=2, n_embd=256, n_ff=768, n_head=4, n_head_kv=2, n_vocab=1024, n_ctx=256)


def _model_and_file(tmp_path, **kw):
    model = jf.Model.synthesize(CFG, seed=3, **kw)
    pkg = tmp_path / "from_model"
    model.write_package(str(pkg))
    header = (pkg / "metadata.gguf").read_bytes()
    blob = gguf_file(header, model.tensor_bytes)
    path = tmp_path / "model.gguf"
    path.write_bytes(bytes(blob))
    return model, pkg, header, blob, path


@pytest.mark.parametrize("types", [(jf.Q4_K, jf.Q4_K, jf.Q6_K), (jf.Q2_K, jf.Q8_0, jf.Q6_K), (jf.Q8_0, jf.F16, jf.F32)])
def test_import_round_trip(tmp_path, types):
    linear, embd, out = types
    model, pkg, header, blob, path = _model_and_file(tmp_path, type_linear=linear, type_embd=embd, type_output=out,
                                                     output_bias=True)
    # the synthesized model's header records GGML ids for its JFM types
    infos, _ = tensor_infos(header)
    assert {ty for _, ty, _, _ in infos} <= set(GGML_IDS.values())
    with jf.Package(str(pkg)) as p:
        assert p.source_sha256() == hashlib.sha256(bytes(blob)).digest()

    imported = jf.Model.open_gguf(str(path))
    assert imported.config == model.config
    assert imported.tensor_names() == model.tensor_names()
    for name in model.tensor_names():
        a, b = model.tensor(name), imported.tensor(name)
        assert (a["type"], a["shape"], a["layer"]) == (b["type"], b["shape"], b["layer"]), name
        assert imported.tensor_bytes(name) == model.tensor_bytes(name), name
    assert imported.source_sha256() == hashlib.sha256(bytes(blob)).hexdigest()

    again = tmp_path / "from_gguf"
    imported.write_package(str(again))
    for name in sorted(os.listdir(pkg)):
        assert (again / name).read_bytes() == (pkg / name).read_bytes(), name
    with jf.Package(str(again)) as p:
        assert p.source_sha256() == hashlib.sha256(bytes(blob)).digest()
        assert p.stats()["layer_count"] == CFG.n_layer


def test_import_errors(tmp_path):
    model, _, header, blob, path = _model_and_file(tmp_path)
    bad = tmp_path / "bad.gguf"

    def rejects(data: bytes, match: str):
        bad.write_bytes(data)
        with pytest.raises(jf.JfhError, match=match):
            jf.Model.open_gguf(str(bad))

    rejects(b"GGML" + bytes(blob[4:]), "not GGUF")
    rejects(bytes(blob[:40]), "truncated")
    rejects(bytes(blob[:-1]), "exceeds the source GGUF")
    infos, _ = tensor_infos(header)
    name, _, _, at = next(i for i in infos if i[0].endswith("attn_q.weight"))
    patched = bytearray(blob)
    struct.pack_into("<I", patched, at, 2)  # GGML Q4_0
    rejects(bytes(patched), "unsupported GGUF tensor type for " + name)
    with pytest.raises(jf.JfhError):
        jf.Model.open_gguf(str(tmp_path / "missing.gguf"))
    # without output.weight (a tied model) there is no JFM v2 package
    key = struct.pack("<Q", 13) + b"output.weight"
    assert bytes(blob).count(key) == 1
    renamed = bytes(blob).replace(key, struct.pack("<Q", 13) + b"outpux.weight")
    rejects(renamed, "output.weight is required")
