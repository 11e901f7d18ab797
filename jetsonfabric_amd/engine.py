"""Python face of the HIP Qwen2 stage engine.

Mirrors the reference's native engine facade
(runtime/engines/native/include/jetsonfabric/native_inference.hpp:98-160):
``NativeEngine`` (load, ``logits``, ``forced_decode_logits``, ``generate``,
``create_session``) and ``NativeSession`` (``prefill_greedy``,
``decode_greedy``, ``rollback``), plus the draft verification and batched
steps the speculative decoder needs. Every call goes through libjfh.so.
"""
from __future__ import annotations

import ctypes
import os
import time
from dataclasses import dataclass, field
from typing import Callable, Iterable, Sequence

import numpy as np

from . import _capi
from ._capi import F16, F32, Q2_K, Q4_K, Q6_K, Q8_0, check, library

__all__ = [
    "F32", "F16", "Q8_0", "Q2_K", "Q4_K", "Q6_K",
    "ModelConfig", "Model", "NativeEngine", "NativeSession", "GenerationResult", "prompt_lookup_propose",
    "type_layout", "sha256",
]


@dataclass
class ModelConfig:
    """Qwen2 hyper-parameters (qwen2_metadata.hpp:10-18)."""

    n_layer: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    n_vocab: int
    n_ctx: int = 32768
    rope_base: float = 1.0e6
    rms_eps: float = 1.0e-6

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    def to_c(self) -> _capi.ModelParams:
        return _capi.ModelParams(self.n_layer, self.n_embd, self.n_ff, self.n_head, self.n_head_kv, self.n_ctx,
                                 self.n_vocab, self.head_dim, self.rope_base, self.rms_eps)

    @staticmethod
    def from_c(p: _capi.ModelParams) -> "ModelConfig":
        return ModelConfig(p.n_layer, p.n_embd, p.n_ff, p.n_head, p.n_head_kv, p.n_vocab, p.n_ctx, p.rope_base,
                           p.rms_eps)


def type_layout(type_id: int) -> tuple[int, int]:
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    check(library().jfh_tensor_type_layout(type_id, ctypes.byref(e), ctypes.byref(b)))
    return e.value, b.value


def activation_encode(values: np.ndarray, codec: str = "f16") -> bytes:
    """Wire bytes of f32 activations under an activation codec ("f32" or "f16";
    builtin_activation_codecs.cpp:112-209)."""
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    width = {"f32": 4, "f16": 2}.get(codec, 2)
    out = ctypes.create_string_buffer(v.size * width)
    check(library().jfh_activation_encode(codec.encode(), v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), v.size,
                                          out, v.size * width))
    return out.raw


def activation_decode(data: bytes, codec: str = "f16") -> np.ndarray:
    """f32 values of an activation codec's wire bytes."""
    width = {"f32": 4, "f16": 2}.get(codec, 2)
    n = len(data) // width
    out = np.zeros(n, dtype=np.float32)
    check(library().jfh_activation_decode(codec.encode(), data, len(data),
                                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n))
    return out


def sha256(data: bytes) -> bytes:
    out = (ctypes.c_uint8 * 32)()
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    check(library().jfh_sha256(buf, len(data), out))
    return bytes(out)


class Package:
    """A JFM v2 package opened for a layer range (jf_model_open, engine.h:106-150)."""

    def __init__(self, path: str, layer_start: int = 0, layer_end: int = 0xFFFFFFFF, verify_hashes: bool = True):
        h = ctypes.c_void_p()
        check(library().jfh_package_open(path.encode(), layer_start, layer_end, int(verify_hashes), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            library().jfh_package_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def stats(self) -> dict:
        s = _capi.PackageStats()
        check(library().jfh_package_get_stats(self._h, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in _capi.PackageStats._fields_ if f != "pad"}

    def tensors(self) -> dict:
        """name -> (type, shape, bytes), sorted by name."""
        lib = library()
        out = {}
        for i in range(lib.jfh_package_tensor_count(self._h)):
            v = _capi.TensorView()
            check(lib.jfh_package_tensor_at(self._h, i, ctypes.byref(v)))
            out[v.name.decode()] = (int(v.type), tuple(int(v.shape[d]) for d in range(v.rank)),
                                    ctypes.string_at(v.data, v.size))
        return out

    def gguf_metadata(self) -> bytes:
        data, size = ctypes.c_void_p(), ctypes.c_size_t()
        check(library().jfh_package_gguf_metadata(self._h, ctypes.byref(data), ctypes.byref(size)))
        return ctypes.string_at(data, size.value)

    def source_sha256(self) -> bytes:
        out = (ctypes.c_uint8 * 32)()
        check(library().jfh_package_source_sha256(self._h, out))
        return bytes(out)


class Model:
    """Host-resident model: a JFM v2 package, synthetic weights, or tensors added one by one."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def open(cls, package: str, layer_start: int = 0, layer_end: int = 0xFFFFFFFF, verify_hashes: bool = True) -> "Model":
        h = ctypes.c_void_p()
        check(library().jfh_model_open(package.encode(), layer_start, layer_end, int(verify_hashes), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def open_gguf(cls, path: str) -> "Model":
        """A qwen2 GGUF file as a model (jf_model_compile's input); write_package() then writes
        its JFM v2 package with the file's SHA-256 as the source digest."""
        h = ctypes.c_void_p()
        check(library().jfh_model_open_gguf(path.encode(), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def synthesize(cls, config: ModelConfig, type_linear: int = Q4_K, type_embd: int = Q4_K, type_output: int = Q6_K,
                   tied_output: bool = False, output_bias: bool = False, seed: int = 1234, stddev: float = 0.02,
                   threads: int = 0) -> "Model":
        spec = _capi.SynthSpec(config.to_c(), type_linear, type_embd, type_output, int(tied_output), int(output_bias),
                               0, seed, stddev, threads)
        h = ctypes.c_void_p()
        check(library().jfh_model_synthesize(ctypes.byref(spec), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def build(cls, config: ModelConfig, tensors: Iterable[tuple[str, int, Sequence[int], bytes]]) -> "Model":
        """tensors: (name, type, GGML shape ne0.., raw bytes)."""
        h = ctypes.c_void_p()
        lib = library()
        params = config.to_c()
        check(lib.jfh_model_create(ctypes.byref(params), ctypes.byref(h)))
        model = cls(h.value)
        for name, type_id, shape, data in tensors:
            dims = (ctypes.c_uint64 * 4)(*list(shape) + [1] * (4 - len(shape)))
            buf = ctypes.create_string_buffer(bytes(data), len(data))
            check(lib.jfh_model_add_tensor(model._h, name.encode(), type_id, len(shape), dims, buf, len(data)))
        check(lib.jfh_model_finalize(model._h))
        return model

    def slice(self, layer_start: int, layer_end: int) -> "Model":
        """Layers [layer_start, layer_end) as a model of their own: an engine over
        it is that pipeline stage (jf_model_open's layer range, engine.h:106-111)."""
        h = ctypes.c_void_p()
        check(library().jfh_model_slice(self._h, layer_start, layer_end, ctypes.byref(h)))
        return Model(h.value)

    def close(self) -> None:
        if self._h:
            library().jfh_model_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def config(self) -> ModelConfig:
        p = _capi.ModelParams()
        check(library().jfh_model_get_params(self._h, ctypes.byref(p)))
        return ModelConfig.from_c(p)

    def stats(self) -> dict:
        s = _capi.ModelStats()
        check(library().jfh_model_get_stats(self._h, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in _capi.ModelStats._fields_}

    def source_sha256(self) -> str:
        buf = (ctypes.c_char * 65)()
        check(library().jfh_model_source_sha256(self._h, buf))
        return buf.value.decode()

    def tensor_names(self) -> list[str]:
        lib = library()
        out = []
        for i in range(lib.jfh_model_tensor_count(self._h)):
            v = _capi.TensorView()
            check(lib.jfh_model_tensor_at(self._h, i, ctypes.byref(v)))
            out.append(v.name.decode())
        return out

    def tensor(self, name: str) -> dict:
        """View of a tensor: type, shape (ne0, ne1, ...), data pointer and a bytes copy accessor."""
        v = _capi.TensorView()
        check(library().jfh_model_find_tensor(self._h, name.encode(), ctypes.byref(v)))
        shape = tuple(int(v.shape[d]) for d in range(v.rank))
        return {"name": name, "type": int(v.type), "shape": shape, "layer": int(v.layer), "data": int(v.data),
                "size": int(v.size)}

    def tensor_bytes(self, name: str) -> bytes:
        t = self.tensor(name)
        return ctypes.string_at(t["data"], t["size"])

    def write_package(self, directory: str) -> None:
        check(library().jfh_model_write_package(self._h, directory.encode()))


@dataclass
class GenerationResult:
    """Result of a generation run (native_inference.hpp:88-96 plus speculation counters)."""

    sampled_tokens: list[int]
    time_to_first_token_ms: float = 0.0
    decode_ms: float = 0.0
    target_decode_passes: int = 0
    speculative_draft_tokens: int = 0
    speculative_accepted_tokens: int = 0
    finish_reason: str = "length"  # "stop": ended at an end-of-generation id
    inter_token_latency_ms: float = 0.0
    decode_tokens_per_second: float = 0.0
    end_to_end_tokens_per_second: float = 0.0
    # PrefillMetrics / ExecutionBufferMetrics (native_inference.hpp:71-85)
    prefill: dict = field(default_factory=dict)
    buffers: dict = field(default_factory=dict)
    extra: dict = field(default_factory=dict)

    @classmethod
    def from_stats(cls, tokens: list[int], st) -> "GenerationResult":
        return cls(
            sampled_tokens=tokens,
            time_to_first_token_ms=st.time_to_first_token_ms,
            decode_ms=st.decode_ms,
            target_decode_passes=int(st.target_decode_passes),
            speculative_draft_tokens=int(st.speculative_draft_tokens),
            speculative_accepted_tokens=int(st.speculative_accepted_tokens),
            finish_reason="stop" if st.stopped else "length",
            inter_token_latency_ms=st.inter_token_latency_ms,
            decode_tokens_per_second=st.decode_tokens_per_second,
            end_to_end_tokens_per_second=st.end_to_end_tokens_per_second,
            prefill={"plan_reused": bool(st.prefill_plan_reused),
                     "attention_matrix_cores": bool(st.prefill_attention_matrix_cores),
                     "planning_ms": st.prefill_planning_ms, "allocation_ms": st.prefill_allocation_ms,
                     "host_input_preparation_ms": st.prefill_host_input_ms, "compute_ms": st.prefill_compute_ms,
                     "output_read_ms": st.prefill_output_read_ms},
            buffers={"kv_cache_bytes": int(st.kv_cache_bytes), "prefill_scratch_bytes": int(st.prefill_scratch_bytes),
                     "decode_scratch_bytes": int(st.decode_scratch_bytes),
                     "prefill_host_input_bytes": int(st.prefill_host_input_bytes)},
        )


def _i32(values: Sequence[int]):
    arr = (ctypes.c_int32 * max(1, len(values)))(*values)
    return arr


class NativeSession:
    """One sequence: F16 KV cache on the device plus its position (native_inference.hpp:98-124)."""

    def __init__(self, engine: "NativeEngine", handle: int):
        self._engine = engine
        self._h = ctypes.c_void_p(handle)

    def close(self) -> None:
        if self._h:
            library().jfh_session_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def capacity(self) -> int:
        return int(library().jfh_session_capacity(self._h))

    def position(self) -> int:
        return int(library().jfh_session_position(self._h))

    def prefill_greedy(self, tokens: Sequence[int], logits: bool = False):
        out = ctypes.c_int32()
        buf = np.zeros(self._engine.vocab, dtype=np.float32) if logits else None
        ptr = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        check(library().jfh_session_prefill(self._h, _i32(tokens), len(tokens), ctypes.byref(out), ptr))
        return (out.value, buf) if logits else out.value

    def decode_greedy(self, token: int, logits: bool = False):
        out = ctypes.c_int32()
        buf = np.zeros(self._engine.vocab, dtype=np.float32) if logits else None
        ptr = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        check(library().jfh_session_decode(self._h, token, ctypes.byref(out), ptr))
        return (out.value, buf) if logits else out.value

    def verify(self, tokens: Sequence[int], logits: bool = False):
        """Decodes [previous, draft...] in one pass: greedy id after every row + accepted draft prefix."""
        n = len(tokens)
        out = (ctypes.c_int32 * n)()
        acc = ctypes.c_uint32()
        buf = np.zeros((n, self._engine.vocab), dtype=np.float32) if logits else None
        ptr = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        check(library().jfh_session_verify(self._h, _i32(tokens), n, out, ctypes.byref(acc), ptr))
        ids = [int(x) for x in out]
        return (ids, int(acc.value), buf) if logits else (ids, int(acc.value))

    def _stage_io(self, activations, n: int):
        e = self._engine
        f32 = ctypes.POINTER(ctypes.c_float)
        src = None
        if activations is not None:
            act = np.ascontiguousarray(activations, dtype=np.float32)
            if act.ndim != 2 or act.shape[1] != e._config.n_embd or act.shape[0] != n:
                raise ValueError(f"stage activations must be f32[{n}, {e._config.n_embd}]")
            src = act
        out = None if e.last_stage else np.zeros((n, e._config.n_embd), dtype=np.float32)
        return (src, src.ctypes.data_as(f32) if src is not None else None, out,
                out.ctypes.data_as(f32) if out is not None else None)

    def _stage_logits(self, logits: bool):
        if not logits:
            return None, None
        if not self._engine.last_stage:
            raise ValueError("only the last stage computes logits")
        buf = np.zeros(self._engine.vocab, dtype=np.float32)
        return buf, buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float))

    def prefill_stage(self, tokens: Sequence[int] | None = None, activations: np.ndarray | None = None,
                      logits: bool = False):
        """Pipeline-stage prefill (NativeSession::prefill_stage_tokens / _activations): token ids
        into the first stage, f32[n, n_embd] activations into later ones. Returns the greedy id of
        the last row on the last stage (with the row's logits when asked), else the stage's output
        activations f32[n, n_embd]."""
        n = len(tokens) if tokens is not None else (len(activations) if activations is not None else 0)
        src, src_p, out, out_p = self._stage_io(activations, n)
        lg, lg_p = self._stage_logits(logits)
        tok = ctypes.c_int32(-1)
        check(library().jfh_session_stage_prefill(self._h, _i32(tokens) if tokens is not None else None, src_p, n,
                                                  ctypes.byref(tok), out_p, lg_p))
        if out is not None:
            return out
        return (tok.value, lg) if logits else tok.value

    def decode_stage(self, token: int | None = None, activation: np.ndarray | None = None, logits: bool = False):
        """One pipeline-stage decode row (NativeSession::decode_stage_token / _activation)."""
        src, src_p, out, out_p = self._stage_io(activation, 1)
        lg, lg_p = self._stage_logits(logits)
        tok = ctypes.c_int32(-1)
        tin = ctypes.c_int32(token) if token is not None else None
        check(library().jfh_session_stage_decode(self._h, ctypes.byref(tin) if tin is not None else None, src_p,
                                                 ctypes.byref(tok), out_p, lg_p))
        if out is not None:
            return out
        return (tok.value, lg) if logits else tok.value

    def rollback(self, token_count: int) -> None:
        check(library().jfh_session_rollback(self._h, token_count))

    def read_kv(self, layer: int, n: int):
        """K and V cache rows [0, n) of one layer as f16 bits, [kv_head][n][head_dim]."""
        c = self._engine._config
        k = np.zeros((c.n_head_kv, n, c.head_dim), dtype=np.uint16)
        v = np.zeros_like(k)
        u16 = ctypes.POINTER(ctypes.c_uint16)
        check(library().jfh_session_read_kv(self._h, layer, n, k.ctypes.data_as(u16), v.ctypes.data_as(u16)))
        return k, v

    def import_kv(self, k: np.ndarray, v: np.ndarray) -> None:
        """Writes cache rows [0, n) of every layer ([layer][kv_head][n][head_dim] f16 bits); the
        session then stands at position n as after a prefill of n tokens."""
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        if k.shape != v.shape or k.ndim != 4:
            raise ValueError("k and v must be [layer][kv_head][n][head_dim]")
        u16 = ctypes.POINTER(ctypes.c_uint16)
        check(library().jfh_session_import_kv(self._h, k.shape[2], k.ctypes.data_as(u16), v.ctypes.data_as(u16)))

    def time_steps(self, tokens: Sequence[int], iterations: int, warmup: int = 2, all_logits: bool | None = None) -> float:
        """Mean device ms per step of `tokens` at the current position (rolled back after each step)."""
        ms = ctypes.c_double()
        if all_logits is None:
            all_logits = len(tokens) > 1
        check(library().jfh_session_time_steps(self._h, _i32(tokens), len(tokens), int(all_logits), warmup,
                                               iterations, ctypes.byref(ms)))
        return ms.value

    def profile_step(self, tokens: Sequence[int], iterations: int = 3, all_logits: bool | None = None) -> list[dict]:
        """Per-kernel device time and algorithmic bytes of one step (HIP events per launch)."""
        if all_logits is None:
            all_logits = len(tokens) > 1
        cap = 64
        out = (_capi.KernelStat * cap)()
        count = ctypes.c_uint32()
        check(library().jfh_session_profile_step(self._h, _i32(tokens), len(tokens), int(all_logits), iterations, out,
                                                 cap, ctypes.byref(count)))
        return [{"kernel": out[i].label.decode(), "launches": out[i].launches, "ms": out[i].total_ms,
                 "bytes": out[i].bytes} for i in range(count.value)]


class NativeEngine:
    """Device-resident Qwen2 weights and the step kernels (native_inference.hpp:126-160)."""

    def __init__(self, model: Model, device: int = 0, use_graphs: bool | None = None):
        if use_graphs is None:
            # JFH_USE_GRAPHS=0 launches every kernel directly instead of replaying captured step graphs
            use_graphs = os.environ.get("JFH_USE_GRAPHS", "1") != "0"
        opts = _capi.EngineOptions(device, int(use_graphs))
        h = ctypes.c_void_p()
        start = time.perf_counter()
        check(library().jfh_engine_create(model.handle, ctypes.byref(opts), ctypes.byref(h)))
        self.load_time_ms = (time.perf_counter() - start) * 1e3
        self._h = h
        self._config = model.config
        self.vocab = self._config.n_vocab
        info = _capi.EngineInfo()
        check(library().jfh_engine_get_info(self._h, ctypes.byref(info)))
        self.weight_bytes = int(info.weight_bytes)
        self.prefill_chunk = int(info.prefill_chunk)
        self.device_name = info.device_name.decode()
        # resident layer range of a pipeline stage (the whole model by default)
        self.layer_start = int(info.layer_start)
        self.layer_end = int(info.layer_end)
        self.first_stage = self.layer_start == 0
        self.last_stage = self.layer_end == self._config.n_layer

    def close(self) -> None:
        if self._h:
            library().jfh_engine_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def model_info(self) -> ModelConfig:
        return self._config

    def set_end_tokens(self, ids: Sequence[int]) -> None:
        """End-of-generation ids (Tokenizer::is_end_token, tokenization/tokenizer.hpp:16): the
        on-GPU acceptance stops at them (generation_runner.cpp:512-517) and generation ends at
        one. At most 16; an empty list clears the set."""
        ids = list(ids)
        check(library().jfh_engine_set_end_tokens(self._h, _i32(ids), len(ids)))

    def create_session(self, capacity: int) -> NativeSession:
        h = ctypes.c_void_p()
        check(library().jfh_session_create(self._h, capacity, ctypes.byref(h)))
        return NativeSession(self, h.value)

    def step_batch(self, sessions: Sequence[NativeSession], token_rows: Sequence[Sequence[int]],
                   logits: bool = False):
        """One pass over several sessions; returns (ids per session, accepted per session) and,
        when asked, the logits rows of each session ([rows, vocab] per session)."""
        count = len(sessions)
        handles = (ctypes.c_void_p * count)(*[s.handle.value for s in sessions])
        flat = [t for row in token_rows for t in row]
        lengths = (ctypes.c_uint32 * count)(*[len(r) for r in token_rows])
        out = (ctypes.c_int32 * len(flat))()
        acc = (ctypes.c_uint32 * count)()
        buf = np.zeros((len(flat), self.vocab), dtype=np.float32) if logits else None
        ptr = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if logits else None
        check(library().jfh_engine_step_batch(self._h, handles, count, _i32(flat), lengths, out, acc, ptr))
        ids, rows, o = [], [], 0
        for row in token_rows:
            ids.append([int(x) for x in out[o:o + len(row)]])
            if logits:
                rows.append(buf[o:o + len(row)])
            o += len(row)
        return (ids, [int(a) for a in acc], rows) if logits else (ids, [int(a) for a in acc])

    def stage_step_batch(self, sessions: Sequence[NativeSession], tokens: Sequence[Sequence[int]] | None = None,
                         activations: Sequence[np.ndarray] | None = None, logits: bool = False):
        """Several sessions' rows through this pipeline stage in one pass (jfh_engine_stage_step_batch):
        token ids per session into the first stage, f32 [rows, n_embd] activations into later ones.
        The last stage returns every row's greedy id per session (and, when asked, [rows, vocab]
        logits per session); the others return every row's output activations per session."""
        count = len(sessions)
        handles = (ctypes.c_void_p * count)(*[s.handle.value for s in sessions])
        rows = [len(t) for t in tokens] if tokens is not None else [len(a) for a in activations]
        total = sum(rows)
        lengths = (ctypes.c_uint32 * count)(*rows)
        f32p = ctypes.POINTER(ctypes.c_float)
        toks = _i32([t for row in tokens for t in row]) if tokens is not None else None
        acts = None
        if activations is not None:
            acts = np.ascontiguousarray(np.concatenate([np.asarray(a, dtype=np.float32) for a in activations]))
        out_ids = (ctypes.c_int32 * total)() if self.last_stage else None
        out_act = None if self.last_stage else np.zeros((total, self._config.n_embd), dtype=np.float32)
        lg = np.zeros((total, self.vocab), dtype=np.float32) if logits and self.last_stage else None
        check(library().jfh_engine_stage_step_batch(
            self._h, handles, count, toks, acts.ctypes.data_as(f32p) if acts is not None else None, lengths, out_ids,
            out_act.ctypes.data_as(f32p) if out_act is not None else None, lg.ctypes.data_as(f32p) if lg is not None else None))
        split = np.cumsum([0] + rows)
        if not self.last_stage:
            return [out_act[split[i]:split[i + 1]] for i in range(count)]
        ids = [[int(out_ids[j]) for j in range(split[i], split[i + 1])] for i in range(count)]
        if logits:
            return ids, [lg[split[i]:split[i + 1]] for i in range(count)]
        return ids

    def profile_batch(self, sessions: Sequence[NativeSession], token_rows: Sequence[Sequence[int]],
                      iterations: int = 3, all_logits: bool = False) -> list[dict]:
        """Per-kernel device time and algorithmic bytes of one batched step (as step_batch) over
        several sessions, rolled back after every iteration."""
        count = len(sessions)
        handles = (ctypes.c_void_p * count)(*[s.handle.value for s in sessions])
        flat = [t for row in token_rows for t in row]
        lengths = (ctypes.c_uint32 * count)(*[len(r) for r in token_rows])
        cap = 64
        out = (_capi.KernelStat * cap)()
        n = ctypes.c_uint32()
        check(library().jfh_engine_profile_batch(self._h, handles, count, _i32(flat), lengths, int(all_logits),
                                                 iterations, out, cap, ctypes.byref(n)))
        return [{"kernel": out[i].label.decode(), "launches": out[i].launches, "ms": out[i].total_ms,
                 "bytes": out[i].bytes} for i in range(n.value)]

    def logits(self, tokens: Sequence[int]) -> np.ndarray:
        """Last-row logits of a fresh prefill (NativeEngine::logits, native_inference.cpp:396-411)."""
        s = self.create_session(len(tokens))
        try:
            _, out = s.prefill_greedy(tokens, logits=True)
            return out
        finally:
            s.close()

    def forced_decode_logits(self, prompt: Sequence[int], forced: Sequence[int]) -> list[np.ndarray]:
        """Prefill logits, then one decode per forced token (native_inference.cpp:413-441)."""
        s = self.create_session(len(prompt) + len(forced))
        try:
            trace = [s.prefill_greedy(prompt, logits=True)[1]]
            for t in forced:
                trace.append(s.decode_greedy(t, logits=True)[1])
            return trace
        finally:
            s.close()

    def dequantize_rows(self, tensor: str, row0: int, n_rows: int, cols: int) -> np.ndarray:
        out = np.zeros((n_rows, cols), dtype=np.float32)
        check(library().jfh_engine_dequantize(self._h, tensor.encode(), row0, n_rows,
                                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def matmul(self, tensor: str, x: np.ndarray, rows: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        y = np.zeros((x.shape[0], rows), dtype=np.float32)
        check(library().jfh_engine_matmul(self._h, tensor.encode(), x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                          x.shape[0], y.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return y

    def generate(self, prompt: Sequence[int], max_tokens: int, draft_max: int = 0, max_ngram: int = 4,
                 min_ngram: int = 2) -> GenerationResult:
        """GenerationRunner loop over the HIP stage executor (generation_runner.cpp:398-566)."""
        out = (ctypes.c_int32 * max_tokens)()
        count = ctypes.c_uint32()
        stats = _capi.GenerationStats()
        check(library().jfh_generate(self._h, _i32(prompt), len(prompt), max_tokens, draft_max, max_ngram, min_ngram,
                                     out, ctypes.byref(count), ctypes.byref(stats)))
        return GenerationResult.from_stats([int(x) for x in out[:count.value]], stats)

    def generate_with_draft(self, prompt: Sequence[int], max_tokens: int, draft_max: int,
                            propose: Callable[[list[int], int], Sequence[int]]) -> GenerationResult:
        """The same runner with a caller's draft strategy (jfh_generate_draft):
        propose(history, max_tokens) returns the draft for the history."""
        def thunk(_user, history, n, limit, out_ptr):
            try:
                draft = list(propose([history[i] for i in range(n)], int(limit)))[:limit]
            except Exception:  # a failing strategy proposes nothing
                return 0
            for i, t in enumerate(draft):
                out_ptr[i] = int(t)
            return len(draft)

        fn = _capi.DraftProposeFn(thunk)
        out = (ctypes.c_int32 * max_tokens)()
        count = ctypes.c_uint32()
        stats = _capi.GenerationStats()
        check(library().jfh_generate_draft(self._h, _i32(prompt), len(prompt), max_tokens, draft_max, fn, None, out,
                                           ctypes.byref(count), ctypes.byref(stats)))
        return GenerationResult.from_stats([int(x) for x in out[:count.value]], stats)


    def generate_concurrent(self, prompts: Sequence[Sequence[int]], max_tokens: int, draft_max: int = 0,
                            max_ngram: int = 4, min_ngram: int = 2, batch_wait_us: int = 500):
        """Concurrent GenerationRunner loops over a continuous-batching executor
        (continuous_batching_executor.cpp:14-200); returns (results per prompt,
        decode wall ms from the common decode start to the last runner's last token)."""
        n = len(prompts)
        flat = [t for p in prompts for t in p]
        lengths = (ctypes.c_uint32 * n)(*[len(p) for p in prompts])
        out = (ctypes.c_int32 * (n * max_tokens))()
        counts = (ctypes.c_uint32 * n)()
        stats = (_capi.GenerationStats * n)()
        wall = ctypes.c_double()
        check(library().jfh_generate_concurrent(self._h, n, _i32(flat), lengths, max_tokens, draft_max, max_ngram,
                                                min_ngram, batch_wait_us, out, counts, stats, ctypes.byref(wall)))
        results = []
        for i in range(n):
            results.append(GenerationResult.from_stats(
                [int(x) for x in out[i * max_tokens:i * max_tokens + counts[i]]], stats[i]))
        return results, wall.value


class Tokenizer:
    """Byte-level BPE tokenizer of a Qwen2 GGUF vocabulary (LlamaCppTokenizer,
    runtime/adapters/llama_cpp_tokenizer.cpp:50-137) from a package directory's
    metadata.gguf or a GGUF file."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(library().jfh_tokenizer_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h
        n = ctypes.c_uint32()
        check(library().jfh_tokenizer_vocab_size(self._h, ctypes.byref(n)))
        self.vocab_size = int(n.value)

    def close(self) -> None:
        if self._h:
            library().jfh_tokenizer_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tokenize(self, text: str | bytes) -> list[int]:
        """Tokenizer::tokenize (tokenization/tokenizer.hpp:14): special tokens parsed, BOS/EOS as
        the metadata asks; raises InvalidArgument when nothing results."""
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        n = ctypes.c_uint32()
        cap = 3 * len(data) + 8  # an invalid UTF-8 byte becomes U+FFFD: three byte tokens
        out = (ctypes.c_int32 * cap)()
        check(library().jfh_tokenizer_tokenize(self._h, data, len(data), out, cap, ctypes.byref(n)))
        return [int(out[i]) for i in range(n.value)]

    def token_piece(self, token: int) -> bytes:
        """Tokenizer::token_piece (tokenizer.hpp:15): the token's bytes."""
        n = ctypes.c_uint32()
        status = library().jfh_tokenizer_token_piece(self._h, int(token), None, 0, ctypes.byref(n))
        if status.code != 0 and n.value == 0:
            check(status)
        buf = ctypes.create_string_buffer(max(1, n.value))
        check(library().jfh_tokenizer_token_piece(self._h, int(token), buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value]

    def is_end_token(self, token: int) -> bool:
        """Tokenizer::is_end_token (tokenizer.hpp:16)."""
        out = ctypes.c_uint32()
        check(library().jfh_tokenizer_is_end_token(self._h, int(token), ctypes.byref(out)))
        return bool(out.value)

    def end_tokens(self) -> list[int]:
        n = ctypes.c_uint32()
        out = (ctypes.c_int32 * 64)()
        check(library().jfh_tokenizer_end_tokens(self._h, out, 64, ctypes.byref(n)))
        return [int(out[i]) for i in range(n.value)]

    def detokenize(self, tokens: Iterable[int]) -> bytes:
        return b"".join(self.token_piece(t) for t in tokens)


def prompt_lookup_propose(history: Sequence[int], max_tokens: int, max_ngram: int = 4, min_ngram: int = 2) -> list[int]:
    """PromptLookupDraft::propose through the C ABI (prompt_lookup_draft.cpp:15-44)."""
    hist = (ctypes.c_uint32 * max(1, len(history)))(*history)
    out = (ctypes.c_uint32 * max(1, max_tokens))()
    n = ctypes.c_uint32()
    check(library().jfh_prompt_lookup_propose(hist, len(history), max_ngram, min_ngram, max_tokens, out,
                                              ctypes.byref(n)))
    return [int(x) for x in out[:n.value]]
