"""Python side of the CPU oracle -- TEST INFRASTRUCTURE ONLY (the checker).

* ctypes binding of oracle/libjfo.so (C restatement of the Qwen2 forward and
  the GGML block formats, see jfo.h for the reference lines it follows);
* pure-Python restatements of the integer host logic on the speculative path:
  prompt-lookup drafting (runtime/speculative/prompt_lookup_draft.cpp:15-44)
  and the greedy acceptance / rollback loop
  (runtime/pipeline_parallel/generation_runner.cpp:469-556);
* a binding of the reference's own JFM v2 loader built from its sources into
  oracle/_ref/libjfref.so (runtime/engines/native/src/engine.c), when present.

Parity status per function is recorded in oracle/README.md.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char, c_char_p, c_double, c_float, c_int16, c_int32, c_int64, c_int8, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p
from typing import Callable, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjfo.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libjfref.so")

F32, F16, Q8_0, Q2_K, Q4_K, Q6_K = 1, 2, 7, 9, 11, 13
MODE_EXACT, MODE_Q8 = 0, 1

__all__ = [
    "F32", "F16", "Q8_0", "Q2_K", "Q4_K", "Q6_K", "MODE_EXACT", "MODE_Q8", "act_block", "lib", "block", "row_bytes",
    "f16_to_f32", "f32_to_f16", "dequantize_row", "quantize_act", "quantize_act_normed", "vec_dot_q8", "vec_dot_f32", "matmul",
    "rope_table", "argmax", "OracleModel", "OracleSession", "prompt_lookup", "speculative_generate",
    "ref_loader", "nrmse", "cosine", "use_library", "build_native",
]


class _Tensor(ctypes.Structure):
    _fields_ = [("type", c_int32), ("pad", c_int32), ("ne0", c_int64), ("ne1", c_int64), ("data", c_void_p)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, _Tensor) for n in ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ffn_norm", "w_gate",
                                       "w_up", "w_down")]


class _Model(ctypes.Structure):
    _fields_ = [
        ("n_layer", c_int32), ("n_embd", c_int32), ("n_ff", c_int32), ("n_head", c_int32), ("n_head_kv", c_int32),
        ("n_ctx", c_int32), ("n_vocab", c_int32), ("pad", c_int32), ("rope_base", c_float), ("rms_eps", c_float),
        ("tok_embd", _Tensor), ("output_norm", _Tensor), ("output", _Tensor), ("output_bias", _Tensor),
        ("layers", POINTER(_Layer)),
    ]


_SIGS = {
    "jfo_f16_to_f32": (c_float, [c_uint16]),
    "jfo_f32_to_f16": (c_uint16, [c_float]),
    "jfo_type_block": (c_int32, [c_int32, POINTER(c_uint32), POINTER(c_uint32)]),
    "jfo_dequantize_row": (c_int32, [c_int32, c_void_p, POINTER(c_float), c_int64]),
    "jfo_quantize_act": (None, [POINTER(c_float), c_int64, POINTER(c_int8), POINTER(c_float), POINTER(c_int16)]),
    "jfo_quantize_act_normed": (None, [POINTER(c_float), POINTER(c_float), c_int64, c_float, POINTER(c_int8),
                                       POINTER(c_float), POINTER(c_int16)]),
    "jfo_vec_dot_q8": (c_double, [c_int32, c_void_p, POINTER(c_int8), POINTER(c_float), POINTER(c_int16), c_int64]),
    "jfo_act_block": (c_int32, [c_int32]),
    "jfo_quantize_act_blk": (None, [POINTER(c_float), c_int64, c_int32, POINTER(c_int8), POINTER(c_float),
                                    POINTER(c_int16)]),
    "jfo_quantize_act_normed_blk": (None, [POINTER(c_float), POINTER(c_float), c_int64, c_float, c_int32,
                                           POINTER(c_int8), POINTER(c_float), POINTER(c_int16)]),
    "jfo_vec_dot_q8_blk": (c_double, [c_int32, c_void_p, POINTER(c_int8), POINTER(c_float), POINTER(c_int16), c_int64,
                                      c_int32]),
    "jfo_vec_dot_f32": (c_double, [c_int32, c_void_p, POINTER(c_float), c_int64]),
    "jfo_matmul": (c_int32, [c_int32, c_void_p, c_int64, c_int64, POINTER(c_float), c_int64, POINTER(c_float), c_int32,
                             c_int32]),
    "jfo_session_create": (c_void_p, [POINTER(_Model), c_int32, c_int32, c_int32]),
    "jfo_session_destroy": (None, [c_void_p]),
    "jfo_session_position": (c_int32, [c_void_p]),
    "jfo_session_forward": (c_int32, [c_void_p, POINTER(c_int32), c_int32, c_int32, POINTER(c_float), POINTER(c_int32)]),
    "jfo_session_forward_range": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_float), c_int32, c_int32, c_int32,
                                            POINTER(c_float), c_int32, POINTER(c_float), POINTER(c_int32)]),
    "jfo_session_rollback": (c_int32, [c_void_p, c_int32]),
    "jfo_session_fill_kv": (c_int32, [c_void_p, c_int32, c_uint64]),
    "jfo_session_read_kv": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_uint16), POINTER(c_uint16)]),
    "jfo_session_write_kv": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_uint16), POINTER(c_uint16)]),
    "jfo_rope_table": (None, [c_float, c_int32, c_int32, c_int32, POINTER(c_float)]),
    "jfo_argmax": (c_int32, [POINTER(c_float), c_int64]),
}

_lib = None


def use_library(path: str) -> None:
    """Load the oracle from another build of the same sources (e.g. one tuned
    with -march=native for timing) instead of libjfo.so. Only before the
    first call into the oracle: handles from one build mean nothing to another."""
    global LIB_PATH
    if _lib is not None and os.path.abspath(path) != os.path.abspath(LIB_PATH):
        raise RuntimeError("the oracle library is already loaded")
    LIB_PATH = path


def build_native(out_dir: str) -> str:
    """Build the oracle for this host's CPU (make -C oracle native) into out_dir."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, "native", f"OUT={os.path.abspath(out_dir)}"], check=True,
                   stdout=subprocess.DEVNULL)
    return os.path.join(out_dir, "libjfo_native.so")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `make -C oracle`")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(POINTER(c_float))


def block(type_id: int) -> tuple[int, int]:
    e, b = c_uint32(), c_uint32()
    if not lib().jfo_type_block(type_id, ctypes.byref(e), ctypes.byref(b)):
        raise ValueError(f"unsupported type {type_id}")
    return e.value, b.value


def row_bytes(type_id: int, n: int) -> int:
    e, b = block(type_id)
    return n // e * b


def f16_to_f32(h: int) -> float:
    return lib().jfo_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().jfo_f32_to_f16(f)


def dequantize_row(type_id: int, data: bytes, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    if lib().jfo_dequantize_row(type_id, buf, _fp(out), n) != 0:
        raise ValueError("dequantization failed")
    return out


def act_block(type_id: int) -> int:
    """Activation block of a quantized matmul input: 32 for Q8_0 weights, else 256."""
    return int(lib().jfo_act_block(type_id))


def quantize_act(x: np.ndarray, blk: int = 256):
    """Codes, scales (one per blk values) and 16-value code sums of x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    q = np.zeros(n, dtype=np.int8)
    d = np.zeros(n // blk, dtype=np.float32)
    s = np.zeros(n // 16, dtype=np.int16)
    lib().jfo_quantize_act_blk(_fp(x), n, blk, q.ctypes.data_as(POINTER(c_int8)), _fp(d),
                               s.ctypes.data_as(POINTER(c_int16)))
    return q, d, s


def quantize_act_normed(x: np.ndarray, gain: np.ndarray, eps: float, blk: int = 256):
    """Codes, block scales and 16-value sums of RMSNorm(x) * gain as the engine stages them."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gain, dtype=np.float32)
    n = x.size
    q = np.zeros(n, dtype=np.int8)
    d = np.zeros(n // blk, dtype=np.float32)
    s = np.zeros(n // 16, dtype=np.int16)
    lib().jfo_quantize_act_normed_blk(_fp(x), _fp(g), n, eps, blk, q.ctypes.data_as(POINTER(c_int8)), _fp(d),
                                      s.ctypes.data_as(POINTER(c_int16)))
    return q, d, s


def vec_dot_q8(type_id: int, row: bytes, q: np.ndarray, d: np.ndarray, s: np.ndarray, blk: int | None = None) -> float:
    """Dot of one encoded weight row with quantized activations (blocks of blk
    values; default: the weight type's rule, act_block(type_id))."""
    buf = ctypes.create_string_buffer(bytes(row), len(row))
    b = act_block(type_id) if blk is None else blk
    return lib().jfo_vec_dot_q8_blk(type_id, buf, q.ctypes.data_as(POINTER(c_int8)), _fp(d),
                                    s.ctypes.data_as(POINTER(c_int16)), q.size, b)


def vec_dot_f32(type_id: int, row: bytes, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    buf = ctypes.create_string_buffer(bytes(row), len(row))
    return lib().jfo_vec_dot_f32(type_id, buf, _fp(x), x.size)


def matmul(type_id: int, w: bytes | int, n: int, rows: int, x: np.ndarray, mode: int = MODE_Q8, threads: int = 8):
    """y[t, r] = W[r] . x[t]; w may be bytes or a raw address. MODE_Q8 quantizes
    the rows by the weight type's block rule (act_block)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    y = np.zeros((x.shape[0], rows), dtype=np.float32)
    keep = None
    if isinstance(w, (bytes, bytearray)):
        keep = ctypes.create_string_buffer(bytes(w), len(w))
        ptr = ctypes.cast(keep, c_void_p)
    else:
        ptr = c_void_p(w)
    if lib().jfo_matmul(type_id, ptr, n, rows, _fp(x), x.shape[0], _fp(y), mode, threads) != 0:
        raise ValueError("oracle matmul failed")
    del keep
    return y


def rope_table(base: float, head_dim: int, pos_begin: int, count: int) -> np.ndarray:
    out = np.zeros((count, head_dim), dtype=np.float32)
    lib().jfo_rope_table(base, head_dim, pos_begin, count, _fp(out))
    return out


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().jfo_argmax(_fp(x), x.size))


class OracleModel:
    """Oracle view of a model's tensors.

    ``tensor(name)`` must return a dict with ``type``, ``shape`` (GGML ne0, ne1)
    and ``data`` (address of the encoded bytes), e.g. jetsonfabric_amd.Model.tensor.
    The memory must outlive this object.
    """

    NAMES = ("attn_norm.weight", "attn_q.weight", "attn_q.bias", "attn_k.weight", "attn_k.bias", "attn_v.weight",
             "attn_v.bias", "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
             "ffn_down.weight")

    def __init__(self, config, tensor: Callable[[str], dict], has: Callable[[str], bool] | None = None):
        self.config = config

        def t(name: str) -> _Tensor:
            v = tensor(name)
            shape = tuple(v["shape"]) + (1,)
            return _Tensor(v["type"], 0, shape[0], shape[1] if len(v["shape"]) > 1 else 1, v["data"])

        self._layers = (_Layer * config.n_layer)()
        for l in range(config.n_layer):
            for field, name in zip([f for f, _ in _Layer._fields_], self.NAMES):
                setattr(self._layers[l], field, t(f"blk.{l}.{name}"))
        bias = _Tensor(F32, 0, 0, 1, None)
        if has is not None and has("output.bias"):
            bias = t("output.bias")
        self._m = _Model(config.n_layer, config.n_embd, config.n_ff, config.n_head, config.n_head_kv, config.n_ctx,
                         config.n_vocab, 0, config.rope_base, config.rms_eps, t("token_embd.weight"),
                         t("output_norm.weight"), t("output.weight"), bias,
                         ctypes.cast(self._layers, POINTER(_Layer)))

    @classmethod
    def from_model(cls, model, overrides: dict | None = None) -> "OracleModel":
        """Oracle over a jetsonfabric_amd Model's host tensors; `overrides`
        maps tensor names to float32 arrays of the same shape used instead
        (kept alive by the returned object)."""
        names = set(model.tensor_names())
        held = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in (overrides or {}).items()}

        def tensor(name: str) -> dict:
            v = model.tensor(name)
            if name not in held:
                return v
            if v["type"] != F32 or held[name].size != int(np.prod(v["shape"])):
                raise ValueError(f"override of {name} must be float32 of shape {v['shape']}")
            return dict(v, data=held[name].ctypes.data)

        om = cls(model.config, tensor, lambda n: n in names)
        om._held = held
        return om

    def session(self, capacity: int, mode: int = MODE_Q8, threads: int = 8) -> "OracleSession":
        return OracleSession(self, capacity, mode, threads)


class OracleSession:
    def __init__(self, model: OracleModel, capacity: int, mode: int = MODE_Q8, threads: int = 8):
        self.model = model
        self._h = lib().jfo_session_create(ctypes.byref(model._m), capacity, mode, threads)
        if not self._h:
            raise ValueError("oracle session rejected its arguments")

    def close(self):
        if self._h:
            lib().jfo_session_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def position(self) -> int:
        return lib().jfo_session_position(self._h)

    def forward(self, tokens: Sequence[int], logits_rows: int = 1):
        """Returns (argmax ids of the logits rows, logits [rows, vocab])."""
        n = len(tokens)
        v = self.model.config.n_vocab
        logits = np.zeros((max(logits_rows, 1), v), dtype=np.float32)
        ids = (c_int32 * max(logits_rows, 1))()
        rc = lib().jfo_session_forward(self._h, (c_int32 * n)(*tokens), n, logits_rows,
                                       _fp(logits) if logits_rows else None, ids if logits_rows else None)
        if rc == -2:
            raise ValueError("native Qwen2 step is outside session capacity")
        if rc == -3:
            raise ValueError("native token ID is outside model vocabulary")
        if rc != 0:
            raise ValueError("oracle forward rejected its arguments")
        return [int(x) for x in ids[:logits_rows]], logits[:logits_rows]

    def forward_range(self, layer_begin: int, layer_end: int, tokens: Sequence[int] | None = None,
                      rows: np.ndarray | None = None, logits_rows: int = 0):
        """Stage forward over layers [layer_begin, layer_end): token ids into the
        first stage, f32 residual rows [n, n_embd] into a later one. Returns
        (boundary rows [layer_end - layer_begin + 1, n, n_embd]: the rows entering
        each layer, then the rows after the last; argmax ids; logits [rows, vocab]
        when the range ends at the last layer and logits_rows > 0)."""
        c = self.model.config
        if (tokens is None) == (rows is None):
            raise ValueError("give token ids or residual rows")
        n = len(tokens) if tokens is not None else int(np.asarray(rows).shape[0])
        out = np.zeros((layer_end - layer_begin + 1, n, c.n_embd), dtype=np.float32)
        rows_in = None
        if rows is not None:
            rows_in = np.ascontiguousarray(rows, dtype=np.float32).reshape(n, c.n_embd)
        logits = np.zeros((max(logits_rows, 1), c.n_vocab), dtype=np.float32) if logits_rows else None
        ids = (c_int32 * max(logits_rows, 1))()
        rc = lib().jfo_session_forward_range(self._h, (c_int32 * n)(*tokens) if tokens is not None else None,
                                             _fp(rows_in) if rows_in is not None else None, n, layer_begin,
                                             layer_end, _fp(out), logits_rows,
                                             _fp(logits) if logits_rows else None, ids if logits_rows else None)
        if rc == -2:
            raise ValueError("native Qwen2 step is outside session capacity")
        if rc != 0:
            raise ValueError("oracle stage forward rejected its arguments")
        return out, [int(x) for x in ids[:logits_rows]], (logits[:logits_rows] if logits_rows else None)

    def rollback(self, n: int) -> None:
        if lib().jfo_session_rollback(self._h, n) != 0:
            raise ValueError("native Qwen2 rollback exceeds the decoded suffix")

    def fill_kv(self, n: int, seed: int = 1) -> None:
        if lib().jfo_session_fill_kv(self._h, n, seed) != 0:
            raise ValueError("fill_kv rejected its arguments")

    def read_kv(self, layer: int, n: int):
        c = self.model.config
        k = np.zeros((c.n_head_kv, n, c.head_dim), dtype=np.uint16)
        v = np.zeros_like(k)
        lib().jfo_session_read_kv(self._h, layer, n, k.ctypes.data_as(POINTER(c_uint16)),
                                  v.ctypes.data_as(POINTER(c_uint16)))
        return k, v


# ----------------------------------------------------------------- host logic restatements

def prompt_lookup(history: Sequence[int], max_tokens: int, max_ngram: int = 4, min_ngram: int = 2) -> list[int]:
    """runtime/speculative/prompt_lookup_draft.cpp:15-44, loop for loop."""
    if min_ngram == 0 or max_ngram < min_ngram:
        raise ValueError("prompt lookup requires 0 < min_ngram <= max_ngram")
    if max_tokens == 0 or len(history) <= min_ngram:
        return []
    largest = min(max_ngram, len(history) - 1)
    for ngram in range(largest, min_ngram - 1, -1):
        suffix_start = len(history) - ngram
        for candidate in range(suffix_start - 1, -1, -1):
            if candidate + ngram > suffix_start:
                continue
            if list(history[candidate:candidate + ngram]) != list(history[suffix_start:]):
                continue
            start = candidate + ngram
            count = min(max_tokens, len(history) - start)
            return list(history[start:start + count])
    return []


def speculative_generate(prefill: Callable[[Sequence[int]], int], verify: Callable[[Sequence[int]], list[int]],
                         rollback: Callable[[int], None], prompt: Sequence[int], max_tokens: int, draft_max: int,
                         max_ngram: int = 4, min_ngram: int = 2, is_eog: Callable[[int], bool] = lambda t: False,
                         propose: Callable[[list[int], int], list[int]] | None = None):
    """GenerationRunner::run speculative section (generation_runner.cpp:398-566) for one stage.

    prefill(prompt) -> first token; verify([prev, draft...]) -> greedy id after every row;
    rollback(n) removes n decoded positions. `propose(history, budget)` replaces
    the prompt-lookup draft strategy (the runner takes any DraftStrategy,
    generation_runner.hpp). Returns (tokens, stats).
    """
    stats = {"target_decode_passes": 0, "speculative_draft_tokens": 0, "speculative_accepted_tokens": 0,
             "rollbacks": []}
    out: list[int] = []
    history = list(prompt)
    first = prefill(prompt)
    eog = is_eog(first)
    previous = first
    if not eog:
        out.append(first)
        history.append(first)
    recover = False
    while len(out) < max_tokens and not eog:
        remaining = max_tokens - len(out)
        draft = []
        if draft_max > 0 and remaining > 1 and not recover:
            budget = min(draft_max, remaining - 1)
            draft = (propose(list(history), budget) if propose is not None
                     else prompt_lookup(history, budget, max_ngram, min_ngram))
        recover = False
        verification = [previous] + draft
        target = verify(verification)
        stats["target_decode_passes"] += 1
        if len(target) != len(verification):
            raise ValueError("target output count does not match speculative verification input")
        accepted = 0
        while accepted < len(draft) and not is_eog(target[accepted]) and target[accepted] == draft[accepted]:
            accepted += 1
        stats["speculative_draft_tokens"] += len(draft)
        stats["speculative_accepted_tokens"] += accepted
        rollback_tokens = len(draft) - accepted if accepted < len(draft) else 0
        if rollback_tokens:
            rollback(rollback_tokens)
            stats["rollbacks"].append(rollback_tokens)
            recover = True
        count = accepted + 1 if accepted < len(draft) else len(target)
        for i in range(count):
            if len(out) >= max_tokens:
                break
            if is_eog(target[i]):
                eog = True
                break
            out.append(target[i])
            history.append(target[i])
            previous = target[i]
    return out, stats


# ----------------------------------------------------------------- metrics

def nrmse(reference: np.ndarray, candidate: np.ndarray) -> float:
    """RMS error normalized by the reference range (native_attention_parity.cpp:133-167 style)."""
    reference = np.asarray(reference, dtype=np.float64)
    candidate = np.asarray(candidate, dtype=np.float64)
    span = float(reference.max() - reference.min())
    return float(np.sqrt(np.mean((reference - candidate) ** 2)) / (span if span > 0 else 1.0))


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


# ----------------------------------------------------------------- reference loader (built from its sources)

class _JfStatus(ctypes.Structure):
    _fields_ = [("code", c_int32), ("message", c_char * 256)]


class _JfPlan(ctypes.Structure):
    _fields_ = [("layer_start", c_uint32), ("layer_end", c_uint32), ("verify_hashes", c_uint32),
                ("evict_before_open", c_uint32)]


class _JfStats(ctypes.Structure):
    _fields_ = [("layer_start", c_uint32), ("layer_end", c_uint32), ("layer_count", c_uint32),
                ("selected_weight_bytes", c_uint64), ("total_weight_bytes", c_uint64), ("mapped_bytes", c_uint64),
                ("selected_tensor_count", c_uint64), ("total_tensor_count", c_uint64)]


class _JfView(ctypes.Structure):
    _fields_ = [("name", c_void_p), ("name_length", c_size_t), ("type", c_uint32), ("rank", c_uint32),
                ("storage_block_elements", c_uint32), ("storage_block_bytes", c_uint32), ("shape", c_uint64 * 4),
                ("layer", c_int32), ("data", c_void_p), ("size", c_uint64)]


class ref_loader:
    """The reference's jf_model_* loader compiled from its sources (oracle/_ref)."""

    _lib = None

    @classmethod
    def available(cls) -> bool:
        return os.path.exists(REF_LIB_PATH)

    @classmethod
    def lib(cls):
        if cls._lib is None:
            l = ctypes.CDLL(REF_LIB_PATH)
            l.jf_model_open.restype = _JfStatus
            l.jf_model_open.argtypes = [c_char_p, POINTER(_JfPlan), POINTER(c_void_p)]
            l.jf_model_close.argtypes = [c_void_p]
            l.jf_model_get_stats.restype = _JfStats
            l.jf_model_get_stats.argtypes = [c_void_p]
            l.jf_model_tensor_count.restype = c_size_t
            l.jf_model_tensor_count.argtypes = [c_void_p]
            l.jf_model_tensor_at.restype = _JfStatus
            l.jf_model_tensor_at.argtypes = [c_void_p, c_size_t, POINTER(_JfView)]
            l.jf_tensor_type_layout.restype = _JfStatus
            l.jf_tensor_type_layout.argtypes = [c_uint32, POINTER(c_uint32), POINTER(c_uint32)]
            l.jf_sha256_buffer.restype = None
            l.jf_sha256_buffer.argtypes = [c_void_p, c_size_t, POINTER(ctypes.c_uint8)]
            cls._lib = l
        return cls._lib

    @classmethod
    def open(cls, path: str, layer_start: int = 0, layer_end: int = 0xFFFFFFFF, verify_hashes: bool = True):
        """Returns (status code, message, stats dict, {name: (type, shape, bytes)})."""
        l = cls.lib()
        plan = _JfPlan(layer_start, layer_end, int(verify_hashes), 0)
        h = c_void_p()
        st = l.jf_model_open(path.encode(), ctypes.byref(plan), ctypes.byref(h))
        if st.code != 0:
            return st.code, st.message.decode(), None, None
        try:
            s = l.jf_model_get_stats(h)
            stats = {f: getattr(s, f) for f, _ in _JfStats._fields_}
            tensors = {}
            for i in range(l.jf_model_tensor_count(h)):
                v = _JfView()
                l.jf_model_tensor_at(h, i, ctypes.byref(v))
                name = ctypes.string_at(v.name, v.name_length).decode()
                tensors[name] = (v.type, tuple(v.shape[d] for d in range(v.rank)), ctypes.string_at(v.data, v.size))
            return 0, "", stats, tensors
        finally:
            l.jf_model_close(h)

    @classmethod
    def type_layout(cls, type_id: int):
        e, b = c_uint32(), c_uint32()
        st = cls.lib().jf_tensor_type_layout(type_id, ctypes.byref(e), ctypes.byref(b))
        return (e.value, b.value) if st.code == 0 else None

    @classmethod
    def sha256(cls, data: bytes) -> bytes:
        out = (ctypes.c_uint8 * 32)()
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        cls.lib().jf_sha256_buffer(buf, len(data), out)
        return bytes(out)
