"""ctypes binding of libjfh.so (declarations in include/jfh.h).

The shared library is built in-tree (``make -C jetsonfabric_amd``) and loaded
from this package directory only; a missing library is an error, never a
fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, c_char, c_char_p, c_double, c_float, c_int32, c_size_t, c_uint8, c_uint16, c_uint32,
                    c_uint64, c_void_p)

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "libjfh.so")

# Stable JFM tensor type ids (runtime/engines/native/include/jetsonfabric/engine.h:13-49).
F32, F16, Q8_0, Q2_K, Q4_K, Q6_K = 1, 2, 7, 9, 11, 13
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K"}


class Status(ctypes.Structure):
    _fields_ = [("code", c_int32), ("message", c_char * 256)]


class ModelParams(ctypes.Structure):
    _fields_ = [
        ("n_layer", c_uint32), ("n_embd", c_uint32), ("n_ff", c_uint32), ("n_head", c_uint32),
        ("n_head_kv", c_uint32), ("n_ctx", c_uint32), ("n_vocab", c_uint32), ("head_dim", c_uint32),
        ("rope_base", c_float), ("rms_eps", c_float),
    ]


class TensorView(ctypes.Structure):
    _fields_ = [
        ("name", c_char_p), ("type", c_uint32), ("rank", c_uint32), ("shape", c_uint64 * 4),
        ("layer", c_int32), ("data", c_void_p), ("size", c_uint64),
    ]


class ModelStats(ctypes.Structure):
    _fields_ = [
        ("layer_start", c_uint32), ("layer_end", c_uint32), ("layer_count", c_uint32),
        ("selected_weight_bytes", c_uint64), ("total_weight_bytes", c_uint64),
        ("selected_tensor_count", c_uint64), ("total_tensor_count", c_uint64),
    ]


class SynthSpec(ctypes.Structure):
    _fields_ = [
        ("params", ModelParams), ("type_linear", c_uint32), ("type_embd", c_uint32), ("type_output", c_uint32),
        ("tied_output", c_uint32), ("output_bias", c_uint32), ("pad", c_uint32), ("seed", c_uint64),
        ("stddev", c_float), ("threads", c_int32),
    ]


class EngineOptions(ctypes.Structure):
    _fields_ = [("device", c_int32), ("use_graphs", c_int32)]


class EngineInfo(ctypes.Structure):
    _fields_ = [("weight_bytes", c_uint64), ("prefill_chunk", c_uint32), ("device_name", c_char * 128),
                ("layer_start", c_uint32), ("layer_end", c_uint32)]


class GenerationStats(ctypes.Structure):
    _fields_ = [
        ("completion_tokens", c_uint32), ("target_decode_passes", c_uint32),
        ("speculative_draft_tokens", c_uint32), ("speculative_accepted_tokens", c_uint32),
        ("time_to_first_token_ms", c_double), ("decode_ms", c_double),
        ("stopped", c_uint32), ("reserved", c_uint32),
        ("inter_token_latency_ms", c_double), ("decode_tokens_per_second", c_double),
        ("end_to_end_tokens_per_second", c_double),
        ("prefill_plan_reused", c_uint32), ("prefill_attention_matrix_cores", c_uint32),
        ("prefill_planning_ms", c_double), ("prefill_allocation_ms", c_double), ("prefill_host_input_ms", c_double),
        ("prefill_compute_ms", c_double), ("prefill_output_read_ms", c_double),
        ("kv_cache_bytes", c_uint64), ("prefill_scratch_bytes", c_uint64), ("decode_scratch_bytes", c_uint64),
        ("prefill_host_input_bytes", c_uint64),
    ]


# jfh_draft_propose_fn: (user, history, n, max_tokens, out) -> count
DraftProposeFn = ctypes.CFUNCTYPE(c_uint32, c_void_p, POINTER(c_uint32), c_size_t, c_uint32, POINTER(c_uint32))


class PackageStats(ctypes.Structure):
    _fields_ = [
        ("layer_start", c_uint32), ("layer_end", c_uint32), ("layer_count", c_uint32), ("pad", c_uint32),
        ("selected_weight_bytes", c_uint64), ("total_weight_bytes", c_uint64), ("mapped_bytes", c_uint64),
        ("selected_tensor_count", c_uint64), ("total_tensor_count", c_uint64),
    ]


class KernelStat(ctypes.Structure):
    _fields_ = [("label", c_char * 64), ("launches", c_double), ("total_ms", c_double), ("bytes", c_double)]


# name -> (restype, argtypes)
SIGNATURES = {
    "jfh_session_profile_step": (Status, [c_void_p, POINTER(c_int32), c_uint32, c_uint32, c_uint32, POINTER(KernelStat),
                                          c_uint32, POINTER(c_uint32)]),
    "jfh_engine_profile_batch": (Status, [c_void_p, POINTER(c_void_p), c_uint32, POINTER(c_int32), POINTER(c_uint32),
                                         c_uint32, c_uint32, POINTER(KernelStat), c_uint32, POINTER(c_uint32)]),
    "jfh_package_open": (Status, [c_char_p, c_uint32, c_uint32, c_uint32, POINTER(c_void_p)]),
    "jfh_package_close": (None, [c_void_p]),
    "jfh_package_get_stats": (Status, [c_void_p, POINTER(PackageStats)]),
    "jfh_package_tensor_count": (c_size_t, [c_void_p]),
    "jfh_package_tensor_at": (Status, [c_void_p, c_size_t, POINTER(TensorView)]),
    "jfh_package_find_tensor": (Status, [c_void_p, c_char_p, POINTER(TensorView)]),
    "jfh_package_gguf_metadata": (Status, [c_void_p, POINTER(c_void_p), POINTER(c_size_t)]),
    "jfh_package_source_sha256": (Status, [c_void_p, POINTER(c_uint8)]),
    "jfh_tensor_type_layout": (Status, [c_uint32, POINTER(c_uint32), POINTER(c_uint32)]),
    "jfh_sha256": (Status, [c_void_p, c_size_t, POINTER(c_uint8)]),
    "jfh_model_open": (Status, [c_char_p, c_uint32, c_uint32, c_uint32, POINTER(c_void_p)]),
    "jfh_model_open_gguf": (Status, [c_char_p, POINTER(c_void_p)]),
    "jfh_model_synthesize": (Status, [POINTER(SynthSpec), POINTER(c_void_p)]),
    "jfh_model_create": (Status, [POINTER(ModelParams), POINTER(c_void_p)]),
    "jfh_model_add_tensor": (Status, [c_void_p, c_char_p, c_uint32, c_uint32, POINTER(c_uint64), c_void_p, c_uint64]),
    "jfh_model_finalize": (Status, [c_void_p]),
    "jfh_model_write_package": (Status, [c_void_p, c_char_p]),
    "jfh_model_slice": (Status, [c_void_p, c_uint32, c_uint32, POINTER(c_void_p)]),
    "jfh_model_close": (None, [c_void_p]),
    "jfh_model_get_params": (Status, [c_void_p, POINTER(ModelParams)]),
    "jfh_model_get_stats": (Status, [c_void_p, POINTER(ModelStats)]),
    "jfh_model_tensor_count": (c_size_t, [c_void_p]),
    "jfh_model_tensor_at": (Status, [c_void_p, c_size_t, POINTER(TensorView)]),
    "jfh_model_find_tensor": (Status, [c_void_p, c_char_p, POINTER(TensorView)]),
    "jfh_model_source_sha256": (Status, [c_void_p, c_char * 65]),
    "jfh_engine_create": (Status, [c_void_p, POINTER(EngineOptions), POINTER(c_void_p)]),
    "jfh_engine_destroy": (None, [c_void_p]),
    "jfh_engine_get_info": (Status, [c_void_p, POINTER(EngineInfo)]),
    "jfh_engine_set_end_tokens": (Status, [c_void_p, POINTER(c_int32), c_uint32]),
    "jfh_engine_get_params": (Status, [c_void_p, POINTER(ModelParams)]),
    "jfh_session_create": (Status, [c_void_p, c_uint32, POINTER(c_void_p)]),
    "jfh_session_destroy": (None, [c_void_p]),
    "jfh_session_capacity": (c_uint32, [c_void_p]),
    "jfh_session_position": (c_uint32, [c_void_p]),
    "jfh_session_prefill": (Status, [c_void_p, POINTER(c_int32), c_uint32, POINTER(c_int32), POINTER(c_float)]),
    "jfh_session_decode": (Status, [c_void_p, c_int32, POINTER(c_int32), POINTER(c_float)]),
    "jfh_session_verify": (Status, [c_void_p, POINTER(c_int32), c_uint32, POINTER(c_int32), POINTER(c_uint32),
                                    POINTER(c_float)]),
    "jfh_session_rollback": (Status, [c_void_p, c_uint32]),
    "jfh_activation_encode": (Status, [c_char_p, POINTER(c_float), c_size_t, c_void_p, c_size_t]),
    "jfh_activation_decode": (Status, [c_char_p, c_void_p, c_size_t, POINTER(c_float), c_size_t]),
    "jfh_session_stage_prefill": (Status, [c_void_p, POINTER(c_int32), POINTER(c_float), c_uint32, POINTER(c_int32),
                                           POINTER(c_float), POINTER(c_float)]),
    "jfh_session_stage_decode": (Status, [c_void_p, POINTER(c_int32), POINTER(c_float), POINTER(c_int32),
                                          POINTER(c_float), POINTER(c_float)]),
    "jfh_engine_step_batch": (Status, [c_void_p, POINTER(c_void_p), c_uint32, POINTER(c_int32), POINTER(c_uint32),
                                       POINTER(c_int32), POINTER(c_uint32), POINTER(c_float)]),
    "jfh_engine_dequantize": (Status, [c_void_p, c_char_p, c_uint32, c_uint32, POINTER(c_float)]),
    "jfh_engine_stage_step_batch": (Status, [c_void_p, POINTER(c_void_p), c_uint32, POINTER(c_int32), POINTER(c_float),
                                             POINTER(c_uint32), POINTER(c_int32), POINTER(c_float), POINTER(c_float)]),
    "jfh_engine_matmul_noalloc": (Status, [c_void_p, c_char_p, c_void_p, c_uint32, c_void_p, c_void_p]),
    "jfh_engine_matmul": (Status, [c_void_p, c_char_p, POINTER(c_float), c_uint32, POINTER(c_float)]),
    "jfh_session_read_kv": (Status, [c_void_p, c_uint32, c_uint32, POINTER(c_uint16), POINTER(c_uint16)]),
    "jfh_session_import_kv": (Status, [c_void_p, c_uint32, POINTER(c_uint16), POINTER(c_uint16)]),
    "jfh_session_time_steps": (Status, [c_void_p, POINTER(c_int32), c_uint32, c_uint32, c_uint32, c_uint32,
                                        POINTER(c_double)]),
    "jfh_prompt_lookup_propose": (Status, [POINTER(c_uint32), c_size_t, c_uint32, c_uint32, c_uint32,
                                           POINTER(c_uint32), POINTER(c_uint32)]),
    "jfh_tokenizer_open": (Status, [c_char_p, POINTER(c_void_p)]),
    "jfh_tokenizer_destroy": (None, [c_void_p]),
    "jfh_tokenizer_tokenize": (Status, [c_void_p, c_char_p, c_size_t, POINTER(c_int32), c_uint32, POINTER(c_uint32)]),
    "jfh_tokenizer_token_piece": (Status, [c_void_p, c_int32, c_char_p, c_uint32, POINTER(c_uint32)]),
    "jfh_tokenizer_is_end_token": (Status, [c_void_p, c_int32, POINTER(c_uint32)]),
    "jfh_tokenizer_end_tokens": (Status, [c_void_p, POINTER(c_int32), c_uint32, POINTER(c_uint32)]),
    "jfh_tokenizer_vocab_size": (Status, [c_void_p, POINTER(c_uint32)]),
    "jfh_generate": (Status, [c_void_p, POINTER(c_int32), c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                              POINTER(c_int32), POINTER(c_uint32), POINTER(GenerationStats)]),
    "jfh_generate_draft": (Status, [c_void_p, POINTER(c_int32), c_uint32, c_uint32, c_uint32, DraftProposeFn, c_void_p,
                                    POINTER(c_int32), POINTER(c_uint32), POINTER(GenerationStats)]),
    "jfh_generate_concurrent": (Status, [c_void_p, c_uint32, POINTER(c_int32), POINTER(c_uint32), c_uint32, c_uint32,
                                         c_uint32, c_uint32, c_uint32, POINTER(c_int32), POINTER(c_uint32),
                                         POINTER(GenerationStats), POINTER(c_double)]),
}

STATUS_NAMES = {0: "ok", 1: "invalid_argument", 2: "io_error", 3: "format_error", 4: "not_found",
                5: "out_of_memory", 6: "device_error"}


class JfhError(RuntimeError):
    """A non-OK jfh_status; ``code`` is the jfh_status_code."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


class InvalidArgument(JfhError, ValueError):
    pass


_lib = None


def library() -> ctypes.CDLL:
    """Loads the in-tree libjfh.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(f"{LIBRARY_PATH} is missing: build it with `make -C jetsonfabric_amd`")
        lib = ctypes.CDLL(LIBRARY_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: Status) -> None:
    if status.code != 0:
        message = status.message.decode("utf-8", "replace")
        if status.code == 1:
            raise InvalidArgument(status.code, message)
        raise JfhError(status.code, message)
