"""MI355X (gfx950) native Qwen2 stage engine for jetsonfabric's speculative decoder.

The compute path is libjfh.so (hand-written HIP kernels + C++ host); this
package is its Python face. Importing it does not touch the GPU.
"""
from ._capi import F16, F32, JfhError, InvalidArgument, LIBRARY_PATH, Q2_K, Q4_K, Q6_K, Q8_0, TYPE_NAMES, library
from .engine import (GenerationResult, Model, ModelConfig, NativeEngine, NativeSession, Package, Tokenizer,
                     activation_decode, activation_encode, prompt_lookup_propose, sha256, type_layout)
from .configs import CONFIGS, config_by_name

__all__ = [
    "F32", "F16", "Q8_0", "Q2_K", "Q4_K", "Q6_K", "TYPE_NAMES", "JfhError", "InvalidArgument", "LIBRARY_PATH",
    "library", "GenerationResult", "Model", "Package", "Tokenizer", "ModelConfig", "NativeEngine", "NativeSession", "prompt_lookup_propose",
    "sha256", "type_layout", "CONFIGS", "config_by_name", "activation_encode", "activation_decode",
]
