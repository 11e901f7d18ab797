"""Qwen2.5-shaped model configurations used for parity and throughput runs.

Shapes are the public Qwen2.5 ones; weights are synthetic (seeded N(0, 0.02)
quantized per tensor type). Each entry also carries the tensor types and the
serving parameters of its workload.
"""
from __future__ import annotations

from dataclasses import dataclass

from ._capi import Q2_K, Q4_K, Q6_K, Q8_0
from .engine import ModelConfig


@dataclass(frozen=True)
class Workload:
    name: str
    model: ModelConfig
    type_linear: int
    type_embd: int
    type_output: int
    tied_output: bool
    concurrency: int
    prompt_tokens: int
    output_tokens: int
    draft_max: int
    ngram: int

    @property
    def description(self) -> str:
        m = self.model
        return (f"{self.name}: {m.n_layer} layers, hidden {m.n_embd}, {m.n_head}/{m.n_head_kv} heads, "
                f"ffn {m.n_ff}, vocab {m.n_vocab}")


QWEN_1_5B = ModelConfig(n_layer=28, n_embd=1536, n_ff=8960, n_head=12, n_head_kv=2, n_vocab=151936)
QWEN_7B = ModelConfig(n_layer=28, n_embd=3584, n_ff=18944, n_head=28, n_head_kv=4, n_vocab=152064)
QWEN_14B = ModelConfig(n_layer=48, n_embd=5120, n_ff=13824, n_head=40, n_head_kv=8, n_vocab=152064)
QWEN_32B = ModelConfig(n_layer=64, n_embd=5120, n_ff=27648, n_head=40, n_head_kv=8, n_vocab=152064)

CONFIGS = {
    "qwen2.5-1.5b-q4k": Workload("qwen2.5-1.5b-q4k", QWEN_1_5B, Q4_K, Q8_0, Q8_0, True, 1, 256, 128, 0, 3),
    "qwen2.5-1.5b-q4k-spec": Workload("qwen2.5-1.5b-q4k-spec", QWEN_1_5B, Q4_K, Q8_0, Q8_0, True, 1, 512, 256, 4, 3),
    "qwen2.5-7b-q4k": Workload("qwen2.5-7b-q4k", QWEN_7B, Q4_K, Q4_K, Q6_K, False, 2, 1024, 256, 4, 3),
    "qwen2.5-14b-q4k": Workload("qwen2.5-14b-q4k", QWEN_14B, Q4_K, Q4_K, Q4_K, False, 2, 4096, 256, 8, 3),
    "qwen2.5-32b-q2k": Workload("qwen2.5-32b-q2k", QWEN_32B, Q2_K, Q2_K, Q6_K, False, 8, 2048, 256, 4, 3),
}


def config_by_name(name: str) -> Workload:
    return CONFIGS[name]
