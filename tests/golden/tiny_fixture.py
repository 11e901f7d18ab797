"""The reference's tiny Qwen2 fixture, restated as data.

runtime/compiler/model_fixture.cpp:76-133 writes a 2-layer F32 Qwen2 GGUF:
hidden 4, FFN 8, 1 head / 1 KV head (head_dim 4), vocab 8, context 16, RoPE
base 1e4 over 4 dims, RMS eps 1e-5. Norm gains are 1, biases 0, every
attention/FFN matrix is the constant 0.01, token_embd row r is 0.1*(r+1) and
output row r is 0.01*(r+1). Its known answer: greedy prompt [2] -> [7, 7]
(runtime/compiler/compiler_integration_test.cmake:55-81) and [2, 2] -> [7]
(114-139).
"""
from __future__ import annotations

import struct

F32 = 1
CONFIG = dict(n_layer=2, n_embd=4, n_ff=8, n_head=1, n_head_kv=1, n_vocab=8, n_ctx=16, rope_base=10000.0,
              rms_eps=1.0e-5)
EXPECTED = {(2,): [7, 7], (2, 2): [7]}


def _f32(values):
    return struct.pack(f"<{len(values)}f", *values)


def _const(cols, rows, value):
    return _f32([value] * (cols * rows))


def _row_scaled(cols, rows, scale):
    return _f32([scale * (r + 1) for r in range(rows) for _ in range(cols)])


def tensors():
    """(name, type, GGML shape (ne0, ne1), bytes) in the order the fixture writer adds them."""
    out = [("token_embd.weight", F32, (4, 8), _row_scaled(4, 8, 0.1))]
    for layer in range(2):
        p = f"blk.{layer}."
        out += [
            (p + "attn_norm.weight", F32, (4,), _const(4, 1, 1.0)),
            (p + "attn_q.weight", F32, (4, 4), _const(4, 4, 0.01)),
            (p + "attn_q.bias", F32, (4,), _const(4, 1, 0.0)),
            (p + "attn_k.weight", F32, (4, 4), _const(4, 4, 0.01)),
            (p + "attn_k.bias", F32, (4,), _const(4, 1, 0.0)),
            (p + "attn_v.weight", F32, (4, 4), _const(4, 4, 0.01)),
            (p + "attn_v.bias", F32, (4,), _const(4, 1, 0.0)),
            (p + "attn_output.weight", F32, (4, 4), _const(4, 4, 0.01)),
            (p + "ffn_norm.weight", F32, (4,), _const(4, 1, 1.0)),
            (p + "ffn_gate.weight", F32, (4, 8), _const(4, 8, 0.01)),
            (p + "ffn_down.weight", F32, (8, 4), _const(8, 4, 0.01)),
            (p + "ffn_up.weight", F32, (4, 8), _const(4, 8, 0.01)),
        ]
    out += [
        ("output_norm.weight", F32, (4,), _const(4, 1, 1.0)),
        ("output.weight", F32, (4, 8), _row_scaled(4, 8, 0.01)),
    ]
    return out
