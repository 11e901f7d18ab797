"""Pins the oracle's Qwen2 forward, session bookkeeping and speculation logic (CPU only).

* The reference's own known answer: its tiny F32 fixture model
  (runtime/compiler/model_fixture.cpp:76-133) decodes prompt [2] -> [7, 7]
  (compiler_integration_test.cmake:55-81) and [2, 2] -> [7] (114-139).
* A float64 brute force of the Qwen2 graph written from its definition
  (qwen2_architecture.cpp:522-598: RMSNorm, biased QKV, NEOX RoPE, causal GQA
  softmax attention, SwiGLU, residuals, output norm + head), evaluated on a
  small random F32 model; the oracle rounds K/V to binary16 like the
  reference cache, hence the tolerance.
* Verify-equals-serial and rollback-replay invariants
  (llama_cpp_stage_adapter_test.cpp:267-408), greedy invariance of the
  speculative loop (generation_runner.cpp:469-556), prompt-lookup KATs
  (runtime/speculative/prompt_lookup_draft_test.cpp:19-32).
* RoPE table closed form.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import jetsonfabric_amd as jf
import oracle as jo
from tests.golden import tiny_fixture


def tiny_model():
    return jf.Model.build(jf.ModelConfig(**tiny_fixture.CONFIG), tiny_fixture.tensors())


def greedy(session, prompt, n):
    ids, _ = session.forward(prompt, 1)
    out = [ids[0]]
    while len(out) < n:
        ids, _ = session.forward([out[-1]], 1)
        out.append(ids[0])
    return out


# ------------------------------------------------------------------ reference known answers

@pytest.mark.parametrize("mode", [jo.MODE_EXACT, jo.MODE_Q8])
def test_tiny_fixture_known_answers(mode):
    model = tiny_model()
    om = jo.OracleModel.from_model(model)
    for prompt, expected in tiny_fixture.EXPECTED.items():
        s = om.session(16, mode, 1)
        assert greedy(s, list(prompt), len(expected)) == expected


# ------------------------------------------------------------------ float64 brute force

CFG = jf.ModelConfig(n_layer=2, n_embd=64, n_ff=96, n_head=4, n_head_kv=2, n_vocab=50, n_ctx=64,
                     rope_base=10000.0, rms_eps=1e-6)


def random_f32_model(seed=0, scale=0.15):
    rng = np.random.default_rng(seed)
    c = CFG
    hd = c.n_embd // c.n_head
    kv = c.n_head_kv * hd
    w = {}

    def mat(name, rows, cols):
        w[name] = rng.normal(0, scale, (rows, cols)).astype(np.float32)

    def vec(name, n, base=0.0, s=0.1):
        w[name] = (base + rng.normal(0, s, n)).astype(np.float32)

    mat("token_embd.weight", c.n_vocab, c.n_embd)
    w["token_embd.weight"] *= 6.0
    for l in range(c.n_layer):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", c.n_embd, 1.0)
        mat(p + "attn_q.weight", c.n_embd, c.n_embd)
        vec(p + "attn_q.bias", c.n_embd)
        mat(p + "attn_k.weight", kv, c.n_embd)
        vec(p + "attn_k.bias", kv)
        mat(p + "attn_v.weight", kv, c.n_embd)
        vec(p + "attn_v.bias", kv)
        mat(p + "attn_output.weight", c.n_embd, c.n_embd)
        vec(p + "ffn_norm.weight", c.n_embd, 1.0)
        mat(p + "ffn_gate.weight", c.n_ff, c.n_embd)
        mat(p + "ffn_up.weight", c.n_ff, c.n_embd)
        mat(p + "ffn_down.weight", c.n_embd, c.n_ff)
    vec("output_norm.weight", c.n_embd, 1.0)
    mat("output.weight", c.n_vocab, c.n_embd)
    tensors = []
    for name, a in w.items():
        shape = (a.shape[1], a.shape[0]) if a.ndim == 2 else (a.shape[0],)
        tensors.append((name, jo.F32, shape, a.tobytes()))
    return jf.Model.build(c, tensors), {k: v.astype(np.float64) for k, v in w.items()}


def brute_force_logits(w, tokens):
    """Logits of every row for tokens at positions 0..n-1 (float64, no caching)."""
    c = CFG
    hd = c.n_embd // c.n_head
    group = c.n_head // c.n_head_kv
    n = len(tokens)

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + c.rms_eps) * g

    def rope(x):  # x [n, heads, hd], NEOX pairs (i, i + hd/2)
        half = hd // 2
        inv = c.rope_base ** (-2.0 * np.arange(half) / hd)
        ang = np.arange(n)[:, None] * inv[None, :]
        cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a, b = x[..., :half], x[..., half:]
        return np.concatenate([a * cos - b * sin, a * sin + b * cos], axis=-1)

    h = w["token_embd.weight"][tokens]
    for l in range(c.n_layer):
        p = f"blk.{l}."
        x = rms(h, w[p + "attn_norm.weight"])
        q = (x @ w[p + "attn_q.weight"].T + w[p + "attn_q.bias"]).reshape(n, c.n_head, hd)
        k = (x @ w[p + "attn_k.weight"].T + w[p + "attn_k.bias"]).reshape(n, c.n_head_kv, hd)
        v = (x @ w[p + "attn_v.weight"].T + w[p + "attn_v.bias"]).reshape(n, c.n_head_kv, hd)
        q, k = rope(q), rope(k)
        out = np.zeros((n, c.n_head, hd))
        for head in range(c.n_head):
            kh = k[:, head // group]
            vh = v[:, head // group]
            s = q[:, head] @ kh.T / np.sqrt(hd)
            s = np.where(np.tril(np.ones((n, n), dtype=bool)), s, -np.inf)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            out[:, head] = (s / s.sum(axis=1, keepdims=True)) @ vh
        h = h + out.reshape(n, c.n_embd) @ w[p + "attn_output.weight"].T
        x = rms(h, w[p + "ffn_norm.weight"])
        g = x @ w[p + "ffn_gate.weight"].T
        u = x @ w[p + "ffn_up.weight"].T
        h = h + (g / (1.0 + np.exp(-g)) * u) @ w[p + "ffn_down.weight"].T
    return rms(h, w["output_norm.weight"]) @ w["output.weight"].T


def test_forward_matches_float64_brute_force():
    model, w = random_f32_model(1)
    tokens = [int(t) for t in np.random.default_rng(2).integers(0, CFG.n_vocab, 12)]
    ref = brute_force_logits(w, tokens)
    s = jo.OracleModel.from_model(model).session(32, jo.MODE_EXACT, 2)
    ids, logits = s.forward(tokens, len(tokens))
    for r in range(len(tokens)):
        assert jo.nrmse(ref[r], logits[r]) < 2e-3, r
        assert jo.cosine(ref[r], logits[r]) > 0.99999, r
    # greedy ids where the brute force has a clear winner
    for r in range(len(tokens)):
        top2 = np.sort(ref[r])[-2:]
        if top2[1] - top2[0] > 1e-2 * (ref[r].max() - ref[r].min()):
            assert ids[r] == int(np.argmax(ref[r])), r


def test_incremental_decode_matches_full_recompute():
    model, w = random_f32_model(3)
    tokens = [int(t) for t in np.random.default_rng(4).integers(0, CFG.n_vocab, 10)]
    ref = brute_force_logits(w, tokens)
    s = jo.OracleModel.from_model(model).session(32, jo.MODE_EXACT, 1)
    s.forward(tokens[:6], 0)
    for i in range(6, 10):
        _, logits = s.forward([tokens[i]], 1)
        assert jo.nrmse(ref[i], logits[0]) < 2e-3


def test_brute_force_detects_a_planted_mistake():
    """Swapping the two kv heads (a wrong GQA mapping) must move the logits far
    beyond the tolerance used above: the comparison has teeth."""
    model, w = random_f32_model(1)
    tokens = [int(t) for t in np.random.default_rng(2).integers(0, CFG.n_vocab, 12)]
    ref = brute_force_logits(w, tokens)
    bad = dict(w)
    for l in range(CFG.n_layer):
        k = bad[f"blk.{l}.attn_k.weight"].copy()
        half = k.shape[0] // 2
        bad[f"blk.{l}.attn_k.weight"] = np.concatenate([k[half:], k[:half]])
    wrong = brute_force_logits(bad, tokens)
    assert max(jo.nrmse(ref[r], wrong[r]) for r in range(len(tokens))) > 1e-2


# ------------------------------------------------------------------ session invariants

def _q4k_model(seed=6):
    cfg = jf.ModelConfig(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=300, n_ctx=128)
    return jf.Model.synthesize(cfg, type_linear=jo.Q4_K, type_embd=jo.Q4_K, type_output=jo.Q6_K, seed=seed,
                               stddev=0.05, output_bias=True)


def test_verify_equals_serial_and_rollback_replay():
    model = _q4k_model()
    om = jo.OracleModel.from_model(model)
    prompt = [5, 17, 99, 3, 250, 7, 7, 12]
    a = om.session(64, jo.MODE_Q8, 2)
    serial = greedy(a, prompt, 6)
    _, serial_logits = a.forward([serial[-1]], 1)

    b = om.session(64, jo.MODE_Q8, 2)
    first, _ = b.forward(prompt, 1)
    assert first[0] == serial[0]
    ids, logits = b.forward(serial[:5], 5)
    assert ids == serial[1:6]
    assert b.position() == len(prompt) + 5
    # roll back three rows and replay them one at a time: same ids
    b.rollback(3)
    assert b.position() == len(prompt) + 2
    for i in range(2, 5):
        nid, nl = b.forward([serial[i]], 1)
        assert nid[0] == serial[i + 1]
        assert np.allclose(nl[0], logits[i], rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError):
        b.rollback(6)  # more than the decoded suffix
    with pytest.raises(ValueError):
        b.rollback(0)


def test_stage_range_forward_equals_the_full_forward():
    """The oracle's stage forward (layers [a, b) on token ids or residual rows,
    qwen2_architecture.cpp:909-947, 977-1027) chained over a split of the
    layers gives the full forward's logits bit for bit, prefill and decode,
    and its boundary rows are the embedding rows, then each layer's output."""
    cfg = jf.ModelConfig(n_layer=3, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=300, n_ctx=128)
    model = jf.Model.synthesize(cfg, type_linear=jo.Q4_K, type_embd=jo.Q8_0, type_output=jo.Q6_K, seed=9,
                                stddev=0.05)
    om = jo.OracleModel.from_model(model)
    prompt = [5, 17, 99, 3, 250, 7]
    full = om.session(32, jo.MODE_Q8, 2)
    f_ids, f_logits = full.forward(prompt, len(prompt))
    whole = om.session(32, jo.MODE_Q8, 2)
    rows, w_ids, w_logits = whole.forward_range(0, 3, tokens=prompt, logits_rows=len(prompt))
    assert w_ids == f_ids and np.array_equal(w_logits, f_logits)
    embd = model.tensor_bytes("token_embd.weight")
    rb = jo.row_bytes(jo.Q8_0, cfg.n_embd)
    for t, tok in enumerate(prompt):
        assert np.array_equal(rows[0][t], jo.dequantize_row(jo.Q8_0, embd[tok * rb:(tok + 1) * rb], cfg.n_embd))
    a, b = om.session(32, jo.MODE_Q8, 2), om.session(32, jo.MODE_Q8, 2)
    a_rows, _, _ = a.forward_range(0, 1, tokens=prompt)
    assert np.array_equal(a_rows, rows[:2])
    b_rows, b_ids, b_logits = b.forward_range(1, 3, rows=a_rows[-1], logits_rows=len(prompt))
    assert np.array_equal(b_rows, rows[1:]) and b_ids == f_ids and np.array_equal(b_logits, f_logits)
    # one decode row through the split
    d_ids, d_logits = full.forward([f_ids[-1]], 1)
    a_rows, _, _ = a.forward_range(0, 1, tokens=[f_ids[-1]])
    _, s_ids, s_logits = b.forward_range(1, 3, rows=a_rows[-1], logits_rows=1)
    assert s_ids == d_ids and np.array_equal(s_logits, d_logits)
    assert a.position() == b.position() == len(prompt) + 1
    with pytest.raises(ValueError):
        b.forward_range(1, 3, tokens=[1])  # a later stage takes rows, not ids
    with pytest.raises(ValueError):
        a.forward_range(0, 1, tokens=[1], logits_rows=1)  # logits only from the last stage


def test_model_slices_hold_their_layer_range():
    cfg = jf.ModelConfig(n_layer=3, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=300, n_ctx=128)
    model = jf.Model.synthesize(cfg, type_linear=jo.Q4_K, type_embd=jo.Q4_K, type_output=jo.Q6_K, seed=3)
    for start, end in ((0, 1), (1, 2), (2, 3), (0, 3), (1, 3)):
        part = model.slice(start, end)
        names = set(part.tensor_names())
        assert ("token_embd.weight" in names) == (start == 0)
        assert ("output.weight" in names) == ("output_norm.weight" in names) == (end == 3)
        layers = {int(n.split(".")[1]) for n in names if n.startswith("blk.")}
        assert layers == set(range(start, end))
        for n in names:
            assert part.tensor_bytes(n) == model.tensor_bytes(n)
        assert part.stats()["layer_start"] == start and part.stats()["layer_end"] == end
        assert part.source_sha256() == model.source_sha256()
    inner = model.slice(1, 3).slice(2, 3)
    assert set(inner.tensor_names()) == set(model.slice(2, 3).tensor_names())
    for start, end in ((1, 1), (2, 1), (0, 4)):
        with pytest.raises(jf.JfhError):
            model.slice(start, end)
    with pytest.raises(jf.JfhError):
        model.slice(1, 3).slice(0, 2)  # outside the slice's own range


def test_capacity_and_vocabulary_errors():
    model = _q4k_model()
    s = jo.OracleModel.from_model(model).session(8, jo.MODE_Q8, 1)
    with pytest.raises(ValueError, match="capacity"):
        s.forward(list(range(9)), 1)
    with pytest.raises(ValueError, match="vocabulary"):
        s.forward([300], 1)


def test_tensor_overrides():
    model = _q4k_model()
    prompt = [5, 17, 99, 3, 250, 7]
    gain = np.frombuffer(model.tensor_bytes("blk.0.attn_norm.weight"), dtype=np.float32).copy()
    _, base = jo.OracleModel.from_model(model).session(16, jo.MODE_Q8, 1).forward(prompt, 1)
    _, same = jo.OracleModel.from_model(model, {"blk.0.attn_norm.weight": gain}).session(16, jo.MODE_Q8, 1).forward(
        prompt, 1)
    assert np.array_equal(base, same)
    gain[3] *= np.float32(1.5)
    _, moved = jo.OracleModel.from_model(model, {"blk.0.attn_norm.weight": gain}).session(16, jo.MODE_Q8, 1).forward(
        prompt, 1)
    assert not np.array_equal(base, moved)
    with pytest.raises(ValueError, match="float32 of shape"):
        jo.OracleModel.from_model(model, {"blk.0.attn_norm.weight": gain[:10]})
    with pytest.raises(ValueError, match="float32 of shape"):
        jo.OracleModel.from_model(model, {"blk.0.attn_q.weight": np.zeros(256 * 256, np.float32)})


def test_quantized_activation_mode_stays_close_to_exact():
    model = _q4k_model()
    om = jo.OracleModel.from_model(model)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, 300, 20)]
    _, lq = om.session(32, jo.MODE_Q8, 2).forward(prompt, 1)
    _, le = om.session(32, jo.MODE_EXACT, 2).forward(prompt, 1)
    # the reference's own logit gates for quantized backends (tools/bench/native_engine_matrix.py:341-342)
    assert jo.nrmse(le[0], lq[0]) <= 0.025
    assert jo.cosine(le[0], lq[0]) >= 0.999


def test_speculative_loop_is_greedy_invariant():
    model = _q4k_model(9)
    om = jo.OracleModel.from_model(model)
    rng = np.random.default_rng(1)
    seg = [int(t) for t in rng.integers(0, 300, 12)]
    prompt = seg + seg + seg[:6]
    serial = greedy(om.session(128, jo.MODE_Q8, 2), prompt, 24)

    s = om.session(128, jo.MODE_Q8, 2)
    out, stats = jo.speculative_generate(lambda p: s.forward(p, 1)[0][0], lambda rows: s.forward(rows, len(rows))[0],
                                         s.rollback, prompt, 24, 4, 4, 2)
    assert out == serial
    assert stats["target_decode_passes"] <= 24
    assert stats["speculative_accepted_tokens"] <= stats["speculative_draft_tokens"]


def test_speculative_loop_reference_harness_case():
    """generation_runner_test.cpp:355-389: history [1,2,1,2,10], a fixed draft
    [20,21] and a target that answers [20,99,30] emit [10,20,99] in one pass
    with one rejected token rolled back."""
    rollbacks = []

    def fixed_draft(history, budget):
        return [20, 21] if history == [1, 2, 1, 2, 10] else []

    out, stats = jo.speculative_generate(lambda p: 10, lambda rows: [20, 99, 30][:len(rows)], rollbacks.append,
                                         [1, 2, 1, 2], 3, 2, propose=fixed_draft)
    assert out == [10, 20, 99]
    assert stats["target_decode_passes"] == 1
    assert stats["speculative_draft_tokens"] == 2 and stats["speculative_accepted_tokens"] == 1
    assert rollbacks == [1]


def test_argmax_first_maximum():
    x = np.array([1.0, 3.0, -2.0, 3.0, 3.0], dtype=np.float32)
    assert jo.argmax(x) == 1
    assert jo.argmax(np.full(7, -np.inf, dtype=np.float32)) == 0


# ------------------------------------------------------------------ prompt lookup

def test_prompt_lookup_reference_known_answers():
    for propose in (jo.prompt_lookup, jf.prompt_lookup_propose):
        assert propose([1, 2, 3, 1, 2, 3, 1, 2], 3) == [3, 1, 2]
        assert propose([1, 2, 3, 4], 3) == []
        assert propose([1, 2, 1, 2], 0) == []
    with pytest.raises(ValueError):
        jo.prompt_lookup([1, 2, 3], 2, max_ngram=1, min_ngram=2)
    with pytest.raises(ValueError):
        jf.prompt_lookup_propose([1, 2, 3], 2, max_ngram=1, min_ngram=2)


def brute_force_lookup(history, max_tokens, max_ngram, min_ngram):
    """Longest suffix n-gram (<= max, >= min) with an earlier occurrence that
    ends at or before the suffix start; the latest such occurrence wins."""
    if max_tokens == 0:
        return []
    n = len(history)
    for g in range(min(max_ngram, n - 1), min_ngram - 1, -1):
        suffix = history[n - g:]
        starts = [c for c in range(0, n - g) if c + g <= n - g and history[c:c + g] == suffix]
        if starts:
            c = max(starts)
            return history[c + g:c + g + max_tokens]
    return []


def test_prompt_lookup_matches_brute_force_and_the_c_abi():
    rng = np.random.default_rng(7)
    for trial in range(300):
        n = int(rng.integers(0, 40))
        hist = [int(t) for t in rng.integers(0, 4 if trial % 2 else 9, n)]
        k = int(rng.integers(0, 6))
        hi = int(rng.integers(2, 6))
        lo = int(rng.integers(1, hi + 1))
        expected = brute_force_lookup(hist, k, hi, lo)
        assert jo.prompt_lookup(hist, k, hi, lo) == expected, (hist, k, hi, lo)
        assert jf.prompt_lookup_propose(hist, k, hi, lo) == expected, (hist, k, hi, lo)


# ------------------------------------------------------------------ RoPE table

def test_rope_table_closed_form():
    base, hd = 1.0e6, 128
    t = jo.rope_table(base, hd, 0, 4096)
    pos = np.arange(4096)[:, None].astype(np.float64)
    inv = base ** (-2.0 * np.arange(hd // 2) / hd)
    ang = pos * inv[None, :]
    assert np.all(t[0, 0::2] == 1.0) and np.all(t[0, 1::2] == 0.0)  # position 0: identity
    # theta advanced by repeated float multiplication (GGML's rope cache): small drift only
    assert np.abs(t[:, 0::2] - np.cos(ang)).max() < 2e-3
    assert np.abs(t[:, 1::2] - np.sin(ang)).max() < 2e-3
    assert np.allclose(t[:, 0::2] ** 2 + t[:, 1::2] ** 2, 1.0, atol=1e-6)  # rotations preserve norms
    tail = jo.rope_table(base, hd, 1000, 8)
    assert np.array_equal(tail, t[1000:1008])


_HOST_BUILD_SCRIPT = """
import sys
import numpy as np
import oracle as jo
jo.use_library(sys.argv[1])
from tests.test_oracle_forward import _q4k_model
model = _q4k_model()
om = jo.OracleModel.from_model(model)
out = []
for mode in (jo.MODE_Q8, jo.MODE_EXACT):
    s = om.session(64, mode, 2)
    out.append(s.forward([5, 17, 99, 3, 250, 7, 7, 12], 8)[1])
np.save(sys.argv[2], np.stack(out))
"""


def test_host_tuned_build_gives_the_same_logits(tmp_path):
    """The -march=native build that bench.py times computes exactly what the portable build does."""
    import os
    import subprocess
    import sys
    lib = jo.build_native(str(tmp_path))
    out = tmp_path / "logits.npy"
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.run([sys.executable, "-c", _HOST_BUILD_SCRIPT, lib, str(out)], check=True, cwd=root)
    model = _q4k_model()
    om = jo.OracleModel.from_model(model)
    want = []
    for mode in (jo.MODE_Q8, jo.MODE_EXACT):
        s = om.session(64, mode, 2)
        want.append(s.forward([5, 17, 99, 3, 250, 7, 7, 12], 8)[1])
    want = np.stack(want)
    assert np.isfinite(want).all()
    assert np.array_equal(np.load(out), want)
