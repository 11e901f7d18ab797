"""GPU parity of the HIP engine against the CPU oracle, through the C ABI.

Bars: bit-exact for dequantization and integer/index work; the matmul on
identical int8 activations differs only in f32 summation order (rtol 1e-4).
Whole-model logits: the GPU's RMSNorm/softmax/SwiGLU results differ from the
oracle's in the last ulp, which occasionally moves one int8 activation by one
step; logits therefore carry an error of ~1e-3. The bound used here, NRMSE
<= 5e-3 and cosine >= 0.9995, is 5x tighter than the reference's own logit
gates (NRMSE <= 0.025, cosine >= 0.999: tools/bench/native_engine_matrix.py:
341-342). Greedy ids must match unless the oracle's top two logits are within
that error (a near tie), which the helper reports.
"""
from __future__ import annotations

import numpy as np
import pytest

import jetsonfabric_amd as jf
import oracle as jo
from tests.golden import tiny_fixture

pytestmark = pytest.mark.gpu

SMALL = jf.ModelConfig(n_layer=3, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=8192, n_ctx=2048)
TYPES = [jf.Q4_K, jf.Q6_K, jf.Q8_0, jf.Q2_K]


NRMSE_MAX = 5e-3
COSINE_MIN = 0.9995


def assert_logits_match(ref: np.ndarray, gpu: np.ndarray, gpu_id: int, where: str = "") -> None:
    assert jo.nrmse(ref, gpu) <= NRMSE_MAX, f"{where} nrmse {jo.nrmse(ref, gpu):.2e}"
    assert jo.cosine(ref, gpu) >= COSINE_MIN, f"{where} cosine {jo.cosine(ref, gpu):.6f}"
    best = int(np.argmax(ref))
    if gpu_id != best:
        margin = float(ref[best] - ref[gpu_id])
        assert margin <= NRMSE_MAX * float(ref.max() - ref.min()), f"{where} greedy {gpu_id} vs {best} (margin {margin})"


def _model(cfg, linear, embd, out, seed=3, tied=False, bias=False):
    return jf.Model.synthesize(cfg, type_linear=linear, type_embd=embd, type_output=out, seed=seed,
                               tied_output=tied, output_bias=bias)


@pytest.fixture(scope="module", params=TYPES, ids=[jf.TYPE_NAMES[t] for t in TYPES])
def typed(request):
    t = request.param
    model = _model(SMALL, t, t, t, seed=10 + t)
    engine = jf.NativeEngine(model)
    yield t, model, engine
    engine.close()


@pytest.fixture(scope="module")
def q4k():
    model = _model(SMALL, jf.Q4_K, jf.Q4_K, jf.Q6_K, seed=21, bias=True)
    engine = jf.NativeEngine(model)
    yield model, engine, jo.OracleModel.from_model(model)
    engine.close()


def test_dequantize_bit_exact(typed):
    t, model, engine = typed
    for name in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight", "output.weight"):
        info = model.tensor(name)
        cols, rows = info["shape"]
        n = min(rows, 96)
        gpu = engine.dequantize_rows(name, rows - n, n, cols)
        raw = model.tensor_bytes(name)
        rb = jo.row_bytes(t, cols)
        for i in range(n):
            r = rows - n + i
            ref = jo.dequantize_row(t, raw[r * rb:(r + 1) * rb], cols)
            assert np.array_equal(gpu[i].view(np.uint32), ref.view(np.uint32)), f"{name} row {r}"


@pytest.mark.parametrize("n_tok", [1, 2, 3, 5, 8, 9, 16, 40, 64])
def test_matmul_matches_oracle(typed, n_tok):
    t, model, engine = typed
    rng = np.random.default_rng(n_tok)
    for name in ("blk.0.attn_q.weight", "blk.2.ffn_down.weight", "blk.1.attn_output.weight"):
        info = model.tensor(name)
        cols, rows = info["shape"]
        x = rng.standard_normal((n_tok, cols)).astype(np.float32)
        gpu = engine.matmul(name, x, rows)
        ref = jo.matmul(t, info["data"], cols, rows, x, jo.MODE_Q8)
        # identical int8 activations and integer dots; only f32 summation order differs
        scale = np.abs(ref).max()
        assert np.allclose(gpu, ref, rtol=1e-4, atol=2e-5 * scale), f"{name} max err {np.abs(gpu - ref).max():.3e}"
        exact = jo.matmul(t, info["data"], cols, rows, x, jo.MODE_EXACT)
        assert jo.nrmse(exact, gpu) < 1e-2


@pytest.mark.parametrize("n_tok", [3, 4, 5, 8, 9, 16, 17, 33, 64, 100, 128, 256])
def test_wide_matmul_rows_equal_single_rows(typed, n_tok):
    """Steps of 3 or more int8 rows run every quantized format on matrix cores
    (token quads below the format's wide threshold, 9 rows for Q4_K / Q8_0 and
    17 for Q6_K / Q2_K, the wide kernel from there, in 16-token tiles); every
    row must equal the same row computed alone (the decode path), bit for bit."""
    t, model, engine = typed
    rng = np.random.default_rng(100 + n_tok)
    for name in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight", "blk.2.attn_output.weight"):
        cols, rows = model.tensor(name)["shape"]
        x = rng.standard_normal((n_tok, cols)).astype(np.float32)
        wide = engine.matmul(name, x, rows)
        for r in range(n_tok):
            single = engine.matmul(name, x[r:r + 1], rows)
            assert np.array_equal(wide[r].view(np.uint32), single[0].view(np.uint32)), f"{name} row {r}"


# A gate/up matrix of 8192 rows (512 row groups): steps of 9..256 rows run the
# wide K-quant matmuls that share activation loads between row groups (Q4_K on
# the folded-scale tile, Q6_K and Q2_K with two or four row groups per
# work-group).
WIDE = jf.ModelConfig(n_layer=1, n_embd=512, n_ff=4096, n_head=8, n_head_kv=2, n_vocab=4096, n_ctx=256)
KQUANTS = [jf.Q4_K, jf.Q6_K, jf.Q2_K]


@pytest.fixture(scope="module", params=KQUANTS, ids=[jf.TYPE_NAMES[t] for t in KQUANTS])
def wide_typed(request):
    t = request.param
    model = _model(WIDE, t, t, t, seed=40 + t)
    engine = jf.NativeEngine(model)
    yield t, model, engine
    engine.close()


def test_wide_matmul_over_row_group_sets_equals_single_rows(wide_typed):
    """The wide matmul that shares each activation load between two or four
    row groups per work-group: every row of a wide step (9, 17, 33, 64, 128 and 256 rows;
    Q6_K and Q2_K run token quads below 17) equals the same row computed alone
    (the decode path), bit for bit, and the step matches the oracle's matmul on
    the same int8 rows."""
    t, model, engine = wide_typed
    name = "blk.0.ffn_gate.weight"
    info = model.tensor(name)
    cols, rows = info["shape"]
    for n_tok in ([9] if t == jf.Q4_K else []) + [17, 33, 64, 128, 256]:
        rng = np.random.default_rng(300 + n_tok)
        x = rng.standard_normal((n_tok, cols)).astype(np.float32)
        wide = engine.matmul(name, x, rows)
        for r in range(n_tok):
            single = engine.matmul(name, x[r:r + 1], rows)
            assert np.array_equal(wide[r].view(np.uint32), single[0].view(np.uint32)), f"{n_tok} rows: row {r}"
        ref = jo.matmul(t, info["data"], cols, rows, x, jo.MODE_Q8)
        # identical int8 activations and integer dots; only f32 summation order differs
        scale = np.abs(ref).max()
        assert np.allclose(wide, ref, rtol=1e-4, atol=2e-5 * scale), f"{n_tok} rows: max err {np.abs(wide - ref).max():.3e}"


# A Q4_K gate/up matrix of 16384 rows (256 sets of four row groups) over K =
# 2560 (ten tiles: the decode waves' chains of two and one tiles): steps of
# 9..256 rows run the whole-K-wave kernel that folds the sub-block scales into
# the weight operand and shares each activation tile through LDS (steps of more
# than 64 rows as several token groups of four 16-token tiles).
WIDE_Q4 = jf.ModelConfig(n_layer=1, n_embd=2560, n_ff=8192, n_head=20, n_head_kv=4, n_vocab=4096, n_ctx=512)


@pytest.fixture(scope="module")
def wide_q4():
    model = _model(WIDE_Q4, jf.Q4_K, jf.Q4_K, jf.Q6_K, seed=77, bias=True)
    engine = jf.NativeEngine(model)
    yield model, engine, jo.OracleModel.from_model(model)
    engine.close()


def test_folded_scale_wide_matmul_equals_single_rows(wide_q4):
    """Every row of a 9..256-row step through the folded-scale kernel equals the
    same row computed alone (the decode path), bit for bit, and the step
    matches the oracle's matmul on the same int8 rows."""
    model, engine, _ = wide_q4
    name = "blk.0.ffn_gate.weight"
    info = model.tensor(name)
    cols, rows = info["shape"]
    for n_tok in (9, 17, 33, 48, 64, 80, 128, 200, 256):
        rng = np.random.default_rng(500 + n_tok)
        x = rng.standard_normal((n_tok, cols)).astype(np.float32)
        wide = engine.matmul(name, x, rows)
        for r in range(n_tok):
            single = engine.matmul(name, x[r:r + 1], rows)
            assert np.array_equal(wide[r].view(np.uint32), single[0].view(np.uint32)), f"{n_tok} rows: row {r}"
        ref = jo.matmul(jf.Q4_K, info["data"], cols, rows, x, jo.MODE_Q8)
        scale = np.abs(ref).max()
        assert np.allclose(wide, ref, rtol=1e-4, atol=2e-5 * scale), f"{n_tok} rows: max err {np.abs(wide - ref).max():.3e}"


def test_folded_scale_prefill_matches_oracle_and_token_by_token(wide_q4):
    """A 300-token prompt (chunks of 256 and 44 rows: the SwiGLU gate/up
    matrix on the folded-scale kernel) matches the oracle's logits, and a
    session fed the prompt one token at a time reaches the same greedy
    continuation."""
    model, engine, om = wide_q4
    prompt = _prompt(300, WIDE_Q4.n_vocab, 31)
    s = engine.create_session(350)
    ref = om.session(350, jo.MODE_Q8)
    tok, lg = s.prefill_greedy(prompt, logits=True)
    _, rl = ref.forward(prompt, 1)
    assert_logits_match(rl[0], lg, tok, "chunked prefill")
    one = engine.create_session(350)
    first = one.prefill_greedy(prompt[:1])
    for t in prompt[1:]:
        first = one.decode_greedy(t)
    assert first == tok
    a, b = [tok], [first]
    for _ in range(4):
        a.append(s.decode_greedy(a[-1]))
        b.append(one.decode_greedy(b[-1]))
    assert a == b


def test_tiny_fixture_known_answer():
    cfg = jf.ModelConfig(**tiny_fixture.CONFIG)
    model = jf.Model.build(cfg, tiny_fixture.tensors())
    engine = jf.NativeEngine(model)
    assert engine.generate([2], 2).sampled_tokens == tiny_fixture.EXPECTED[(2,)]
    s = engine.create_session(2)
    assert s.prefill_greedy([2, 2]) == tiny_fixture.EXPECTED[(2, 2)][0]
    engine.close()


def _prompt(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def test_forward_matches_oracle(q4k):
    model, engine, om = q4k
    prompt = _prompt(40, SMALL.n_vocab, 1)
    s = engine.create_session(64)
    ref = om.session(64, jo.MODE_Q8)
    tok, logits = s.prefill_greedy(prompt, logits=True)
    _, ref_logits = ref.forward(prompt, 1)
    assert_logits_match(ref_logits[0], logits, tok, "prefill")
    for step in range(8):
        nxt, lg = s.decode_greedy(tok, logits=True)
        _, rl = ref.forward([tok], 1)
        assert_logits_match(rl[0], lg, nxt, f"decode step {step}")
        tok = nxt


def test_chunked_prefill_matches_oracle_and_token_by_token(q4k):
    """A 300-token prompt is prefilled in chunks of up to 256 rows (matrix-core
    matmuls); its logits match the oracle's, and a session fed the same
    prompt one token at a time reaches the same greedy continuation."""
    model, engine, om = q4k
    prompt = _prompt(300, SMALL.n_vocab, 12)
    s = engine.create_session(350)
    ref = om.session(350, jo.MODE_Q8)
    tok, lg = s.prefill_greedy(prompt, logits=True)
    _, rl = ref.forward(prompt, 1)
    assert_logits_match(rl[0], lg, tok, "chunked prefill")
    one = engine.create_session(350)
    first = one.prefill_greedy(prompt[:1])
    for t in prompt[1:]:
        first = one.decode_greedy(t)
    assert first == tok
    a, b = [tok], [first]
    for _ in range(6):
        a.append(s.decode_greedy(a[-1]))
        b.append(one.decode_greedy(b[-1]))
    assert a == b


@pytest.mark.parametrize("types", [(jf.Q4_K, jf.Q8_0, jf.Q8_0, True), (jf.Q2_K, jf.Q2_K, jf.Q6_K, False),
                                   (jf.Q8_0, jf.Q8_0, jf.Q6_K, False)], ids=["q4k-q80-tied", "q2k-q6k", "q80-q6k"])
def test_forward_mixed_types(types):
    linear, embd, out, tied = types
    model = _model(SMALL, linear, embd, out, seed=5, tied=tied)
    engine = jf.NativeEngine(model)
    om = jo.OracleModel.from_model(model)
    prompt = _prompt(17, SMALL.n_vocab, 2)
    s = engine.create_session(32)
    ref = om.session(32, jo.MODE_Q8)
    tok, lg = s.prefill_greedy(prompt, logits=True)
    _, rl = ref.forward(prompt, 1)
    assert_logits_match(rl[0], lg, tok, "prefill")
    nxt, lg = s.decode_greedy(tok, logits=True)
    _, rl = ref.forward([tok], 1)
    assert_logits_match(rl[0], lg, nxt, "decode")
    engine.close()


def test_verify_equals_serial_and_rollback_replay(q4k):
    model, engine, _ = q4k
    prompt = _prompt(30, SMALL.n_vocab, 3)
    serial_s = engine.create_session(64)
    serial = [serial_s.prefill_greedy(prompt)]
    for _ in range(6):
        serial.append(serial_s.decode_greedy(serial[-1]))
    v = engine.create_session(64)
    assert v.prefill_greedy(prompt) == serial[0]
    ids, accepted = v.verify(serial[:5])
    assert ids == serial[1:6] and accepted == 4
    assert v.position() == len(prompt) + 5
    # a wrong draft: accept the matching prefix, roll back the rest, replay the correction
    w = engine.create_session(64)
    w.prefill_greedy(prompt)
    draft = [serial[0], serial[1], serial[2], (serial[3] + 1) % SMALL.n_vocab, 5]
    ids, accepted = w.verify(draft)
    assert ids[:3] == serial[1:4] and accepted == 2
    w.rollback(len(draft) - 1 - accepted)
    assert w.position() == len(prompt) + 3
    assert w.decode_greedy(ids[accepted]) == serial[4]


def test_batch_step_equals_individual(q4k):
    model, engine, _ = q4k
    prompts = [_prompt(n, SMALL.n_vocab, 40 + n) for n in (9, 21, 14)]
    rows = []
    singles = []
    for p in prompts:
        s = engine.create_session(64)
        first = s.prefill_greedy(p)
        rows.append(s)
        singles.append(first)
    inputs = [[singles[0]], [singles[1], 7, 8], [singles[2], 11]]
    ids, _ = engine.step_batch(rows, inputs)
    for p, row, got in zip(prompts, inputs, ids):
        s = engine.create_session(64)
        s.prefill_greedy(p)
        if len(row) == 1:
            assert got == [s.decode_greedy(row[0])]
        else:
            assert got == s.verify(row)[0]


def test_long_context_decode_matches_oracle(q4k):
    model, engine, om = q4k
    prompt = _prompt(700, SMALL.n_vocab, 4)
    s = engine.create_session(720)
    ref = om.session(720, jo.MODE_Q8)
    tok, lg = s.prefill_greedy(prompt, logits=True)
    _, rl = ref.forward(prompt, 1)
    assert_logits_match(rl[0], lg, tok, "prefill")
    for step in range(3):
        nxt, lg = s.decode_greedy(tok, logits=True)
        _, rl = ref.forward([tok], 1)
        assert_logits_match(rl[0], lg, nxt, f"decode step {step}")
        tok = nxt


def test_speculative_generation_is_greedy_invariant(q4k):
    model, engine, _ = q4k
    seg = _prompt(16, SMALL.n_vocab, 6)
    prompt = seg + seg + seg  # repetitive: prompt lookup finds drafts
    plain = engine.generate(prompt, 24, draft_max=0)
    spec = engine.generate(prompt, 24, draft_max=4, max_ngram=3, min_ngram=3)
    assert spec.sampled_tokens == plain.sampled_tokens
    assert spec.target_decode_passes <= plain.target_decode_passes
    # the same loop restated in the oracle, driven by the engine's session calls
    s = engine.create_session(len(prompt) + 24)
    out, stats = jo.speculative_generate(lambda p: s.prefill_greedy(p), lambda v: s.verify(v)[0] if len(v) > 1 else
                                         [s.decode_greedy(v[0])], s.rollback, prompt, 24, 4, 3, 3)
    assert out == spec.sampled_tokens
    assert stats["target_decode_passes"] == spec.target_decode_passes
    assert stats["speculative_draft_tokens"] == spec.speculative_draft_tokens
    assert stats["speculative_accepted_tokens"] == spec.speculative_accepted_tokens


@pytest.mark.parametrize("draft", [0, 4])
def test_concurrent_generation_equals_each_alone(q4k, draft):
    """Continuous batching of 3 runners (decode steps coalesced into one
    multi-sequence forward) produces every request's tokens and speculation
    counters exactly as that request generated alone."""
    model, engine, _ = q4k
    prompts = []
    for i in range(3):
        seg = _prompt(12 + 2 * i, SMALL.n_vocab, 40 + i)
        prompts.append(seg + seg + seg[: 5 + i])  # repetitive: prompt lookup finds drafts
    results, wall_ms = engine.generate_concurrent(prompts, 20, draft_max=draft, max_ngram=3, min_ngram=3,
                                                  batch_wait_us=2000)
    assert wall_ms > 0.0
    for prompt, got in zip(prompts, results):
        alone = engine.generate(prompt, 20, draft_max=draft, max_ngram=3, min_ngram=3)
        assert got.sampled_tokens == alone.sampled_tokens
        assert got.target_decode_passes == alone.target_decode_passes
        assert got.speculative_accepted_tokens == alone.speculative_accepted_tokens
    if draft:
        assert sum(r.speculative_accepted_tokens for r in results) > 0


def test_invalid_inputs_raise(q4k):
    model, engine, _ = q4k
    s = engine.create_session(8)
    with pytest.raises(jf.InvalidArgument):
        s.decode_greedy(1)  # decode before prefill
    with pytest.raises(jf.InvalidArgument):
        s.prefill_greedy([SMALL.n_vocab])  # token outside the vocabulary
    with pytest.raises(jf.InvalidArgument):
        s.prefill_greedy(list(range(9)))  # beyond capacity
    s.prefill_greedy([1, 2, 3])
    with pytest.raises(jf.InvalidArgument):
        s.rollback(1)  # nothing decoded yet
    with pytest.raises(jf.InvalidArgument):
        engine.create_session(SMALL.n_ctx + 1)
