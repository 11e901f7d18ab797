"""Generation with a caller's draft strategy and the generation metrics, through the C ABI.

jfh_generate_draft runs GenerationRunner::run (generation_runner.cpp:469-556)
with any DraftStrategy (draft_strategy.hpp:9-17), as the reference's harness
installs FixedDraft (generation_runner_test.cpp:108-119). Greedy speculation
never changes the tokens: with the model's own continuation as the draft every
token is accepted and the passes drop to one per k + 1 tokens; with wrong
drafts nothing is accepted and every rejected pass is followed by a recovery
pass. The statistics carry GenerationResult's rates, PrefillMetrics and
ExecutionBufferMetrics (native_inference.hpp:71-96).
"""
from __future__ import annotations

import numpy as np
import pytest

import jetsonfabric_amd as jf

pytestmark = pytest.mark.gpu

CFG = jf.ModelConfig(n_layer=2, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=4096, n_ctx=1024)
K = 4


@pytest.fixture(scope="module")
def engine():
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=91)
    eng = jf.NativeEngine(model)
    yield eng
    eng.close()
    model.close()


def _prompt(n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, CFG.n_vocab, n)]


class Recorded:
    """Proposes the recorded greedy continuation after the history; position j
    of a draft is replaced by a wrong id when wrong(pass, j)."""

    def __init__(self, prompt_len, tokens, wrong=lambda p, j: False):
        self.prompt_len, self.tokens, self.wrong = prompt_len, tokens, wrong
        self.calls = 0

    def __call__(self, history, max_tokens):
        i = len(history) - self.prompt_len  # tokens generated so far
        truth = self.tokens[i:i + max_tokens]
        out = [(t + 1 + j) % CFG.n_vocab if self.wrong(self.calls, j) else t for j, t in enumerate(truth)]
        self.calls += 1
        return out


def test_caller_draft_with_the_true_continuation_is_fully_accepted(engine):
    prompt = _prompt(40, 1)
    n = 25
    plain = engine.generate(prompt, n)
    assert len(plain.sampled_tokens) == n and plain.speculative_draft_tokens == 0
    spec = engine.generate_with_draft(prompt, n, K, Recorded(len(prompt), plain.sampled_tokens))
    assert spec.sampled_tokens == plain.sampled_tokens
    assert spec.speculative_accepted_tokens == spec.speculative_draft_tokens > 0
    # the prefill gives token 1; each pass then brings its k accepted drafts plus the target's own token
    # (the last draft is shortened to the tokens still missing)
    assert spec.target_decode_passes == -(-(n - 1) // (K + 1))
    assert spec.target_decode_passes < plain.target_decode_passes == n - 1


def test_caller_draft_with_wrong_tokens_is_rejected_and_recovers(engine):
    prompt = _prompt(40, 2)
    n = 17
    plain = engine.generate(prompt, n)
    strategy = Recorded(len(prompt), plain.sampled_tokens, wrong=lambda p, j: True)
    spec = engine.generate_with_draft(prompt, n, K, strategy)
    assert spec.sampled_tokens == plain.sampled_tokens
    assert spec.speculative_accepted_tokens == 0 and spec.speculative_draft_tokens > 0
    # a rejected verify pass emits the target's token, then a recovery pass (no draft) emits one more
    assert spec.target_decode_passes == n - 1
    assert strategy.calls == -(-(n - 1) // 2)


def test_caller_draft_at_a_seeded_acceptance_rate_keeps_greedy_tokens(engine):
    prompt = _prompt(64, 3)
    n = 60
    plain = engine.generate(prompt, n)
    rng = np.random.default_rng(5)
    flips = rng.random((200, K)) > 0.7
    spec = engine.generate_with_draft(prompt, n, K,
                                      Recorded(len(prompt), plain.sampled_tokens, wrong=lambda p, j: flips[p, j]))
    assert spec.sampled_tokens == plain.sampled_tokens
    assert 0 < spec.speculative_accepted_tokens < spec.speculative_draft_tokens
    assert spec.target_decode_passes < plain.target_decode_passes


def test_failing_draft_strategy_proposes_nothing(engine):
    prompt = _prompt(30, 4)
    plain = engine.generate(prompt, 9)

    def broken(history, max_tokens):
        raise RuntimeError("no draft")

    spec = engine.generate_with_draft(prompt, 9, K, broken)
    assert spec.sampled_tokens == plain.sampled_tokens and spec.speculative_draft_tokens == 0


def test_generation_metrics(engine):
    prompt = _prompt(300, 6)  # several prefill chunks
    n = 12
    first = engine.generate(prompt, n)
    again = engine.generate(prompt, n)
    for r in (first, again):
        decoded = len(r.sampled_tokens) - 1
        assert r.inter_token_latency_ms == pytest.approx(r.decode_ms / decoded, rel=1e-9)
        assert r.decode_tokens_per_second == pytest.approx(decoded / (r.decode_ms * 1e-3), rel=1e-9)
        total = (r.time_to_first_token_ms + r.decode_ms) * 1e-3
        assert r.end_to_end_tokens_per_second == pytest.approx(len(r.sampled_tokens) / total, rel=1e-9)
        pf = r.prefill
        assert pf["compute_ms"] > 0.0 and pf["host_input_preparation_ms"] > 0.0 and pf["output_read_ms"] >= 0.0
        assert pf["allocation_ms"] > 0.0
        assert pf["attention_matrix_cores"]  # head dim 64
        # device and host parts of the prefill fit inside the time to the first token
        assert pf["compute_ms"] + pf["planning_ms"] <= r.time_to_first_token_ms * 1.05 + 0.05
        b = r.buffers
        chunks = -(-len(prompt) // engine.prefill_chunk)
        assert b["prefill_host_input_bytes"] >= chunks * 1000  # one step descriptor per chunk
        # the session the runner opened: capacity prompt + n rounded up to 16 positions, F16 K and V
        stride = -(-(len(prompt) + n) // 16) * 16
        assert b["kv_cache_bytes"] == 2 * CFG.n_layer * CFG.n_head_kv * stride * (CFG.n_embd // CFG.n_head) * 2
        assert b["prefill_scratch_bytes"] == min(engine.prefill_chunk, len(prompt)) * b["decode_scratch_bytes"] > 0
    # the second run replays the step graphs the first one captured
    assert again.prefill["plan_reused"] and again.prefill["planning_ms"] == 0.0
    assert first.sampled_tokens == again.sampled_tokens


def test_concurrent_generation_reports_metrics_per_request(engine):
    prompts = [_prompt(70, 10 + i) for i in range(2)]
    results, wall = engine.generate_concurrent(prompts, 8)
    for r in results:
        assert r.prefill["compute_ms"] > 0.0 and r.buffers["kv_cache_bytes"] > 0
        assert r.decode_tokens_per_second > 0.0
