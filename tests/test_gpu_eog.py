"""End-of-generation ids in the on-GPU acceptance and in generation, through the C ABI.

The rule (runtime/pipeline_parallel/generation_runner.cpp:512-517): draft
token j is accepted while the target's greedy id after row j equals it and is
not an end-of-generation id; generation ends, finish reason "stop", at the
first end id the target samples (generation_runner.cpp:540-560), which is not
emitted. The verify rows here are the model's own greedy continuation, so
without end ids every draft token is accepted and an end id at draft position
e cuts the accepted length to e exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

import jetsonfabric_amd as jf
from jetsonfabric_amd._capi import InvalidArgument

pytestmark = pytest.mark.gpu

CFG = jf.ModelConfig(n_layer=2, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=4096, n_ctx=1024)
K = 4


@pytest.fixture(scope="module")
def engine():
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=77)
    eng = jf.NativeEngine(model)
    yield eng
    eng.set_end_tokens([])
    eng.close()
    model.close()


def _prompt(n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, CFG.n_vocab, n)]


def _continuation(session, tok, n):
    """The greedy continuation [tok, c1..cn] from the session's position (restored afterwards)."""
    cont = [tok]
    for _ in range(n):
        cont.append(session.decode_greedy(cont[-1]))
    session.rollback(n)
    return cont


def _rule(ids, draft, ends):
    accepted = 0
    while accepted < len(draft) and ids[accepted] not in ends and ids[accepted] == draft[accepted]:
        accepted += 1
    return accepted


def test_verify_acceptance_stops_at_end_token(engine):
    s = engine.create_session(128)
    tok = s.prefill_greedy(_prompt(24, 1))
    cont = _continuation(s, tok, K + 1)
    rows = cont[:K + 1]
    engine.set_end_tokens([])
    ids, acc = s.verify(rows)
    assert ids == cont[1:K + 2], "verify of the greedy continuation must reproduce serial decode"
    assert acc == K
    s.rollback(K + 1)
    for e in range(K):
        end = cont[1 + e]  # the greedy id after row e, equal to draft token e
        engine.set_end_tokens([end])
        ids, acc = s.verify(rows)
        assert acc == _rule(ids, rows[1:], {end})
        if end not in cont[1:1 + e]:
            assert acc == e, f"end id at draft position {e}: accepted {acc}"
        s.rollback(K + 1)
    # an end id that is no greedy id of these rows leaves the acceptance alone
    other = next(t for t in range(CFG.n_vocab) if t not in cont)
    engine.set_end_tokens([other, other + 1 if other + 1 not in cont else other])
    _, acc = s.verify(rows)
    assert acc == K
    s.rollback(K + 1)
    engine.set_end_tokens([])
    s.close()


def test_batched_acceptance_stops_at_end_token(engine):
    sessions = [engine.create_session(128) for _ in range(2)]
    conts = []
    for i, s in enumerate(sessions):
        tok = s.prefill_greedy(_prompt(20 + 5 * i, 10 + i))
        conts.append(_continuation(s, tok, K + 1))
    rows = [c[:K + 1] for c in conts]
    end = conts[0][3]  # draft position 2 of the first sequence
    engine.set_end_tokens([end])
    ids, acc = engine.step_batch(sessions, rows)
    for i in range(2):
        assert ids[i] == conts[i][1:K + 2]
        assert acc[i] == _rule(ids[i], rows[i][1:], {end})
    if end not in conts[0][1:3]:
        assert acc[0] == 2
    engine.set_end_tokens([])
    for s in sessions:
        s.close()


@pytest.mark.parametrize("draft", [0, K])
def test_generation_ends_at_end_token(engine, draft):
    prompt = _prompt(40, 5)
    engine.set_end_tokens([])
    plain = engine.generate(prompt, 24, draft_max=draft, max_ngram=3, min_ngram=1)
    assert plain.finish_reason == "length" and len(plain.sampled_tokens) == 24
    end = plain.sampled_tokens[12]
    stop_at = plain.sampled_tokens.index(end)
    engine.set_end_tokens([end])
    stopped = engine.generate(prompt, 24, draft_max=draft, max_ngram=3, min_ngram=1)
    engine.set_end_tokens([])
    assert stopped.finish_reason == "stop"
    assert stopped.sampled_tokens == plain.sampled_tokens[:stop_at]


def test_concurrent_generation_ends_each_request_at_end_token(engine):
    prompts = [_prompt(30, 6), _prompt(36, 7)]
    engine.set_end_tokens([])
    plain, _ = engine.generate_concurrent(prompts, 20, draft_max=K)
    end = plain[0].sampled_tokens[8]
    engine.set_end_tokens([end])
    stopped, _ = engine.generate_concurrent(prompts, 20, draft_max=K)
    engine.set_end_tokens([])
    for p, s in zip(plain, stopped):
        if end in p.sampled_tokens:
            assert s.finish_reason == "stop"
            assert s.sampled_tokens == p.sampled_tokens[:p.sampled_tokens.index(end)]
        else:
            assert s.finish_reason == "length" and s.sampled_tokens == p.sampled_tokens


def test_end_token_arguments_are_checked(engine):
    with pytest.raises(InvalidArgument):
        engine.set_end_tokens(list(range(17)))
    with pytest.raises(InvalidArgument):
        engine.set_end_tokens([CFG.n_vocab])
    with pytest.raises(InvalidArgument):
        engine.set_end_tokens([-1])
    engine.set_end_tokens([])
