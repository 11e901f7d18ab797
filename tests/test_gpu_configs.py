"""GPU parity at the benchmark workloads' real widths, through the C ABI.

Each workload's model keeps its hidden size, heads, FFN width, vocabulary and
tensor types but only one or two layers, so the CPU oracle answers in
seconds while the kernels see every shape the full models use. Long contexts
(up to the 8192-position, 8-sequence workload) are set up by importing the
oracle's seeded KV cache into the GPU sessions instead of prefilling them.

Bars as in test_gpu_parity: KV rows written by the engine match the oracle's
f16 rows (layer 0: bit-exact but for rare last-ulp differences); logits within
NRMSE 5e-3 / cosine 0.9995 of the oracle; verify == serial and batch ==
individual exactly.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import jetsonfabric_amd as jf
import oracle as jo
from tests.test_gpu_parity import assert_logits_match

pytestmark = pytest.mark.gpu

# workload -> (layers kept, context of the long-context case)
CASES = {
    "qwen2.5-1.5b-q4k-spec": (2, 1024),
    "qwen2.5-7b-q4k": (1, 2048),
    "qwen2.5-14b-q4k": (1, 4096),
    "qwen2.5-32b-q2k": (1, 8192),
}


@pytest.fixture(scope="module", params=list(CASES))
def workload(request):
    wl = jf.config_by_name(request.param)
    layers, ctx = CASES[request.param]
    cfg = dataclasses.replace(wl.model, n_layer=layers)
    model = jf.Model.synthesize(cfg, type_linear=wl.type_linear, type_embd=wl.type_embd, type_output=wl.type_output,
                                tied_output=wl.tied_output, seed=77, threads=16)
    engine = jf.NativeEngine(model)
    om = jo.OracleModel.from_model(model)
    print(f"[{request.param}] {layers} layer(s), hidden {cfg.n_embd}, heads {cfg.n_head}/{cfg.n_head_kv}, "
          f"ffn {cfg.n_ff}, vocab {cfg.n_vocab}", flush=True)
    yield wl, cfg, model, engine, om, ctx
    engine.close()


def _prompt(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def test_prefill_decode_and_kv_rows(workload):
    wl, cfg, _, engine, om, _ = workload
    prompt = _prompt(16, cfg.n_vocab, 1)
    s = engine.create_session(32)
    ref = om.session(32, jo.MODE_Q8, 16)
    tok, lg = s.prefill_greedy(prompt, logits=True)
    _, rl = ref.forward(prompt, 1)
    assert_logits_match(rl[0], lg, tok, "prefill")
    # layer 0's K/V rows: same codes and scales, so f16 rows agree but for last-ulp roundings
    gk, gv = s.read_kv(0, len(prompt))
    rk, rv = ref.read_kv(0, len(prompt))
    for g, r, name in ((gk, rk, "K"), (gv, rv, "V")):
        gf, rf = g.view(np.float16).astype(np.float32), r.view(np.float16).astype(np.float32)
        assert np.mean(g == r) >= 0.97, f"{name} rows bit-identical fraction {np.mean(g == r):.4f}"
        assert np.allclose(gf, rf, rtol=2e-3, atol=1e-4), f"{name} rows differ beyond an f16 ulp"
    for step in range(2):
        nxt, lg = s.decode_greedy(tok, logits=True)
        _, rl = ref.forward([tok], 1)
        assert_logits_match(rl[0], lg, nxt, f"decode step {step}")
        tok = nxt
    ref.close()


def test_verify_width_equals_serial(workload):
    wl, cfg, _, engine, _, _ = workload
    k = max(wl.draft_max, 4)
    prompt = _prompt(20, cfg.n_vocab, 2)
    a = engine.create_session(64)
    serial = [a.prefill_greedy(prompt)]
    for _ in range(k):
        serial.append(a.decode_greedy(serial[-1]))
    b = engine.create_session(64)
    assert b.prefill_greedy(prompt) == serial[0]
    ids, accepted = b.verify(serial[:k + 1])
    assert ids[:k] == serial[1:k + 1] and accepted == k


def test_long_context_with_imported_cache(workload):
    wl, cfg, _, engine, om, ctx = workload
    k = max(wl.draft_max, 4)
    n = ctx - 2 * (k + 2)
    ref = om.session(ctx, jo.MODE_Q8, 16)
    ref.fill_kv(n, seed=5)
    kv = [ref.read_kv(layer, n) for layer in range(cfg.n_layer)]
    s = engine.create_session(ctx)
    s.import_kv(np.stack([x[0] for x in kv]), np.stack([x[1] for x in kv]))
    assert s.position() == n
    tok = 3
    for step in range(2):
        nxt, lg = s.decode_greedy(tok, logits=True)
        _, rl = ref.forward([tok], 1)
        assert_logits_match(rl[0], lg, nxt, f"decode at {n + step}")
        tok = int(np.argmax(rl[0]))
    rows = [tok] + _prompt(k, cfg.n_vocab, 3)
    ids, _, lg = s.verify(rows, logits=True)
    r_ids, rl = ref.forward(rows, len(rows))
    for r in range(len(rows)):
        assert_logits_match(rl[r], lg[r], ids[r], f"verify row {r} at {n + 2}")
    ref.close()


def test_batch_of_sessions_matches_individual_steps(workload):
    """A batched step over the workload's concurrent sequences (each with its
    own context length and k + 1 draft rows): every sequence's logits rows
    match its own oracle session's (NRMSE 5e-3 / cosine 0.9995), and its ids
    and accepted count equal the same rows verified alone, bit for bit."""
    wl, cfg, _, engine, om, ctx = workload
    k = max(wl.draft_max, 4)
    count = max(wl.concurrency, 2)
    n = ctx - (k + 2)
    refs = [om.session(ctx, jo.MODE_Q8, 16) for _ in range(count)]
    caches = []
    for i, ref in enumerate(refs):
        ref.fill_kv(n - 7 * i, seed=11 + i)
        kv = [ref.read_kv(layer, n - 7 * i) for layer in range(cfg.n_layer)]
        caches.append((np.stack([x[0] for x in kv]), np.stack([x[1] for x in kv])))
    rows = [[5 + i] + _prompt(k, cfg.n_vocab, 20 + i) for i in range(count)]
    batch = [engine.create_session(ctx) for _ in range(count)]
    for s, (ck, cv) in zip(batch, caches):
        s.import_kv(ck, cv)
    ids, accepted, logits = engine.step_batch(batch, rows, logits=True)
    for i, ref in enumerate(refs):
        r_ids, rl = ref.forward(rows[i], len(rows[i]))
        for r in range(len(rows[i])):
            assert_logits_match(rl[r], logits[i][r], ids[i][r], f"sequence {i} row {r}")
        ref.close()
    for i in range(count):
        single = engine.create_session(ctx)
        single.import_kv(*caches[i])
        s_ids, s_acc = single.verify(rows[i])
        assert ids[i] == s_ids and accepted[i] == s_acc, f"sequence {i}"
        single.close()


def test_concurrent_generation_equals_each_alone(workload):
    """The workload's continuous batching at its real widths: concurrent
    runners (decode steps, and draft-verify steps where the workload drafts,
    coalesced into one multi-sequence forward) give every request the tokens
    and pass counts it gets alone."""
    wl, cfg, _, engine, _, _ = workload
    count = min(max(wl.concurrency, 2), 4)
    prompts = []
    for i in range(count):
        seg = _prompt(10 + 2 * i, cfg.n_vocab, 60 + i)
        prompts.append(seg + seg + seg[: 4 + i])  # repetitive: prompt lookup finds drafts
    draft = wl.draft_max
    results, _ = engine.generate_concurrent(prompts, 12, draft_max=draft, max_ngram=3, min_ngram=3,
                                            batch_wait_us=2000)
    for prompt, got in zip(prompts, results):
        alone = engine.generate(prompt, 12, draft_max=draft, max_ngram=3, min_ngram=3)
        assert got.sampled_tokens == alone.sampled_tokens
        assert got.target_decode_passes == alone.target_decode_passes
