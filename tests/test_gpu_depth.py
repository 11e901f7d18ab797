"""Layer-by-layer parity of the full-depth benchmark model against the oracle.

The benchmarked Qwen2.5-7B-shape model (28 layers, Q4_K weights and
embedding, Q6_K head, the benchmark's seed) runs once through the oracle's
stage forward over all layers (qwen2_architecture.cpp:909-947, 977-1027),
which keeps the residual rows entering and leaving every layer. Every layer
then runs alone on the GPU as a one-layer pipeline stage (Model.slice, an
engine over layers [l, l + 1)) fed the oracle's rows entering it:

* eight prefill rows at positions 0..7 (the multi-row kernels: normalized
  rows quantized once, token-quad matrix-core matmuls);
* one decode row at position 1024, its layer's KV cache of the earlier
  positions imported from the oracle's seeded cache (the one-row kernels and
  attention over a long context);
* a k = 4 draft-verify step: five rows at positions 1024..1028 over the same
  cache (the verify path's kernels: normalized rows quantized once, 8-slot
  token quads, causal attention inside the step);
* a two-sequence batched step: that decode row beside five rows at positions
  600..604 of a second sequence with its own seeded cache (batched
  attention over two caches, token quads over both sequences' rows).

Bars, per layer: NRMSE <= 5e-3 between the GPU's and the oracle's update of
the residual stream (rows out - rows in, what the layer computes) and
between the output rows; the last layer, whose stage ends in the head, is
held to the same bar on its logits (and cosine >= 0.9995). A depth- or
position-dependent kernel defect shows up in the layer where it happens,
instead of being folded into the full model's end-to-end spread.
"""
from __future__ import annotations

import numpy as np
import pytest

import jetsonfabric_amd as jf
import oracle as jo

pytestmark = pytest.mark.gpu

WORKLOAD = "qwen2.5-7b-q4k"
SEED = 1234          # bench.py's model seed: the benchmarked weights
PREFILL = 8
CONTEXT = 1024
OTHER = 600         # the second sequence of the batched step: its cached positions
VERIFY = 5          # k = 4 draft verification
BAR = 5e-3


@pytest.fixture(scope="module")
def depth():
    wl = jf.config_by_name(WORKLOAD)
    cfg = wl.model
    model = jf.Model.synthesize(cfg, type_linear=wl.type_linear, type_embd=wl.type_embd, type_output=wl.type_output,
                                tied_output=wl.tied_output, seed=SEED, threads=16)
    om = jo.OracleModel.from_model(model)
    prompt = [int(t) for t in np.random.default_rng(21).integers(0, cfg.n_vocab, PREFILL)]
    pre = om.session(PREFILL + 2, jo.MODE_Q8, 16)
    pre_rows, _, pre_logits = pre.forward_range(0, cfg.n_layer, tokens=prompt, logits_rows=1)
    pre.close()
    dec = om.session(CONTEXT + VERIFY + 2, jo.MODE_Q8, 16)
    dec.fill_kv(CONTEXT, seed=31)
    kv = [dec.read_kv(layer, CONTEXT) for layer in range(cfg.n_layer)]
    token = 4242
    dec_rows, _, dec_logits = dec.forward_range(0, cfg.n_layer, tokens=[token], logits_rows=1)
    dec.rollback(1)
    vtoks = [token] + [int(t) for t in np.random.default_rng(22).integers(0, cfg.n_vocab, VERIFY - 1)]
    ver_rows, _, ver_logits = dec.forward_range(0, cfg.n_layer, tokens=vtoks, logits_rows=VERIFY)
    dec.close()
    other = om.session(OTHER + VERIFY + 2, jo.MODE_Q8, 16)
    other.fill_kv(OTHER, seed=47)
    kv_other = [other.read_kv(layer, OTHER) for layer in range(cfg.n_layer)]
    btoks = [int(t) for t in np.random.default_rng(23).integers(0, cfg.n_vocab, VERIFY)]
    oth_rows, _, oth_logits = other.forward_range(0, cfg.n_layer, tokens=btoks, logits_rows=VERIFY)
    other.close()
    print(f"[depth] oracle rows of {cfg.n_layer} layers ready", flush=True)
    yield {"cfg": cfg, "model": model, "prompt": prompt, "token": token, "pre_rows": pre_rows,
           "pre_logits": pre_logits[0], "dec_rows": dec_rows, "dec_logits": dec_logits[0], "kv": kv,
           "vtoks": vtoks, "ver_rows": ver_rows, "ver_logits": ver_logits, "kv_other": kv_other, "btoks": btoks,
           "oth_rows": oth_rows, "oth_logits": oth_logits}
    model.close()


def _check_rows(what, rows_in, got, want, report):
    upd = jo.nrmse(want - rows_in, got - rows_in)
    out = jo.nrmse(want, got)
    report.append((what, upd, out))
    assert upd <= BAR and out <= BAR, f"{what}: update NRMSE {upd:.2e}, output NRMSE {out:.2e}"


def _check_logits(what, got, want, report):
    e, c = jo.nrmse(want, got), jo.cosine(want, got)
    report.append((what, e, 1.0 - c))
    assert e <= BAR and c >= 0.9995, f"{what}: logits NRMSE {e:.2e}, cosine {c:.6f}"


def test_every_layer_matches_the_oracle(depth):
    cfg, model, prompt, token = depth["cfg"], depth["model"], depth["prompt"], depth["token"]
    pre_rows, pre_logits, dec_rows, dec_logits, kv = (depth["pre_rows"], depth["pre_logits"], depth["dec_rows"],
                                                      depth["dec_logits"], depth["kv"])
    vtoks, ver_rows, ver_logits = depth["vtoks"], depth["ver_rows"], depth["ver_logits"]
    kv_other, btoks, oth_rows, oth_logits = depth["kv_other"], depth["btoks"], depth["oth_rows"], depth["oth_logits"]
    report = []
    for layer in range(cfg.n_layer):
        print(f"[depth] layer {layer}", flush=True)
        part = model.slice(layer, layer + 1)
        engine = jf.NativeEngine(part)
        try:
            first, last = layer == 0, layer == cfg.n_layer - 1
            s = engine.create_session(PREFILL + 2)
            if last:
                _, lg = s.prefill_stage(activations=pre_rows[layer], logits=True)
                _check_logits(f"layer {layer} prefill logits", lg, pre_logits, report)
            else:
                got = s.prefill_stage(tokens=prompt) if first else s.prefill_stage(activations=pre_rows[layer])
                _check_rows(f"layer {layer} prefill", pre_rows[layer], got, pre_rows[layer + 1], report)
            s.close()
            d = engine.create_session(CONTEXT + 2)
            d.import_kv(kv[layer][0][None], kv[layer][1][None])
            if last:
                _, lg = d.decode_stage(activation=dec_rows[layer], logits=True)
                _check_logits(f"layer {layer} decode logits", lg, dec_logits, report)
            else:
                got = d.decode_stage(token=token) if first else d.decode_stage(activation=dec_rows[layer])
                _check_rows(f"layer {layer} decode at {CONTEXT}", dec_rows[layer], got, dec_rows[layer + 1], report)
            d.close()
            # k = 4 verify rows at 1024..1028 over the same cache
            v = engine.create_session(CONTEXT + VERIFY + 2)
            v.import_kv(kv[layer][0][None], kv[layer][1][None])
            if last:
                _, (lg,) = engine.stage_step_batch([v], activations=[ver_rows[layer]], logits=True)
                for r in range(VERIFY):
                    _check_logits(f"layer {layer} verify row {r} logits", lg[r], ver_logits[r], report)
            else:
                (got,) = (engine.stage_step_batch([v], tokens=[vtoks]) if first
                          else engine.stage_step_batch([v], activations=[ver_rows[layer]]))
                _check_rows(f"layer {layer} verify rows at {CONTEXT}", ver_rows[layer], got, ver_rows[layer + 1], report)
            v.close()
            # two sequences in one step: the decode row at 1024 and five rows at 600..604
            a = engine.create_session(CONTEXT + 2)
            a.import_kv(kv[layer][0][None], kv[layer][1][None])
            b = engine.create_session(OTHER + VERIFY + 2)
            b.import_kv(kv_other[layer][0][None], kv_other[layer][1][None])
            if last:
                _, (la, lb) = engine.stage_step_batch([a, b], activations=[dec_rows[layer], oth_rows[layer]], logits=True)
                _check_logits(f"layer {layer} batched decode logits", la[0], dec_logits, report)
                for r in range(VERIFY):
                    _check_logits(f"layer {layer} batched row {r} logits", lb[r], oth_logits[r], report)
            else:
                ga, gb = (engine.stage_step_batch([a, b], tokens=[[token], btoks]) if first
                          else engine.stage_step_batch([a, b], activations=[dec_rows[layer], oth_rows[layer]]))
                _check_rows(f"layer {layer} batched decode", dec_rows[layer], ga, dec_rows[layer + 1], report)
                _check_rows(f"layer {layer} batched rows at {OTHER}", oth_rows[layer], gb, oth_rows[layer + 1], report)
            a.close()
            b.close()
        finally:
            engine.close()
            part.close()
    worst = max(r[1] for r in report)
    print(f"[depth] {len(report)} checks, worst update/logits NRMSE {worst:.2e}; " +
          ", ".join(f"{w}: {a:.1e}/{b:.1e}" for w, a, b in report), flush=True)
