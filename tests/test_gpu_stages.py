"""Pipeline stages on one GPU (LayerRange, model_architecture.hpp:15-21;
Qwen2Session::prefill_stage_* / decode_stage_*, qwen2_architecture.cpp:
909-947, 977-1027): a package opened with a layer range gives an engine that
holds only those layers; the first stage embeds token ids, later stages take
the previous stage's residual-stream rows f32[n, n_embd], the last stage
returns the greedy id. Chained stages run the same kernels on the same rows
as the full-model engine, so their tokens (and the last stage's input rows)
must equal the full model's bit for bit.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import jetsonfabric_amd as jf
import oracle as jo

pytestmark = pytest.mark.gpu

CFG = jf.ModelConfig(n_layer=4, n_embd=512, n_ff=1536, n_head=8, n_head_kv=2, n_vocab=8192, n_ctx=2048)
RANGES = ((0, 1), (1, 3), (3, 4))


@pytest.fixture(scope="module")
def staged(tmp_path_factory):
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=5)
    pkg = tmp_path_factory.mktemp("stages")
    model.write_package(str(pkg))
    full = jf.NativeEngine(jf.Model.open(str(pkg)))
    stages = [jf.NativeEngine(jf.Model.open(str(pkg), a, b)) for a, b in RANGES]
    yield full, stages
    for e in stages + [full]:
        e.close()


def _prompt(n, seed=7):
    return [int(t) for t in np.random.default_rng(seed).integers(0, CFG.n_vocab, n)]


def test_stage_engines_hold_their_layer_ranges(staged):
    full, stages = staged
    assert (full.layer_start, full.layer_end, full.first_stage, full.last_stage) == (0, 4, True, True)
    got = [(e.layer_start, e.layer_end, e.first_stage, e.last_stage) for e in stages]
    assert got == [(0, 1, True, False), (1, 3, False, False), (3, 4, False, True)]
    # a stage uploads only its layers (plus embedding / head at the ends)
    assert sum(e.weight_bytes for e in stages) == full.weight_bytes


@pytest.mark.parametrize("n_prompt", [5, 300])
def test_three_stage_pipeline_equals_full_model(staged, n_prompt):
    """Prefill in chunks (300 rows > the 256-row chunk) and six decode steps
    through three stages give the full model's greedy ids; the middle
    stage's output equals what the last stage reads, row for row."""
    full, stages = staged
    prompt = _prompt(n_prompt)
    ref = full.create_session(320)
    tok = ref.prefill_greedy(prompt)
    s = [e.create_session(320) for e in stages]
    a0 = s[0].prefill_stage(tokens=prompt)
    assert a0.shape == (n_prompt, CFG.n_embd) and a0.dtype == np.float32 and np.isfinite(a0).all()
    a1 = s[1].prefill_stage(activations=a0)
    assert not np.array_equal(a0, a1)
    assert s[2].prefill_stage(activations=a1) == tok
    for step in range(6):
        want = ref.decode_greedy(tok)
        x = s[0].decode_stage(token=tok)
        x = s[1].decode_stage(activation=x)
        got = s[2].decode_stage(activation=x)
        assert got == want, f"decode step {step}"
        tok = want
    assert [si.position() for si in s] == [ref.position()] * 3


def test_stage_activations_match_the_oracle(staged):
    """Each stage's output rows against the oracle's stage forward over the
    same layer range and input rows (qwen2_architecture.cpp:909-947,
    977-1027): prefill rows (16, multi-row kernels) and two decode rows;
    NRMSE <= 5e-3 on the stage's update of the residual stream and on its
    output, the last stage's logits within NRMSE 5e-3 / cosine 0.9995."""
    full, stages = staged
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=5)
    om = jo.OracleModel.from_model(model)
    prompt = _prompt(16, seed=13)
    refs = [om.session(64, jo.MODE_Q8, 8) for _ in RANGES]
    gpu = [e.create_session(64) for e in stages]

    def check(i, rows_in, got, want, what):
        upd, out = jo.nrmse(want - rows_in, got - rows_in), jo.nrmse(want, got)
        assert upd <= 5e-3 and out <= 5e-3, f"stage {RANGES[i]} {what}: update {upd:.2e}, output {out:.2e}"

    rows = None
    for i, (a, b) in enumerate(RANGES):
        last = b == CFG.n_layer
        r_rows, _, r_lg = refs[i].forward_range(a, b, tokens=prompt if a == 0 else None,
                                                rows=None if a == 0 else rows, logits_rows=1 if last else 0)
        if last:
            tok, lg = gpu[i].prefill_stage(activations=rows, logits=True)
            assert jo.nrmse(r_lg[0], lg) <= 5e-3 and jo.cosine(r_lg[0], lg) >= 0.9995
        else:
            got = gpu[i].prefill_stage(tokens=prompt) if a == 0 else gpu[i].prefill_stage(activations=rows)
            check(i, r_rows[0], got, r_rows[-1], "prefill")
        rows = r_rows[-1]
    for step in range(2):
        token = prompt[step]
        rows = None
        for i, (a, b) in enumerate(RANGES):
            last = b == CFG.n_layer
            r_rows, _, r_lg = refs[i].forward_range(a, b, tokens=[token] if a == 0 else None,
                                                    rows=None if a == 0 else rows, logits_rows=1 if last else 0)
            if last:
                _, lg = gpu[i].decode_stage(activation=rows, logits=True)
                assert jo.nrmse(r_lg[0], lg) <= 5e-3 and jo.cosine(r_lg[0], lg) >= 0.9995
            else:
                got = gpu[i].decode_stage(token=token) if a == 0 else gpu[i].decode_stage(activation=rows)
                check(i, r_rows[0], got, r_rows[-1], f"decode {step}")
            rows = r_rows[-1]
    for r in refs:
        r.close()


def test_in_memory_slices_are_the_package_stages(staged):
    """Stages made from an in-memory model (Model.slice) hold the same layers
    as the package opened with a layer range and give the same rows."""
    _, stages = staged
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=5)
    prompt = _prompt(12, seed=17)
    rows = None
    for (a, b), pkg_stage in zip(RANGES, stages):
        e = jf.NativeEngine(model.slice(a, b))
        assert (e.layer_start, e.layer_end, e.weight_bytes) == (pkg_stage.layer_start, pkg_stage.layer_end,
                                                               pkg_stage.weight_bytes)
        s1, s2 = e.create_session(32), pkg_stage.create_session(32)
        if a == 0:
            got, want = s1.prefill_stage(tokens=prompt), s2.prefill_stage(tokens=prompt)
        else:
            got, want = s1.prefill_stage(activations=rows), s2.prefill_stage(activations=rows)
        if b == CFG.n_layer:
            assert got == want
        else:
            assert np.array_equal(got, want)
            rows = got
        e.close()


def test_two_runs_of_a_stage_are_identical(staged):
    _, stages = staged
    prompt = _prompt(20, seed=9)
    outs = []
    for _ in range(2):
        sess = stages[0].create_session(64)
        outs.append(sess.prefill_stage(tokens=prompt))
        outs.append(sess.decode_stage(token=prompt[-1]))
    assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[1], outs[3])


def test_stage_input_errors(staged):
    full, stages = staged
    first, middle, last = stages
    act = np.zeros((3, CFG.n_embd), dtype=np.float32)
    with pytest.raises(jf.JfhError, match="first native stage does not accept activations"):
        first.create_session(16).prefill_stage(tokens=None, activations=act)
    with pytest.raises(jf.JfhError, match="only the first native stage accepts tokens"):
        middle.create_session(16).prefill_stage(tokens=[1, 2, 3])
    with pytest.raises(jf.JfhError, match="native stage activation shape is invalid"):
        last.create_session(16).prefill_stage(activations=None)
    with pytest.raises(ValueError):
        middle.create_session(16).prefill_stage(activations=np.zeros((3, 7), dtype=np.float32))
    s = middle.create_session(16)
    with pytest.raises(jf.JfhError, match="decode is outside session capacity"):
        s.decode_stage(activation=np.zeros((1, CFG.n_embd), dtype=np.float32))
    with pytest.raises(jf.JfhError, match="only the first native stage accepts decode tokens"):
        s.decode_stage(token=3)
    with pytest.raises(jf.JfhError, match="prefill is outside session capacity"):
        middle.create_session(2).prefill_stage(activations=act)
    # full-model entry points need every layer
    with pytest.raises(jf.JfhError, match="full-model native inference requires every model layer"):
        first.create_session(16).prefill_greedy([1, 2, 3])
    with pytest.raises(jf.JfhError, match="full-model native inference requires every model layer"):
        last.create_session(16).prefill_greedy([1, 2, 3])
    # and the full model runs stage calls as a single first-and-last stage
    s = full.create_session(16)
    t = s.prefill_stage(tokens=[1, 2, 3])
    assert isinstance(t, int) and t == full.create_session(16).prefill_greedy([1, 2, 3])


def _library_inputs():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    csrc = os.path.join(root, "jetsonfabric_amd", "csrc")
    yield os.path.join(root, "jetsonfabric_amd", "libjfh.so")
    yield os.path.join(root, "include", "jfh.h")
    for name in os.listdir(csrc):
        if name.endswith(".hpp"):
            yield os.path.join(csrc, name)


def test_stage_executors_chain_like_the_whole_model(capfd):
    """tests/cpp/stage_test.cpp, in this process: two HipStageExecutors over
    layer ranges, chained by activation payloads (f32, and f16 on the wire),
    sample the whole-model executor's tokens; stage payload and assignment
    errors."""
    path = os.path.join(os.path.dirname(__file__), "cpp", "libstage_test.so")
    assert os.path.exists(path), "tests/cpp/libstage_test.so is not built (make -C tests/cpp)"
    # it constructs the engine's C++ classes itself: built against older headers
    # it would allocate them with a stale layout
    newest = max(os.path.getmtime(f) for f in _library_inputs())
    assert os.path.getmtime(path) >= newest, "tests/cpp/libstage_test.so is older than the library: make -C tests/cpp"
    jf.library()  # the engine library first, so the test links against the loaded copy
    rc = ctypes.CDLL(path).jfh_stage_test_main()
    out = capfd.readouterr().out
    assert rc == 0, out
    assert "stage tests passed" in out
