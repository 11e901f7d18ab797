// The HIP engine through the reference runtime's own compiled contract: the
// reference's inference types (runtime/inference/stage.cpp,
// token_payload.cpp) and its ContinuousBatchingExecutor
// (runtime/pipeline_parallel/continuous_batching_executor.cpp), built from
// their sources, around the C-ABI HipStageExecutor of this directory.
//
//   serving: the cases of native_stage_executor_test.cpp:72-137 on the
//     reference's two-layer fixture package (prompt "fixture" = [2], greedy
//     token 7, piece "x")
//   distributed: native_stage_executor_test.cpp:139-230, two stages of the
//     same package chained over activation payloads
//   verify and execute_batch: multi-row decode equals serial decode; a batch
//     of sessions equals each session alone
//   text: a text prompt through the executor with the C-ABI tokenizer (the
//     LlamaCppTokenizer drop-in) on a package with a byte-level BPE vocabulary
//   continuous batching: continuous_batching_executor_test.cpp:99-133 with
//     this executor as the delegate: concurrent decode steps coalesce into one
//     engine step; then two concurrent prompt-lookup-shaped generations on a
//     synthetic Q4_K model sample the tokens of direct C-ABI decode loops
//
// Built as a shared library whose jfh_refbind_test_main(package) the GPU
// test calls in its own process.
#include "hip_stage_executor.hpp"

#include "inference/token_payload.hpp"
#include "pipeline_parallel/continuous_batching_executor.hpp"

#include <chrono>
#include <cstdio>
#include <future>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace {

namespace rt = jetsonfabric::runtime;
using rt::adapters::HipStageConfig;
using rt::adapters::HipStageExecutor;
using rt::inference::ExecutionResult;
using rt::inference::LayerRange;
using rt::inference::Payload;
using rt::inference::PayloadKind;
using rt::inference::Phase;
using rt::inference::StageInput;
using rt::inference::StagePosition;

int failures = 0;

void expect(bool condition, const std::string& what) {
    if (!condition) {
        std::printf("FAIL: %s\n", what.c_str());
        ++failures;
    }
}

void ok(const jfh_status& s, const char* what) {
    if (s.code != JFH_STATUS_OK) throw std::runtime_error(std::string(what) + ": " + s.message);
}

// The fixture package's tokenizer (native_stage_executor_test.cpp:31-46).
class FixtureTokenizer final : public rt::tokenization::Tokenizer {
public:
    std::vector<std::int32_t> tokenize(std::string_view text) const override {
        if (text != "fixture") throw std::invalid_argument("unexpected fixture prompt");
        return {2};
    }
    std::string token_piece(std::int32_t token) const override {
        if (token != 7) throw std::invalid_argument("unexpected fixture token");
        return "x";
    }
    bool is_end_token(std::int32_t) const override { return false; }
};

// Token ids as pieces, for the synthetic model.
class IdsTokenizer final : public rt::tokenization::Tokenizer {
public:
    std::vector<std::int32_t> tokenize(std::string_view) const override {
        throw std::invalid_argument("the synthetic model takes token payloads");
    }
    std::string token_piece(std::int32_t token) const override { return std::to_string(token) + " "; }
    bool is_end_token(std::int32_t) const override { return false; }
};

Payload text_payload(const std::string& text) {
    Payload p;
    p.kind = PayloadKind::Text;
    p.encoding = "utf-8";
    p.bytes.assign(text.begin(), text.end());
    return p;
}

Payload tokens_payload(const std::vector<std::int32_t>& ids) {
    Payload p;
    p.kind = PayloadKind::Tokens;
    p.tensor.dtype = "i32";
    p.tensor.shape = {static_cast<std::int64_t>(ids.size())};
    p.tensor.byte_order = "little";
    p.tensor.layout = "row_major";
    for (const std::int32_t t : ids) {
        const auto u = static_cast<std::uint32_t>(t);
        for (int b = 0; b < 4; ++b) p.bytes.push_back(static_cast<std::uint8_t>(u >> (8 * b)));
    }
    return p;
}

StageInput make_input(const std::string& session, Phase phase, int step, StagePosition pos, LayerRange layers,
                      Payload payload, int max_tokens) {
    StageInput in;
    in.session_id = session;
    in.request_id = session + "-request";
    in.model_id = "fixture";
    in.phase = phase;
    in.decode_step = step;
    in.position = pos;
    in.layers = layers;
    in.payload = std::move(payload);
    in.max_tokens = max_tokens;
    return in;
}

// native_stage_executor_test.cpp:78-87
void expect_sampled_seven(const ExecutionResult& r, const std::string& where) {
    expect(r.ok, where + ": " + r.error.message);
    if (!r.ok) return;
    expect(rt::inference::decode_single_token(r.output.payload) == 7, where + ": sampled token");
    expect(r.output.token_text == "x", where + ": token text");
    expect(r.output.completion_tokens == 1, where + ": completion count");
}

struct Engine {
    jfh_model* model = nullptr;
    jfh_engine* engine = nullptr;
    Engine(const char* package, std::uint32_t start, std::uint32_t end) {
        ok(jfh_model_open(package, start, end, 1, &model), "open package");
        jfh_engine_options opt{0, 1};
        ok(jfh_engine_create(model, &opt, &engine), "create engine");
    }
    explicit Engine(const jfh_synth_spec& spec) {
        ok(jfh_model_synthesize(&spec, &model), "synthesize model");
        jfh_engine_options opt{0, 1};
        ok(jfh_engine_create(model, &opt, &engine), "create engine");
    }
    ~Engine() {
        jfh_engine_destroy(engine);
        jfh_model_close(model);
    }
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;
};

HipStageConfig stage_config(jfh_engine* e, std::shared_ptr<const rt::tokenization::Tokenizer> tok, int ctx,
                            StagePosition pos, LayerRange layers) {
    HipStageConfig c;
    c.engine = e;
    c.tokenizer = std::move(tok);
    c.ctx_size = ctx;
    c.position = pos;
    c.layers = layers;
    c.speculative_max_tokens = 4;
    return c;
}

std::vector<std::int32_t> sampled(const ExecutionResult& r) {
    if (!r.ok) throw std::runtime_error("stage failed: " + r.error.code + ": " + r.error.message);
    return rt::inference::decode_token_ids(r.output.payload);
}

void serving_cases(const char* package) {
    Engine whole(package, 0, std::numeric_limits<std::uint32_t>::max());
    jfh_model_params params{};
    ok(jfh_engine_get_params(whole.engine, &params), "engine params");
    const int layers = static_cast<int>(params.n_layer);

    // the session below the executor (native_stage_executor_test.cpp:92-101)
    jfh_session* s = nullptr;
    ok(jfh_session_create(whole.engine, 2, &s), "session");
    const std::int32_t prompt[1] = {2};
    std::int32_t t = -1;
    expect(jfh_session_position(s) == 0, "session starts empty");
    ok(jfh_session_prefill(s, prompt, 1, &t, nullptr), "prefill");
    expect(t == 7 && jfh_session_position(s) == 1, "session prefill token and position");
    ok(jfh_session_decode(s, 7, &t, nullptr), "decode");
    expect(t == 7 && jfh_session_position(s) == 2, "session decode token and position");
    ok(jfh_session_rollback(s, 1), "rollback");
    expect(jfh_session_position(s) == 1, "session rollback position");
    jfh_session_destroy(s);

    auto tok = std::make_shared<FixtureTokenizer>();
    HipStageExecutor executor(stage_config(whole.engine, tok, 16, {0, 1}, {0, layers}));
    const StageInput prefill = make_input("native-serving-session", Phase::Prefill, 0, {0, 1}, {0, layers},
                                          text_payload("fixture"), 2);
    const ExecutionResult pre = executor.execute(prefill);
    expect_sampled_seven(pre, "prefill");
    expect(pre.output.prompt_tokens == 1, "prefill prompt token count");
    expect(pre.output.prompt_token_ids == std::vector<std::uint32_t>{2}, "prefill prompt token ids");
    expect(executor.session_count() == 1, "prefill keeps a session");
    const ExecutionResult dup = executor.execute(prefill);
    expect(!dup.ok && dup.error.code == "duplicate_stage_session", "duplicate prefill: " + dup.error.code);

    StageInput decode = prefill;
    decode.phase = Phase::Decode;
    decode.decode_step = 1;
    decode.payload = rt::inference::sampled_token_payload(7);
    expect_sampled_seven(executor.execute(decode), "decode");
    executor.rollback_session(prefill.session_id, 1);
    expect_sampled_seven(executor.execute(decode), "decode after rollback");
    executor.close_session(prefill.session_id);
    expect(executor.session_count() == 0, "close releases the session");
    const ExecutionResult closed = executor.execute(decode);
    expect(!closed.ok && closed.error.code == "stage_session_not_found", "decode after close: " + closed.error.code);

    StageInput wrong = prefill;
    wrong.layers = {0, layers - 1};
    const ExecutionResult mismatch = executor.execute(wrong);
    expect(!mismatch.ok && mismatch.error.code == "native_stage_assignment_mismatch",
           "assignment mismatch: " + mismatch.error.code);
    StageInput too_long = prefill;
    too_long.session_id = "too-long";
    too_long.max_tokens = 17;
    const ExecutionResult exceeded = executor.execute(too_long);
    expect(!exceeded.ok && exceeded.error.code == "invalid_native_stage_input",
           "context exceeded: " + exceeded.error.code);

    try {
        HipStageExecutor bad(stage_config(whole.engine, tok, 16, {0, 1}, {1, layers}));
        expect(false, "a first stage that does not start at layer 0 was accepted");
    } catch (const std::invalid_argument& e) {
        expect(std::string(e.what()) == "native serving stage assignment is invalid", e.what());
    }
}

void distributed_cases(const char* package) {
    Engine first_engine(package, 0, 1), final_engine(package, 1, 2);
    jfh_model_stats a{}, b{};
    ok(jfh_model_get_stats(first_engine.model, &a), "stats");
    ok(jfh_model_get_stats(final_engine.model, &b), "stats");
    expect(a.layer_start == 0 && a.layer_end == 1 && b.layer_start == 1 && b.layer_end == 2, "stage layer ranges");
    expect(a.selected_weight_bytes < a.total_weight_bytes && b.selected_weight_bytes < b.total_weight_bytes,
           "stages hold part of the weights");
    auto tok = std::make_shared<FixtureTokenizer>();
    HipStageExecutor first(stage_config(first_engine.engine, tok, 16, {0, 2}, {0, 1}));
    HipStageExecutor final(stage_config(final_engine.engine, tok, 16, {1, 2}, {1, 2}));

    const StageInput first_prefill = make_input("s", Phase::Prefill, 0, {0, 2}, {0, 1}, text_payload("fixture"), 2);
    const ExecutionResult fp = first.execute(first_prefill);
    expect(fp.ok && fp.output.payload.kind == PayloadKind::Activation, "first prefill returns an activation");
    if (!fp.ok) return;
    StageInput final_prefill = first_prefill;
    final_prefill.position = {1, 2};
    final_prefill.layers = {1, 2};
    final_prefill.payload = fp.output.payload;
    expect_sampled_seven(final.execute(final_prefill), "final prefill");

    StageInput oversized = final_prefill;
    oversized.session_id = "oversized-activation";
    oversized.payload.tensor.shape[0] = std::numeric_limits<std::int64_t>::max();
    oversized.payload.bytes.clear();
    const ExecutionResult o = final.execute(oversized);
    expect(!o.ok && o.error.code == "invalid_native_stage_input", "oversized activation: " + o.error.code);

    StageInput first_decode = first_prefill;
    first_decode.phase = Phase::Decode;
    first_decode.decode_step = 1;
    first_decode.payload = rt::inference::sampled_token_payload(7);
    const ExecutionResult fd = first.execute(first_decode);
    expect(fd.ok && fd.output.payload.kind == PayloadKind::Activation, "first decode returns an activation");
    if (!fd.ok) return;
    StageInput final_decode = final_prefill;
    final_decode.phase = Phase::Decode;
    final_decode.decode_step = 1;
    final_decode.payload = fd.output.payload;
    expect_sampled_seven(final.execute(final_decode), "final decode");
}

jfh_synth_spec synthetic_spec() {
    jfh_synth_spec spec{};
    spec.params = {2, 512, 1536, 8, 2, 256, 4096, 64, 1.0e6F, 1.0e-6F};
    spec.type_linear = JFH_TENSOR_Q4_K;
    spec.type_embd = JFH_TENSOR_Q4_K;
    spec.type_output = JFH_TENSOR_Q6_K;
    spec.seed = 29;
    spec.stddev = 0.02F;
    return spec;
}

std::vector<std::int32_t> prompt_of(int n, int seed) {
    std::vector<std::int32_t> p;
    std::uint32_t x = 2654435761U * static_cast<std::uint32_t>(seed + 1);
    for (int i = 0; i < n; ++i) {
        x = x * 1664525U + 1013904223U;
        p.push_back(static_cast<std::int32_t>((x >> 8) % 4096U));
    }
    return p;
}

// greedy continuation of `prompt` by direct C-ABI calls
std::vector<std::int32_t> direct_greedy(jfh_engine* e, const std::vector<std::int32_t>& prompt, int n) {
    jfh_session* s = nullptr;
    ok(jfh_session_create(e, static_cast<std::uint32_t>(prompt.size() + n), &s), "session");
    std::vector<std::int32_t> out(1);
    ok(jfh_session_prefill(s, prompt.data(), static_cast<std::uint32_t>(prompt.size()), &out[0], nullptr), "prefill");
    while (static_cast<int>(out.size()) < n) {
        std::int32_t t = -1;
        ok(jfh_session_decode(s, out.back(), &t, nullptr), "decode");
        out.push_back(t);
    }
    jfh_session_destroy(s);
    return out;
}

void verify_and_batch_cases(Engine& model) {
    auto tok = std::make_shared<IdsTokenizer>();
    HipStageExecutor executor(stage_config(model.engine, tok, 128, {0, 1}, {0, 2}));
    const std::vector<std::int32_t> pa = prompt_of(20, 1), pb = prompt_of(27, 2);
    const std::vector<std::int32_t> ga = direct_greedy(model.engine, pa, 8), gb = direct_greedy(model.engine, pb, 8);

    // verify: [previous, draft...] with the greedy continuation as the draft
    const StageInput pre = make_input("a", Phase::Prefill, 0, {0, 1}, {0, 2}, tokens_payload(pa), 16);
    expect(sampled(executor.execute(pre)) == std::vector<std::int32_t>{ga[0]}, "prefill token");
    StageInput verify = pre;
    verify.phase = Phase::Decode;
    verify.decode_step = 1;
    verify.payload = tokens_payload({ga[0], ga[1], ga[2], ga[3], ga[4]});
    const ExecutionResult v = executor.execute(verify);
    expect(v.ok && v.output.payload.kind == PayloadKind::SampledTokens && v.output.verification_width == 5,
           "verify answers sampled_tokens of width 5");
    expect(sampled(v) == std::vector<std::int32_t>(ga.begin() + 1, ga.begin() + 6), "verify equals serial decode");
    executor.rollback_session("a", 2);  // keep [previous, d1, d2]; the next input is d3 at decode step 4
    StageInput next = verify;
    next.decode_step = 4;
    next.payload = rt::inference::sampled_token_payload(ga[3]);
    expect(sampled(executor.execute(next)) == std::vector<std::int32_t>{ga[4]}, "decode after verify rollback");
    StageInput too_wide = next;
    too_wide.decode_step = 5;
    too_wide.payload = tokens_payload(std::vector<std::int32_t>(6, ga[4]));
    const ExecutionResult w = executor.execute(too_wide);
    expect(!w.ok && w.error.code == "invalid_verification_width", "verify wider than k + 1: " + w.error.code);

    // execute_batch: two sessions in one engine step equal each alone
    const StageInput pre_b = make_input("b", Phase::Prefill, 0, {0, 1}, {0, 2}, tokens_payload(pb), 16);
    expect(sampled(executor.execute(pre_b)) == std::vector<std::int32_t>{gb[0]}, "prefill token b");
    StageInput da = next, db = pre_b;
    da.decode_step = 5;
    da.payload = rt::inference::sampled_token_payload(ga[4]);
    db.phase = Phase::Decode;
    db.decode_step = 1;
    db.payload = tokens_payload({gb[0], gb[1], gb[2]});
    const std::vector<ExecutionResult> r = executor.execute_batch({da, db});
    expect(r.size() == 2 && r[0].ok && r[1].ok, "batch ran");
    if (r.size() == 2 && r[0].ok && r[1].ok) {
        expect(sampled(r[0]) == std::vector<std::int32_t>{ga[5]}, "batched decode equals serial");
        expect(sampled(r[1]) == std::vector<std::int32_t>({gb[1], gb[2], gb[3]}), "batched verify equals serial");
        expect(r[0].output.execution_batch_size == 2 && r[1].output.execution_batch_size == 2, "batch size telemetry");
    }
    executor.close_session("a");
    executor.close_session("b");
}

// continuous_batching_executor_test.cpp:99-133 with the HIP executor as delegate,
// then two greedy generations through it against direct decode loops
void continuous_batching_cases(Engine& model) {
    auto tok = std::make_shared<IdsTokenizer>();
    rt::pipeline_parallel::ContinuousBatchingConfig bc;
    bc.max_batch_size = 2;
    bc.max_wait = std::chrono::milliseconds(20);
    rt::pipeline_parallel::ContinuousBatchingExecutor executor(
        std::make_unique<HipStageExecutor>(stage_config(model.engine, tok, 128, {0, 1}, {0, 2})), bc);
    const std::vector<std::int32_t> pa = prompt_of(24, 3), pb = prompt_of(31, 4);
    const int n = 12;
    const std::vector<std::int32_t> ga = direct_greedy(model.engine, pa, n), gb = direct_greedy(model.engine, pb, n);

    auto run = [&](const std::string& id, const std::vector<std::int32_t>& prompt) {
        std::vector<std::int32_t> out;
        std::vector<int> batch_sizes;
        const StageInput pre = make_input(id, Phase::Prefill, 0, {0, 1}, {0, 2}, tokens_payload(prompt), n);
        out.push_back(sampled(executor.execute(pre)).at(0));
        for (int step = 1; step < n; ++step) {
            StageInput d = pre;
            d.phase = Phase::Decode;
            d.decode_step = step;
            d.payload = rt::inference::sampled_token_payload(out.back());
            const ExecutionResult r = executor.execute(d);
            out.push_back(sampled(r).at(0));
            batch_sizes.push_back(r.output.execution_batch_size);
        }
        executor.close_session(id);
        return std::make_pair(out, batch_sizes);
    };
    auto fa = std::async(std::launch::async, [&] { return run("ca", pa); });
    auto fb = std::async(std::launch::async, [&] { return run("cb", pb); });
    const auto [ta, sa] = fa.get();
    const auto [tb, sb] = fb.get();
    expect(ta == ga, "batched generation a equals direct decode");
    expect(tb == gb, "batched generation b equals direct decode");
    int coalesced = 0;
    for (const int s : sa) coalesced += s == 2;
    expect(coalesced > 0, "concurrent decode steps were coalesced into two-sequence engine steps");
}

// A text prompt through the executor with the C-ABI tokenizer, on a model
// whose package carries a byte-level BPE vocabulary
// (native_stage_executor.cpp:176-210: the prompt text is tokenized, the
// sampled token's piece and end flag come from the tokenizer): the prompt
// ids, the sampled tokens, their pieces and end flags equal the C ABI's
// tokenizer and a direct session on the same ids.
void text_cases(const char* package) {
    Engine whole(package, 0, std::numeric_limits<std::uint32_t>::max());
    jfh_model_params params{};
    ok(jfh_engine_get_params(whole.engine, &params), "engine params");
    const int layers = static_cast<int>(params.n_layer);
    auto tok = std::make_shared<rt::adapters::CAbiTokenizer>(package);
    const std::vector<std::int32_t> end = tok->end_tokens();
    expect(!end.empty() && tok->is_end_token(-1), "the vocabulary has end-of-generation ids");
    ok(jfh_engine_set_end_tokens(whole.engine, end.data(), static_cast<std::uint32_t>(end.size())), "end tokens");
    const std::string prompt = "<|im_start|>user\nReply with OK only.<|im_end|>\n<|im_start|>assistant\n";
    const std::vector<std::int32_t> ids = tok->tokenize(prompt);

    jfh_session* direct = nullptr;
    ok(jfh_session_create(whole.engine, 64, &direct), "session");
    std::int32_t want = -1;
    ok(jfh_session_prefill(direct, ids.data(), static_cast<std::uint32_t>(ids.size()), &want, nullptr), "prefill");

    HipStageExecutor executor(stage_config(whole.engine, tok, 64, {0, 1}, {0, layers}));
    StageInput in = make_input("text-session", Phase::Prefill, 0, {0, 1}, {0, layers}, text_payload(prompt), 4);
    ExecutionResult r = executor.execute(in);
    expect(r.ok, "text prefill: " + r.error.message);
    if (!r.ok) return;
    std::vector<std::uint32_t> uids(ids.begin(), ids.end());
    expect(r.output.prompt_token_ids == uids, "prompt ids are the tokenizer's");
    for (int step = 1; step <= 3; ++step) {
        const std::int32_t got = rt::inference::decode_single_token(r.output.payload);
        expect(got == want, "text step " + std::to_string(step) + " samples the direct session's token");
        expect(r.output.token_text == tok->token_piece(got), "token text is the tokenizer's piece");
        expect(r.output.end_of_generation == tok->is_end_token(got), "end flag is the tokenizer's");
        in.phase = Phase::Decode;
        in.decode_step = step;
        in.payload = rt::inference::sampled_token_payload(got);
        r = executor.execute(in);
        expect(r.ok, "text decode: " + r.error.message);
        if (!r.ok) break;
        ok(jfh_session_decode(direct, got, &want, nullptr), "decode");
    }
    jfh_session_destroy(direct);
    executor.close_session(in.session_id);
    try {
        (void) tok->tokenize("");
        expect(false, "an empty prompt tokenized");
    } catch (const std::invalid_argument& e) {
        expect(std::string(e.what()) == "native prompt tokenization produced no tokens", e.what());
    }
}

}  // namespace

// The text case alone, on a package with a vocabulary.
extern "C" int jfh_refbind_text_main(const char* package) try {
    failures = 0;
    text_cases(package);
    if (failures == 0) std::printf("refbind text tests passed\n");
    std::fflush(stdout);
    return failures;
} catch (const std::exception& e) {
    std::printf("FAIL: %s\n", e.what());
    std::fflush(stdout);
    return 1;
}

extern "C" int jfh_refbind_test_main(const char* fixture_package) try {
    failures = 0;
    serving_cases(fixture_package);
    distributed_cases(fixture_package);
    {
        Engine model(synthetic_spec());
        verify_and_batch_cases(model);
        continuous_batching_cases(model);
    }
    if (failures == 0) std::printf("refbind tests passed\n");
    std::fflush(stdout);
    return failures;
} catch (const std::exception& e) {
    std::printf("FAIL: %s\n", e.what());
    std::fflush(stdout);
    return 1;
}
