// Host-side tests of the speculative runtime (no GPU): prompt-lookup
// drafting, the greedy acceptance / rollback loop over a scripted executor,
// the continuous-batching executor, the stage payload helpers and the
// activation codecs. Mirrors
// the reference's own cases in
// runtime/speculative/prompt_lookup_draft_test.cpp:15-36,
// runtime/pipeline_parallel/generation_runner_test.cpp:108-190, 355-430 and
// runtime/pipeline_parallel/continuous_batching_executor_test.cpp and
// runtime/activation/activation_codec_test.cpp.
#include "jfh_runtime.hpp"

#include <chrono>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

using namespace jfh::runtime;

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what);
        ++failures;
    }
}

// Proposes [20, 21] only for the history the runner holds after the first
// token (prompt [1, 2, 1, 2] + sampled 10), like the reference's FixedDraft.
class FixedDraft final : public speculative::DraftStrategy {
public:
    std::vector<std::uint32_t> propose(const std::vector<std::uint32_t>& history, std::size_t) const override {
        return history == std::vector<std::uint32_t>({1, 2, 1, 2, 10}) ? std::vector<std::uint32_t>({20, 21})
                                                                      : std::vector<std::uint32_t>{};
    }
};

// Single-stage executor with scripted outputs: prefill samples 10 and
// reports prompt ids [1, 2, 1, 2]; every decode pass returns [20, 99, 30]
// truncated to the verification width.
class ScriptedExecutor final : public inference::Executor {
public:
    mutable int rollback_calls = 0;
    mutable int last_rollback = 0;
    mutable int close_calls = 0;
    mutable std::vector<std::vector<std::int32_t>> passes;
    mutable std::vector<int> steps;
    bool fail_rollback = false;

    inference::ExecutionResult execute(const inference::StageInput& in) const override {
        inference::StageOutput out;
        std::vector<std::int32_t> rows = inference::decode_token_ids(in.payload);
        if (in.phase == inference::Phase::Prefill) {
            out.payload = inference::sampled_token_payload(10);
            out.prompt_tokens = 4;
            out.prompt_token_ids = {1, 2, 1, 2};
            out.completion_tokens = 1;
            return inference::ExecutionResult::success(out);
        }
        passes.push_back(rows);
        steps.push_back(in.decode_step);
        const std::int32_t script[] = {20, 99, 30, 31, 32, 33, 34, 35, 36};
        std::vector<std::int32_t> sampled(script, script + rows.size());
        if (rows.size() == 1) {
            out.payload = inference::sampled_token_payload(sampled[0]);
        } else {
            out.payload = inference::sampled_tokens_payload(sampled);
            out.token_eog.assign(sampled.size(), 0);
            out.verification_width = static_cast<int>(sampled.size());
        }
        out.completion_tokens = static_cast<int>(sampled.size());
        return inference::ExecutionResult::success(out);
    }
    void close_session(const std::string&) const override { ++close_calls; }
    void rollback_session(const std::string&, int n) const override {
        ++rollback_calls;
        last_rollback = n;
        if (fail_rollback) throw std::runtime_error("injected rollback failure");
    }
};

void test_prompt_lookup() {
    speculative::PromptLookupDraft draft;
    expect(draft.propose({1, 2, 3, 1, 2, 3, 1, 2}, 3) == std::vector<std::uint32_t>({3, 1, 2}),
           "prompt lookup continues the latest matching suffix");
    expect(draft.propose({1, 2, 3, 4}, 3).empty(), "unique history gives no draft");
    expect(draft.propose({1, 2, 1, 2}, 0).empty(), "zero budget gives no draft");
    expect(draft.propose({7, 7}, 4).empty(), "history no longer than min_ngram gives no draft");
    bool rejected = false;
    try {
        speculative::PromptLookupDraft bad(1, 2);
    } catch (const std::invalid_argument&) {
        rejected = true;
    }
    expect(rejected, "max_ngram < min_ngram is rejected");
}

void test_accepts_prefix_and_rolls_back_suffix() {
    ScriptedExecutor ex;
    FixedDraft draft;
    GenerationRequest req;
    req.prompt = {1, 2, 1, 2};
    req.max_tokens = 3;
    req.layer_count = 2;
    GenerationResult r = run_generation(ex, req, &draft, 2);
    expect(r.ok, "speculative generation succeeds");
    expect(r.sampled_tokens == std::vector<std::uint32_t>({10, 20, 99}), "accepted prefix + correction emitted");
    expect(r.target_decode_passes == 1, "one verify pass");
    expect(r.speculative_draft_tokens == 2 && r.speculative_accepted_tokens == 1, "acceptance telemetry");
    expect(ex.rollback_calls == 1 && ex.last_rollback == 1, "rejected suffix of 1 rolled back once");
    expect(ex.passes.size() == 1 && ex.passes[0] == std::vector<std::int32_t>({10, 20, 21}),
           "verification rows are [previous] + draft");
    expect(ex.steps.size() == 1 && ex.steps[0] == 1, "first decode pass is step 1");
    expect(ex.close_calls == 1, "session closed once");
    expect(r.finish_reason == "length", "finish reason length");
}

void test_recovery_pass_after_rejection() {
    ScriptedExecutor ex;
    FixedDraft draft;
    GenerationRequest req;
    req.prompt = {1, 2, 1, 2};
    req.max_tokens = 5;
    GenerationResult r = run_generation(ex, req, &draft, 2);
    expect(r.ok, "generation succeeds");
    // pass 1 verifies [10, 20, 21] -> emits 20, 99 and rolls back 1; pass 2 is a
    // forced single-token pass [99]; pass 3 drafts nothing for the new history.
    expect(ex.passes.size() == 3, "three passes");
    if (ex.passes.size() == 3) {
        expect(ex.passes[1] == std::vector<std::int32_t>({99}), "recovery pass is single-token");
        expect(ex.steps[1] == 3, "decode_step advances by len(verification) - rollback");
        expect(ex.steps[2] == 4, "decode_step advances by one after a single-token pass");
    }
    expect(r.sampled_tokens == std::vector<std::uint32_t>({10, 20, 99, 20, 20}), "emitted stream");
}

void test_rollback_failure_emits_nothing_rejected() {
    ScriptedExecutor ex;
    ex.fail_rollback = true;
    FixedDraft draft;
    GenerationRequest req;
    req.prompt = {1, 2, 1, 2};
    req.max_tokens = 3;
    GenerationResult r = run_generation(ex, req, &draft, 2);
    expect(!r.ok, "rollback failure fails the generation");
    expect(r.error_code == "generation_rollback_failed", "rollback failure code");
    expect(r.sampled_tokens == std::vector<std::uint32_t>({10}), "no token of the rejected pass is emitted");
    expect(ex.close_calls == 1, "session closed after the failure");
}

void test_payloads() {
    const std::int32_t ids[] = {3, 0, 151935, 7};
    inference::Payload p = inference::tokens_payload(ids);
    expect(p.bytes.size() == 16 && p.tensor.dtype == "i32", "token payload is i32 little-endian");
    expect(inference::decode_token_ids(p) == std::vector<std::int32_t>({3, 0, 151935, 7}), "token payload round trip");
    inference::Payload u;
    u.kind = inference::PayloadKind::Tokens;
    u.tensor.dtype = "u32";
    u.tensor.shape = {2};
    u.tensor.byte_order = "little";
    u.tensor.layout = "row_major";
    u.bytes = {5, 0, 0, 0, 1, 1, 0, 0};
    expect(inference::decode_token_ids(u) == std::vector<std::int32_t>({5, 257}), "u32 token payload decodes");
    inference::StageInput in;
    in.session_id = "s";
    in.request_id = "r";
    in.model_id = "m";
    in.layers = {0, 2};
    in.payload = p;
    expect(inference::validate_stage_input(in).empty(), "valid stage input accepted");
    in.session_id.clear();
    expect(!inference::validate_stage_input(in).empty(), "missing session id rejected");
}

// Answers decode rows with row + 1 and records the batches it is handed.
class BatchRecorder final : public inference::Executor {
public:
    mutable std::mutex mutex;
    mutable std::vector<std::size_t> batches;
    mutable int prefills = 0, closes = 0, rollbacks = 0;
    bool fail_batches = false;
    bool throw_non_standard = false;  // execute_batch throws an int
    bool short_batches = false;  // answers one step fewer than it is handed

    inference::ExecutionResult execute(const inference::StageInput& in) const override {
        inference::StageOutput out;
        const std::vector<std::int32_t> rows = inference::decode_token_ids(in.payload);
        if (in.phase == inference::Phase::Prefill) {
            ++prefills;
            out.payload = inference::sampled_token_payload(7);
        } else {
            out.payload = inference::sampled_token_payload(rows.at(0) + 1);
        }
        return inference::ExecutionResult::success(out);
    }
    std::vector<inference::ExecutionResult> execute_batch(
        const std::vector<inference::StageInput>& inputs) const override {
        {
            std::lock_guard lock(mutex);
            batches.push_back(inputs.size());
        }
        if (fail_batches) throw std::runtime_error("injected batch failure");
        if (throw_non_standard) throw 42;
        std::vector<inference::ExecutionResult> out;
        for (const auto& in : inputs) out.push_back(execute(in));
        if (short_batches) out.pop_back();
        return out;
    }
    void close_session(const std::string&) const override { ++closes; }
    void rollback_session(const std::string&, int) const override { ++rollbacks; }
};

inference::StageInput step_input(inference::Phase phase, const std::string& session, std::int32_t token) {
    inference::StageInput in;
    in.session_id = session;
    in.request_id = "r-" + session;
    in.model_id = "m";
    in.phase = phase;
    in.decode_step = phase == inference::Phase::Prefill ? 0 : 1;
    in.position = {0, 1};
    in.layers = {0, 1};
    const std::int32_t t[1] = {token};
    in.payload = inference::tokens_payload(std::span<const std::int32_t>(t, 1));
    in.max_tokens = 4;
    return in;
}

void test_continuous_batching() {
    using pipeline_parallel::ContinuousBatchingConfig;
    using pipeline_parallel::ContinuousBatchingExecutor;
    using std::chrono::microseconds;
    // two concurrent decode steps run as one batch
    {
        auto rec = std::make_unique<BatchRecorder>();
        const BatchRecorder* r = rec.get();
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{2, microseconds(2000000)});
        inference::ExecutionResult a, b;
        std::thread ta([&] { a = ex.execute(step_input(inference::Phase::Decode, "a", 10)); });
        std::thread tb([&] { b = ex.execute(step_input(inference::Phase::Decode, "b", 20)); });
        ta.join();
        tb.join();
        expect(a.ok && b.ok, "batched decode results are ok");
        expect(inference::decode_token_ids(a.output.payload) == std::vector<std::int32_t>{11}, "first result is its own");
        expect(inference::decode_token_ids(b.output.payload) == std::vector<std::int32_t>{21}, "second result is its own");
        expect(r->batches == std::vector<std::size_t>{2}, "two concurrent steps form one batch of two");
        // prefill is immediate and bypasses the batcher; rollback and close pass through
        const inference::ExecutionResult p = ex.execute(step_input(inference::Phase::Prefill, "c", 1));
        expect(p.ok && r->prefills == 1 && r->batches.size() == 1, "prefill runs immediately");
        ex.rollback_session("a", 1);
        ex.close_session("a");
        expect(r->rollbacks == 1 && r->closes == 1, "rollback and close reach the delegate");
    }
    // a lone step runs as a batch of one after the wait
    {
        auto rec = std::make_unique<BatchRecorder>();
        const BatchRecorder* r = rec.get();
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{2, microseconds(3000)});
        const auto t0 = std::chrono::steady_clock::now();
        const inference::ExecutionResult a = ex.execute(step_input(inference::Phase::Decode, "a", 5));
        const double waited = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        expect(a.ok && r->batches == std::vector<std::size_t>{1}, "a lone step runs alone");
        expect(waited >= 3000.0, "a lone step waits for the batch to fill");
    }
    // delegate failures reach every step of the batch
    {
        auto rec = std::make_unique<BatchRecorder>();
        rec->fail_batches = true;
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{2, microseconds(0)});
        const inference::ExecutionResult a = ex.execute(step_input(inference::Phase::Decode, "a", 5));
        expect(!a.ok && a.error.code == "continuous_batch_failed", "batch failure is reported per step");
    }
    // a delegate that throws something that is no std::exception: every step of
    // every batch gets the batch failure, nobody waits forever, and the
    // executor keeps serving (later steps lead new batches)
    {
        auto rec = std::make_unique<BatchRecorder>();
        rec->throw_non_standard = true;
        BatchRecorder* r = rec.get();
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{2, microseconds(1000)});
        std::vector<inference::ExecutionResult> res(5);
        std::vector<std::thread> ts;
        for (int i = 0; i < 5; ++i) {
            ts.emplace_back([&, i] { res[i] = ex.execute(step_input(inference::Phase::Decode, std::to_string(i), i)); });
        }
        for (auto& t : ts) t.join();
        for (const auto& x : res) {
            expect(!x.ok && x.error.code == "continuous_batch_failed", "a non-standard delegate exception fails the step");
        }
        r->throw_non_standard = false;
        const inference::ExecutionResult after = ex.execute(step_input(inference::Phase::Decode, "z", 9));
        expect(after.ok && inference::decode_token_ids(after.output.payload) == std::vector<std::int32_t>{10},
               "the executor serves steps after a failed batch");
    }
    // a delegate that answers the wrong number of steps fails every step of the batch
    {
        auto rec = std::make_unique<BatchRecorder>();
        rec->short_batches = true;
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{2, microseconds(0)});
        const inference::ExecutionResult a = ex.execute(step_input(inference::Phase::Decode, "a", 5));
        expect(!a.ok && a.error.code == "continuous_batch_result_mismatch", "a short batch answer is a mismatch");
    }
    // more concurrent steps than one batch holds: every step gets its own
    // answer, in batches of at most max_batch_size
    {
        auto rec = std::make_unique<BatchRecorder>();
        const BatchRecorder* r = rec.get();
        ContinuousBatchingExecutor ex(std::move(rec), ContinuousBatchingConfig{3, microseconds(2000)});
        std::vector<inference::ExecutionResult> res(8);
        std::vector<std::thread> ts;
        for (int i = 0; i < 8; ++i) {
            ts.emplace_back([&, i] { res[i] = ex.execute(step_input(inference::Phase::Decode, std::to_string(i), 100 * i)); });
        }
        for (auto& t : ts) t.join();
        std::size_t total = 0;
        for (const std::size_t b : r->batches) {
            expect(b >= 1 && b <= 3, "a batch holds at most max_batch_size steps");
            total += b;
        }
        expect(total == 8, "every step ran exactly once");
        for (int i = 0; i < 8; ++i) {
            expect(res[i].ok && inference::decode_token_ids(res[i].output.payload) == std::vector<std::int32_t>{100 * i + 1},
                   "every step gets its own answer");
        }
    }
    // configuration errors
    bool threw = false;
    try {
        ContinuousBatchingExecutor ex(std::make_unique<BatchRecorder>(), ContinuousBatchingConfig{1, microseconds(0)});
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    expect(threw, "batch size one is rejected");
    threw = false;
    try {
        ContinuousBatchingExecutor ex(nullptr, ContinuousBatchingConfig{2, microseconds(0)});
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    expect(threw, "a missing delegate is rejected");
}

}  // namespace

// activation_codec_test.cpp:60-99: factory registration and codec guards
void test_activation_codecs() {
    auto factory = activation::make_default_activation_codec_factory();
    expect(factory->supports("f32") && factory->supports("f16") && !factory->supports("missing"),
           "default factory registers f32 and f16 only");
    bool rejected = false;
    try {
        (void) factory->create_codec("missing");
    } catch (const std::invalid_argument&) {
        rejected = true;
    }
    expect(rejected, "unknown encoding is rejected");
    struct Misnamed final : activation::ActivationCodec {
        const std::string& name() const noexcept override {
            static const std::string n = "other";
            return n;
        }
        inference::Payload encode(inference::Payload p) const override { return p; }
        inference::Payload decode(inference::Payload p) const override { return p; }
    };
    activation::ActivationCodecFactory custom;
    custom.register_codec("registered", [] { return std::make_shared<Misnamed>(); });
    bool misnamed = false;
    try {
        (void) custom.create_codec("registered");
    } catch (const std::runtime_error&) {
        misnamed = true;
    }
    expect(misnamed, "a codec whose name differs from its registration is rejected");
    bool duplicate = false;
    try {
        custom.register_codec("registered", [] { return std::make_shared<Misnamed>(); });
    } catch (const std::invalid_argument&) {
        duplicate = true;
    }
    expect(duplicate, "a name registers once");

    const auto f16 = factory->create_codec("f16");
    inference::Payload p;
    p.kind = inference::PayloadKind::Activation;
    p.tensor.dtype = "f32";
    p.tensor.shape = {1, 3};
    for (const float v : {1.0F, -0.5F, 3.0e5F}) {
        std::uint8_t b[4];
        std::memcpy(b, &v, 4);
        p.bytes.insert(p.bytes.end(), b, b + 4);
    }
    const inference::Payload wire = f16->encode(p);
    expect(wire.tensor.dtype == "f16" && wire.bytes.size() == 6, "f16 wire payload is half the bytes");
    expect(wire.bytes[0] == 0x00 && wire.bytes[1] == 0x3C && wire.bytes[2] == 0x00 && wire.bytes[3] == 0xB8 &&
               wire.bytes[4] == 0x00 && wire.bytes[5] == 0x7C,
           "1, -0.5 and an overflowing value encode as 0x3C00, 0xB800, +inf");
    const inference::Payload back = f16->decode(wire);
    expect(back.tensor.dtype == "f32" && back.bytes.size() == 12, "decode restores f32 rows");
    bool wrong_dtype = false;
    try {
        (void) f16->decode(p);
    } catch (const std::invalid_argument&) {
        wrong_dtype = true;
    }
    expect(wrong_dtype, "f16 decode rejects an f32 payload");
    inference::Payload tokens;
    tokens.kind = inference::PayloadKind::Tokens;
    tokens.tensor.dtype = "f32";
    bool not_activation = false;
    try {
        (void) f16->encode(tokens);
    } catch (const std::invalid_argument&) {
        not_activation = true;
    }
    expect(not_activation, "codecs take activation payloads only");
}

int main() {
    test_prompt_lookup();
    test_activation_codecs();
    test_accepts_prefix_and_rolls_back_suffix();
    test_recovery_pass_after_rejection();
    test_rollback_failure_emits_nothing_rejected();
    test_payloads();
    test_continuous_batching();
    if (failures) {
        std::printf("%d runtime check(s) failed\n", failures);
        return 1;
    }
    std::printf("runtime tests passed\n");
    return 0;
}
