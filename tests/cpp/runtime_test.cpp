// Host-side tests of the speculative runtime (no GPU): prompt-lookup
// drafting, the greedy acceptance / rollback loop over a scripted executor,
// and the stage payload helpers. Mirrors the reference's own cases in
// runtime/speculative/prompt_lookup_draft_test.cpp:15-36 and
// runtime/pipeline_parallel/generation_runner_test.cpp:108-190, 355-430.
#include "jfh_runtime.hpp"

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
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

}  // namespace

int main() {
    test_prompt_lookup();
    test_accepts_prefix_and_rolls_back_suffix();
    test_recovery_pass_after_rejection();
    test_rollback_failure_emits_nothing_rejected();
    test_payloads();
    if (failures) {
        std::printf("%d runtime check(s) failed\n", failures);
        return 1;
    }
    std::printf("runtime tests passed\n");
    return 0;
}
