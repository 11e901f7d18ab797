// GPU test of pipeline stages behind the executor interface: a synthetic
// model written as a JFM package, opened whole and as two layer ranges; the
// two stage executors chained over activation payloads must sample the
// whole-model executor's tokens (same kernels on the same rows), and the
// stage contract's errors follow the reference's NativeStageExecutor
// (runtime/adapters/native_stage_executor.cpp:16-47, 84-104, 226-320;
// native_stage_executor_test.cpp:72-230). Built as a shared library whose
// jfh_stage_test_main tests/test_gpu_stages.py calls in its own process.
#include "jfh_runtime.hpp"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include <unistd.h>

using namespace jfh;
using namespace jfh::runtime;
using inference::ExecutionResult;
using inference::Payload;
using inference::PayloadKind;
using inference::Phase;
using inference::StageInput;

namespace {

int failures = 0;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        ++failures;
    }
}

StageInput input(const std::string& session, Phase phase, int step, int index, int count, int start, int end,
                 Payload payload) {
    StageInput in;
    in.session_id = session;
    in.request_id = "request-" + session;
    in.model_id = "synthetic";
    in.phase = phase;
    in.decode_step = step;
    in.position = {index, count};
    in.layers = {start, end};
    in.payload = std::move(payload);
    in.max_tokens = 8;
    return in;
}

Payload tokens(std::vector<std::int32_t> ids) { return inference::tokens_payload(ids); }

std::int32_t sampled(const ExecutionResult& r) {
    if (!r.ok) throw std::runtime_error("stage failed: " + r.error.code + ": " + r.error.message);
    const std::vector<std::int32_t> ids = inference::decode_token_ids(r.output.payload);
    if (ids.size() != 1) throw std::runtime_error("expected one sampled token");
    return ids[0];
}

}  // namespace

extern "C" int jfh_stage_test_main() try {
    failures = 0;
    SynthSpec spec;
    spec.params = {4, 256, 768, 4, 2, 512, 4096, 64, 1.0e6F, 1.0e-6F};
    spec.seed = 11;
    const std::filesystem::path dir = std::filesystem::temp_directory_path() / ("jfh_stage_test_" + std::to_string(::getpid()));
    std::filesystem::create_directories(dir);
    HostModel::synthesize(spec)->write_package(dir.string());
    auto open = [&](uint32_t a, uint32_t b) {
        StagePlan plan;
        plan.layer_start = a;
        plan.layer_end = b;
        return std::make_shared<Engine>(*HostModel::open_package(dir.string(), plan), EngineOptions{});
    };
    auto whole_engine = open(0, 4), first_engine = open(0, 2), last_engine = open(2, 4);
    std::filesystem::remove_all(dir);
    auto tok = std::make_shared<tokenization::IdTokenizer>();
    auto config = [&](std::shared_ptr<Engine> e, int index, int count, int start, int end) {
        adapters::HipStageConfig c;
        c.engine = std::move(e);
        c.tokenizer = tok;
        c.ctx_size = 128;
        c.position = {index, count};
        c.layers = {start, end};
        return c;
    };
    adapters::HipStageExecutor whole(config(whole_engine, 0, 1, 0, 4));
    adapters::HipStageExecutor first(config(first_engine, 0, 2, 0, 2));
    adapters::HipStageExecutor last(config(last_engine, 1, 2, 2, 4));

    // assignments must match the stage's resident layers (native_stage_executor.cpp:84-104)
    auto rejects = [&](std::shared_ptr<Engine> e, int index, int count, int start, int end, const char* msg) {
        try {
            adapters::HipStageExecutor bad(config(std::move(e), index, count, start, end));
            expect(false, std::string("accepted: ") + msg);
        } catch (const std::invalid_argument& ex) {
            expect(std::string(ex.what()) == msg, std::string("message: ") + ex.what());
        }
    };
    rejects(first_engine, 0, 2, 0, 3, "native stage exceeds its resident layer range");
    rejects(first_engine, 1, 2, 0, 2, "native serving stage assignment is invalid");
    rejects(last_engine, 0, 1, 2, 4, "native serving stage assignment is invalid");

    const std::vector<std::int32_t> prompt = {5, 17, 301, 42, 7, 7, 99, 1024, 3};
    std::int32_t want = sampled(whole.execute(input("w", Phase::Prefill, 0, 0, 1, 0, 4, tokens(prompt))));
    const ExecutionResult a = first.execute(input("s", Phase::Prefill, 0, 0, 2, 0, 2, tokens(prompt)));
    expect(a.ok, "first stage prefill");
    expect(a.output.payload.kind == PayloadKind::Activation && a.output.payload.tensor.dtype == "f32" &&
               a.output.payload.tensor.shape == std::vector<std::int64_t>({9, 256}) &&
               a.output.payload.bytes.size() == 9 * 256 * 4,
           "first stage returns f32[9, 256] activations");
    expect(a.output.prompt_tokens == 9, "first stage reports the prompt");
    std::int32_t got = sampled(last.execute(input("s", Phase::Prefill, 0, 1, 2, 2, 4, a.output.payload)));
    expect(got == want, "two-stage prefill samples the whole model's token");

    // the f16 wire codec between the stages still drives the last stage
    auto f16 = activation::make_default_activation_codec_factory()->create_codec("f16");
    const Payload wire = f16->encode(a.output.payload);
    expect(wire.bytes.size() == a.output.payload.bytes.size() / 2, "f16 halves the activation bytes");
    const ExecutionResult via_f16 = last.execute(input("h", Phase::Prefill, 0, 1, 2, 2, 4, f16->decode(wire)));
    expect(via_f16.ok, "last stage runs on f16-carried activations");

    for (int step = 1; step <= 4; ++step) {
        const std::int32_t w = sampled(whole.execute(input("w", Phase::Decode, step, 0, 1, 0, 4, tokens({want}))));
        const ExecutionResult x = first.execute(input("s", Phase::Decode, step, 0, 2, 0, 2, tokens({want})));
        expect(x.ok && x.output.payload.tensor.shape == std::vector<std::int64_t>({1, 256}), "first stage decode row");
        got = sampled(last.execute(input("s", Phase::Decode, step, 1, 2, 2, 4, x.output.payload)));
        expect(got == w, "two-stage decode step " + std::to_string(step) + " samples the whole model's token");
        want = w;
    }

    // stage payload errors
    const ExecutionResult wrong_kind = last.execute(input("e1", Phase::Prefill, 0, 1, 2, 2, 4, tokens({1, 2})));
    expect(!wrong_kind.ok && wrong_kind.error.code == "invalid_native_stage_input" &&
               wrong_kind.error.message == "native activation must be f32[sequence_length, hidden_size]",
           "later stage rejects token input: " + wrong_kind.error.message);
    const ExecutionResult two = first.execute(input("s", Phase::Decode, 5, 0, 2, 0, 2, tokens({1, 2})));
    expect(!two.ok && two.error.code == "native_multi_token_verification_unsupported",
           "a stage decodes one token per pass");
    const ExecutionResult mismatch = first.execute(input("s", Phase::Decode, 5, 0, 2, 0, 4, tokens({1})));
    expect(!mismatch.ok && mismatch.error.code == "native_stage_assignment_mismatch", "assignment mismatch");
    const ExecutionResult missing = last.execute(input("nope", Phase::Decode, 1, 1, 2, 2, 4, a.output.payload));
    expect(!missing.ok && missing.error.code == "stage_session_not_found", "decode without a session");

    // idle sessions are closed after their TTL (llama_cpp_stage_adapter_test.cpp:410-437)
    {
        adapters::HipStageConfig c = config(whole_engine, 0, 1, 0, 4);
        c.session_idle_ttl = std::chrono::milliseconds(30);
        c.session_reap_interval = std::chrono::milliseconds(5);
        adapters::HipStageExecutor expiring(c);
        const ExecutionResult p = expiring.execute(input("expiring", Phase::Prefill, 0, 0, 1, 0, 4, tokens(prompt)));
        expect(p.ok, "expiring stage prefill");
        expect(expiring.session_count() == 1U, "expiring stage retains its new session");
        const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(2);
        while (expiring.session_count() != 0U && std::chrono::steady_clock::now() < deadline) {
            std::this_thread::sleep_for(std::chrono::milliseconds(5));
        }
        expect(expiring.session_count() == 0U, "idle stage session is reaped after its TTL");
        const ExecutionResult gone = expiring.execute(input("expiring", Phase::Decode, 1, 0, 1, 0, 4, tokens({want})));
        expect(!gone.ok && gone.error.code == "stage_session_not_found", "a reaped session is gone");
        c.session_idle_ttl = std::chrono::milliseconds(0);
        try {
            adapters::HipStageExecutor bad(c);
            expect(false, "accepted a zero session TTL");
        } catch (const std::invalid_argument& ex) {
            expect(std::string(ex.what()) == "native session expiration intervals must be greater than zero",
                   std::string("message: ") + ex.what());
        }
    }
    expect(whole.session_count() == 1U, "sessions in use are not reaped");

    if (failures) {
        std::printf("%d stage check(s) failed\n", failures);
        return 1;
    }
    std::printf("stage tests passed\n");
    return 0;
} catch (const std::exception& e) {
    std::printf("FAIL: %s\n", e.what());
    return 1;
}
