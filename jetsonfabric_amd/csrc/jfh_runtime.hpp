// Stage-engine contract and speculative generation loop around the HIP engine.
//
// The types mirror the reference runtime so the engine can be dropped in
// behind its Executor interface:
//   inference::{Payload, StageInput, StageOutput, ExecutionResult, Executor}
//     runtime/inference/stage.hpp:9-110, runtime/inference/executor.hpp:14-39,
//     token codecs runtime/inference/token_payload.cpp:36-80
//   speculative::{DraftStrategy, PromptLookupDraft}
//     runtime/speculative/draft_strategy.hpp:9-17, prompt_lookup_draft.cpp:8-44
//   adapters::HipStageExecutor -- NativeStageExecutor semantics
//     (runtime/adapters/native_stage_executor.cpp:76-340) plus multi-token
//     verification and rollback as the llama.cpp adapter provides them
//     (runtime/adapters/llama_cpp_stage_adapter.cpp:350-475, 895-937)
//   run_generation -- GenerationRunner::run for one local stage
//     (runtime/pipeline_parallel/generation_runner.cpp:398-566)
//   pipeline_parallel::ContinuousBatchingExecutor -- coalesces concurrent
//     decode steps into execute_batch calls
//     (runtime/pipeline_parallel/continuous_batching_executor.{hpp,cpp})
//   activation::{ActivationCodec, ActivationCodecFactory} -- the f32 / f16
//     codecs of activations between pipeline stages
//     (runtime/activation/activation_codec.hpp:9-18,
//     activation_codec_factory.cpp:8-46, builtin_activation_codecs.cpp)
#pragma once

#include "jfh_engine.hpp"

#include <chrono>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <span>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace jfh::runtime {

namespace inference {

enum class Phase { Prefill, Decode };
enum class PayloadKind { Text, Tokens, Activation, SampledToken, SampledTokens };
enum class ErrorKind { InvalidInput, ExecutionFailure };

struct StagePosition {
    int index = 0;
    int count = 1;
    bool is_first() const { return index == 0; }
    bool is_last() const { return index == count - 1; }
};

struct LayerRange {
    int start = 0;
    int end = 0;
};

struct TensorDescriptor {
    std::string dtype;
    std::vector<std::int64_t> shape;
    std::string byte_order;
    std::string layout;
};

struct Payload {
    PayloadKind kind = PayloadKind::Text;
    std::string encoding;
    TensorDescriptor tensor;
    std::vector<std::uint8_t> bytes;
};

struct StageInput {
    std::string session_id;
    std::string request_id;
    std::string model_id;
    Phase phase = Phase::Prefill;
    int decode_step = 0;
    StagePosition position;
    LayerRange layers;
    Payload payload;
    int max_tokens = 128;
};

struct StageOutput {
    Payload payload;
    int prompt_tokens = 0;
    std::vector<std::uint32_t> prompt_token_ids;
    int completion_tokens = 0;
    int execution_batch_size = 1;
    int verification_width = 1;
    std::string token_text;
    std::vector<std::uint32_t> token_text_offsets;
    std::vector<std::uint8_t> token_eog;
    bool end_of_generation = false;
};

struct ExecutionError {
    ErrorKind kind = ErrorKind::ExecutionFailure;
    std::string code;
    std::string message;
};

struct ExecutionResult {
    bool ok = false;
    StageOutput output;
    ExecutionError error;

    static ExecutionResult success(StageOutput output);
    static ExecutionResult invalid_input(std::string code, std::string message);
    static ExecutionResult failure(std::string code, std::string message);
};

class Executor {
public:
    virtual ~Executor() = default;
    virtual ExecutionResult execute(const StageInput& input) const = 0;
    virtual std::vector<ExecutionResult> execute_batch(const std::vector<StageInput>& inputs) const {
        std::vector<ExecutionResult> results;
        results.reserve(inputs.size());
        for (const StageInput& input : inputs) results.push_back(execute(input));
        return results;
    }
    virtual void close_session(const std::string& session_id) const { (void) session_id; }
    virtual void rollback_session(const std::string& session_id, int token_count) const;
};

std::string validate_stage_input(const StageInput& input);
std::vector<std::int32_t> decode_token_ids(const Payload& payload);
Payload tokens_payload(std::span<const std::int32_t> tokens);
Payload sampled_token_payload(std::int32_t token);
Payload sampled_tokens_payload(std::span<const std::int32_t> tokens);

}  // namespace inference

namespace tokenization {

// Tokenizer surface the stage adapter needs (runtime/tokenization/tokenizer.hpp).
class Tokenizer {
public:
    virtual ~Tokenizer() = default;
    virtual std::vector<std::int32_t> tokenize(std::string_view text) const = 0;
    virtual std::string token_piece(std::int32_t token) const = 0;
    virtual bool is_end_token(std::int32_t token) const = 0;
};

// Token-id tokenizer for synthetic models: text is whitespace-separated ids,
// a piece is the decimal id followed by a space, end tokens are configured.
class IdTokenizer final : public Tokenizer {
public:
    explicit IdTokenizer(std::vector<std::int32_t> end_tokens = {}) : end_tokens_(std::move(end_tokens)) {}
    std::vector<std::int32_t> tokenize(std::string_view text) const override;
    std::string token_piece(std::int32_t token) const override;
    bool is_end_token(std::int32_t token) const override;

private:
    std::vector<std::int32_t> end_tokens_;
};

}  // namespace tokenization

namespace speculative {

class DraftStrategy {
public:
    virtual ~DraftStrategy() = default;
    virtual std::vector<std::uint32_t> propose(const std::vector<std::uint32_t>& history,
                                               std::size_t max_tokens) const = 0;
};

class PromptLookupDraft final : public DraftStrategy {
public:
    explicit PromptLookupDraft(std::size_t max_ngram = 4, std::size_t min_ngram = 2);
    std::vector<std::uint32_t> propose(const std::vector<std::uint32_t>& history,
                                       std::size_t max_tokens) const override;

private:
    std::size_t max_ngram_;
    std::size_t min_ngram_;
};

}  // namespace speculative

namespace activation {

// IEEE 754 binary16 conversions: f32 -> f16 rounds to nearest, ties to even
// (overflow to infinity, gradual underflow to subnormals and signed zero);
// NaNs stay NaNs with the quiet bit set and the top ten payload bits kept.
// f16 -> f32 is exact.
std::uint16_t f32_to_f16(float value);
float f16_to_f32(std::uint16_t value);

// Converts activation payloads between the engine's f32 rows and the
// representation carried between pipeline stages.
class ActivationCodec {
public:
    virtual ~ActivationCodec() = default;
    virtual const std::string& name() const noexcept = 0;
    virtual inference::Payload encode(inference::Payload payload) const = 0;
    virtual inference::Payload decode(inference::Payload payload) const = 0;
};

class ActivationCodecFactory {
public:
    using Builder = std::function<std::shared_ptr<const ActivationCodec>()>;
    void register_codec(std::string name, Builder builder);
    bool supports(const std::string& name) const;
    std::shared_ptr<const ActivationCodec> create_codec(const std::string& name) const;

private:
    std::unordered_map<std::string, Builder> builders_;
};

// "f32" (identity) and "f16" (half the wire bytes).
std::shared_ptr<const ActivationCodecFactory> make_default_activation_codec_factory();

}  // namespace activation

namespace adapters {

struct HipStageConfig {
    std::shared_ptr<Engine> engine;
    std::shared_ptr<const tokenization::Tokenizer> tokenizer;
    int ctx_size = 0;
    inference::StagePosition position;
    inference::LayerRange layers;
    int speculative_max_tokens = 8;  // verify width limit - 1 (worker/config.cpp:105-107)
    // A session unused for session_idle_ttl is closed (its KV cache freed), checked
    // every session_reap_interval and at every call, so that a caller that fails
    // between steps cannot hold device memory forever (the reference's stage
    // adapter, llama_cpp_stage_adapter.hpp:26-33, .cpp:151-153, 193-196, 939-967).
    std::chrono::milliseconds session_idle_ttl = std::chrono::minutes(5);
    std::chrono::milliseconds session_reap_interval = std::chrono::seconds(1);
};

class HipStageExecutor final : public inference::Executor {
public:
    explicit HipStageExecutor(HipStageConfig config);
    ~HipStageExecutor() override;

    inference::ExecutionResult execute(const inference::StageInput& input) const override;
    std::vector<inference::ExecutionResult> execute_batch(const std::vector<inference::StageInput>& inputs) const override;
    void close_session(const std::string& session_id) const override;
    void rollback_session(const std::string& session_id, int token_count) const override;
    std::size_t session_count() const;

private:
    class Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace adapters

struct GenerationRequest {
    std::string session_id = "session";
    std::string request_id = "request";
    std::string model_id = "model";
    std::vector<std::int32_t> prompt;
    int max_tokens = 16;
    int layer_count = 0;
    // Called once after the prefill's token is read and before the first
    // decode pass (no counterpart in the reference runner: it lets a caller
    // start the decode phases of several runners together).
    std::function<void()> after_prefill;
};

struct GenerationResult {
    bool ok = false;
    std::vector<std::uint32_t> sampled_tokens;
    int completion_tokens = 0;
    int target_decode_passes = 0;
    int speculative_draft_tokens = 0;
    int speculative_accepted_tokens = 0;
    std::string finish_reason;
    std::string error_code;
    std::string error_message;
    double time_to_first_token_ms = 0.0;
    double decode_ms = 0.0;
    // when the last token was read (before the session is closed)
    std::chrono::steady_clock::time_point decode_end{};
};

// GenerationRunner::run restricted to one local stage that owns every layer.
GenerationResult run_generation(const inference::Executor& executor, const GenerationRequest& request,
                                const speculative::DraftStrategy* draft, int speculative_max_tokens);

namespace pipeline_parallel {

// continuous_batching_executor.hpp:11-14
struct ContinuousBatchingConfig {
    std::size_t max_batch_size = 1;
    std::chrono::microseconds max_wait = std::chrono::microseconds(500);
};

// Coalesces concurrently arriving decode steps into delegate execute_batch
// calls of up to max_batch_size steps, waiting at most max_wait for a batch
// to fill; the submitting threads themselves form and run the batches (one
// of them leads each batch). Prefill runs immediately on the caller's thread.
// Contract and error codes of the reference's decorator
// (continuous_batching_executor.hpp:16-39, continuous_batching_executor.cpp:
// 44-127): continuous_batch_failed, continuous_batch_result_mismatch.
class ContinuousBatchingExecutor final : public inference::Executor {
public:
    ContinuousBatchingExecutor(std::unique_ptr<inference::Executor> delegate, ContinuousBatchingConfig config);
    ~ContinuousBatchingExecutor() override;
    ContinuousBatchingExecutor(const ContinuousBatchingExecutor&) = delete;
    ContinuousBatchingExecutor& operator=(const ContinuousBatchingExecutor&) = delete;

    inference::ExecutionResult execute(const inference::StageInput& input) const override;
    std::vector<inference::ExecutionResult> execute_batch(const std::vector<inference::StageInput>& inputs) const override;
    void close_session(const std::string& session_id) const override;
    void rollback_session(const std::string& session_id, int token_count) const override;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace pipeline_parallel

}  // namespace jfh::runtime
