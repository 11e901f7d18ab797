// The HIP engine behind the reference runtime's stage-engine interface: a
// jetsonfabric::runtime::inference::Executor (runtime/inference/executor.hpp:
// 14-39) over the engine's C ABI (include/jfh.h), written the way a
// maintainer would add it beside runtime/adapters/native_stage_executor.
// {hpp,cpp}. It compiles against the reference's own contract headers
// (runtime/inference/{executor,stage,token_payload}.hpp,
// runtime/tokenization/tokenizer.hpp) and nothing else of the reference.
//
// Semantics follow NativeStageExecutor (native_stage_executor.cpp:76-340):
// the same assignment checks and error codes, one engine session per stage
// session, prefill and one-row decode through every stage. The last stage of
// a whole-model executor also verifies k draft tokens in one pass (the
// decode payload [previous, draft...], answered with sampled_tokens as the
// llama.cpp adapter answers it, llama_cpp_stage_adapter.cpp:350-386) and runs
// execute_batch's decode steps as one multi-sequence engine step.
#pragma once

#include "inference/executor.hpp"
#include "tokenization/tokenizer.hpp"

#include "jfh.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace jetsonfabric::runtime::adapters {

struct HipStageConfig {
    jfh_engine* engine = nullptr;  // not owned; outlives the executor
    std::shared_ptr<const tokenization::Tokenizer> tokenizer;
    int ctx_size = 0;
    inference::StagePosition position;
    inference::LayerRange layers;
    int speculative_max_tokens = 8;  // verify width - 1 (worker/config.cpp:105-107)
};

// The reference's tokenizer interface (runtime/tokenization/tokenizer.hpp:
// 10-17) over the engine's C-ABI tokenizer: the drop-in for
// LlamaCppTokenizer (runtime/adapters/llama_cpp_tokenizer.hpp:11-31), from a
// package directory's metadata.gguf or a GGUF file.
class CAbiTokenizer final : public tokenization::Tokenizer {
public:
    explicit CAbiTokenizer(const std::string& path);
    ~CAbiTokenizer() override;
    CAbiTokenizer(const CAbiTokenizer&) = delete;
    CAbiTokenizer& operator=(const CAbiTokenizer&) = delete;

    std::vector<std::int32_t> tokenize(std::string_view text) const override;
    std::string token_piece(std::int32_t token) const override;
    bool is_end_token(std::int32_t token) const override;
    // the end-of-generation ids, for jfh_engine_set_end_tokens
    std::vector<std::int32_t> end_tokens() const;

private:
    jfh_tokenizer* handle_ = nullptr;
};

class HipStageExecutor final : public inference::Executor {
public:
    explicit HipStageExecutor(HipStageConfig config);
    ~HipStageExecutor() override;
    HipStageExecutor(const HipStageExecutor&) = delete;
    HipStageExecutor& operator=(const HipStageExecutor&) = delete;

    inference::ExecutionResult execute(const inference::StageInput& input) const override;
    std::vector<inference::ExecutionResult> execute_batch(
        const std::vector<inference::StageInput>& inputs) const override;
    void close_session(const std::string& session_id) const override;
    void rollback_session(const std::string& session_id, int token_count) const override;
    std::size_t session_count() const;

private:
    struct Session {
        jfh_session* handle = nullptr;
        int expected_decode_step = 1;
    };

    inference::ExecutionResult execute_locked(const inference::StageInput& input) const;
    inference::ExecutionResult prefill(const inference::StageInput& input) const;
    inference::ExecutionResult decode(const inference::StageInput& input) const;
    bool assignment_matches(const inference::StageInput& input) const;
    bool whole_model() const;
    std::vector<std::int32_t> input_tokens(const inference::StageInput& input) const;
    std::vector<float> input_activation(const inference::Payload& payload) const;
    inference::StageOutput token_output(std::int32_t token) const;
    inference::StageOutput rows_output(const std::vector<std::int32_t>& tokens) const;
    inference::Payload activation_payload(const std::vector<float>& rows) const;
    std::size_t session_capacity(std::size_t prompt_tokens, int max_tokens) const;
    void close_all() const;

    HipStageConfig config_;
    jfh_model_params params_{};
    mutable std::mutex mutex_;
    mutable std::unordered_map<std::string, Session> sessions_;
};

}  // namespace jetsonfabric::runtime::adapters
