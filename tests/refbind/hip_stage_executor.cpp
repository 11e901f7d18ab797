#include "hip_stage_executor.hpp"

#include "inference/token_payload.hpp"

#include <cstring>
#include <limits>
#include <stdexcept>
#include <string_view>
#include <utility>

namespace jetsonfabric::runtime::adapters {

namespace {
[[noreturn]] void tokenizer_fail(const jfh_status& s) {
    // the messages LlamaCppTokenizer's callers see: invalid input as std::invalid_argument
    if (s.code == JFH_STATUS_INVALID_ARGUMENT || s.code == JFH_STATUS_NOT_FOUND || s.code == JFH_STATUS_FORMAT_ERROR) {
        throw std::invalid_argument(s.message);
    }
    throw std::runtime_error(s.message);
}
}  // namespace

CAbiTokenizer::CAbiTokenizer(const std::string& path) {
    const jfh_status s = jfh_tokenizer_open(path.c_str(), &handle_);
    if (s.code != JFH_STATUS_OK) tokenizer_fail(s);
}

CAbiTokenizer::~CAbiTokenizer() { jfh_tokenizer_destroy(handle_); }

std::vector<std::int32_t> CAbiTokenizer::tokenize(std::string_view text) const {
    uint32_t n = 0;
    jfh_status s = jfh_tokenizer_tokenize(handle_, text.data(), text.size(), nullptr, 0, &n);
    if (s.code != JFH_STATUS_OK && n == 0) tokenizer_fail(s);
    std::vector<std::int32_t> ids(n);
    s = jfh_tokenizer_tokenize(handle_, text.data(), text.size(), ids.data(), n, &n);
    if (s.code != JFH_STATUS_OK) tokenizer_fail(s);
    return ids;
}

std::string CAbiTokenizer::token_piece(std::int32_t token) const {
    uint32_t n = 0;
    jfh_status s = jfh_tokenizer_token_piece(handle_, token, nullptr, 0, &n);
    if (s.code != JFH_STATUS_OK && n == 0) tokenizer_fail(s);
    std::string piece(n, '\0');
    s = jfh_tokenizer_token_piece(handle_, token, piece.data(), n, &n);
    if (s.code != JFH_STATUS_OK) tokenizer_fail(s);
    return piece;
}

bool CAbiTokenizer::is_end_token(std::int32_t token) const {
    uint32_t out = 0;
    const jfh_status s = jfh_tokenizer_is_end_token(handle_, token, &out);
    if (s.code != JFH_STATUS_OK) tokenizer_fail(s);
    return out != 0;
}

std::vector<std::int32_t> CAbiTokenizer::end_tokens() const {
    uint32_t n = 0;
    jfh_status s = jfh_tokenizer_end_tokens(handle_, nullptr, 0, &n);
    if (s.code != JFH_STATUS_OK && n == 0) tokenizer_fail(s);
    std::vector<std::int32_t> ids(n);
    s = jfh_tokenizer_end_tokens(handle_, ids.data(), n, &n);
    if (s.code != JFH_STATUS_OK) tokenizer_fail(s);
    return ids;
}
namespace {

using inference::ExecutionResult;
using inference::Payload;
using inference::PayloadKind;
using inference::Phase;
using inference::StageInput;
using inference::StageOutput;

// A failed C ABI call. Invalid arguments become invalid_input results, every
// other status an execution failure (native_stage_executor.cpp:110-140).
class AbiError : public std::runtime_error {
public:
    AbiError(int code, const char* message) : std::runtime_error(message), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

void ok(const jfh_status& status) {
    if (status.code != JFH_STATUS_OK) throw AbiError(status.code, status.message);
}

constexpr std::size_t kMaxBatchSequences = 16;  // sequences of one engine step
constexpr std::size_t kMaxBatchRows = 64;       // token rows of one engine step

}  // namespace

HipStageExecutor::HipStageExecutor(HipStageConfig config) : config_(std::move(config)) {
    if (config_.engine == nullptr || !config_.tokenizer) {
        throw std::invalid_argument("native executor requires engine and tokenizer");
    }
    if (config_.ctx_size <= 0) throw std::invalid_argument("native executor context size must be positive");
    ok(jfh_engine_get_params(config_.engine, &params_));
    jfh_engine_info info{};
    ok(jfh_engine_get_info(config_.engine, &info));
    const int layer_count = static_cast<int>(params_.n_layer);
    const inference::StagePosition& pos = config_.position;
    if (pos.count <= 0 || pos.index < 0 || pos.index >= pos.count || config_.layers.start < 0 ||
        config_.layers.end <= config_.layers.start || config_.layers.end > layer_count ||
        (pos.is_first() && config_.layers.start != 0) || (pos.is_last() && config_.layers.end != layer_count)) {
        throw std::invalid_argument("native serving stage assignment is invalid");
    }
    if (config_.layers.start != static_cast<int>(info.layer_start) ||
        config_.layers.end != static_cast<int>(info.layer_end)) {
        throw std::invalid_argument("native stage exceeds its resident layer range");
    }
    if (static_cast<std::uint32_t>(config_.ctx_size) > params_.n_ctx) {
        throw std::invalid_argument("native context size exceeds model context");
    }
    if (config_.speculative_max_tokens < 0 || config_.speculative_max_tokens > 8) {
        throw std::invalid_argument("speculative width must be 0..8");
    }
}

HipStageExecutor::~HipStageExecutor() { close_all(); }

void HipStageExecutor::close_all() const {
    for (auto& [id, s] : sessions_) jfh_session_destroy(s.handle);
    sessions_.clear();
}

ExecutionResult HipStageExecutor::execute(const StageInput& input) const {
    const std::lock_guard lock(mutex_);
    return execute_locked(input);
}

ExecutionResult HipStageExecutor::execute_locked(const StageInput& input) const {
    try {
        const std::string error = inference::validate_stage_input(input);
        if (!error.empty()) return ExecutionResult::invalid_input("invalid_native_stage_input", error);
        if (!assignment_matches(input)) {
            return ExecutionResult::invalid_input("native_stage_assignment_mismatch",
                                                  "stage input does not match the configured native assignment");
        }
        return input.phase == Phase::Prefill ? prefill(input) : decode(input);
    } catch (const std::invalid_argument& e) {
        return ExecutionResult::invalid_input("invalid_native_stage_input", e.what());
    } catch (const AbiError& e) {
        if (e.code() == JFH_STATUS_INVALID_ARGUMENT) {
            return ExecutionResult::invalid_input("invalid_native_stage_input", e.what());
        }
        return ExecutionResult::failure("native_stage_execution_failed", e.what());
    } catch (const std::exception& e) {
        return ExecutionResult::failure("native_stage_execution_failed", e.what());
    }
}

std::vector<ExecutionResult> HipStageExecutor::execute_batch(const std::vector<StageInput>& inputs) const {
    const std::lock_guard lock(mutex_);
    std::vector<ExecutionResult> results(inputs.size());
    std::vector<std::size_t> batch;
    std::vector<jfh_session*> handles;
    std::vector<std::int32_t> tokens;
    std::vector<std::uint32_t> lengths;
    for (std::size_t i = 0; i < inputs.size(); ++i) {
        const StageInput& in = inputs[i];
        bool batchable = whole_model() && in.phase == Phase::Decode && inference::validate_stage_input(in).empty() &&
                         assignment_matches(in) && batch.size() < kMaxBatchSequences;
        std::vector<std::int32_t> mine;
        if (batchable) {
            const auto it = sessions_.find(in.session_id);
            batchable = it != sessions_.end() && in.decode_step == it->second.expected_decode_step;
            for (const std::size_t j : batch) batchable = batchable && inputs[j].session_id != in.session_id;
            if (batchable) {
                try {
                    mine = input_tokens(in);
                } catch (const std::exception&) {
                    batchable = false;
                }
                batchable = batchable && !mine.empty() &&
                            mine.size() <= static_cast<std::size_t>(config_.speculative_max_tokens + 1) &&
                            tokens.size() + mine.size() <= kMaxBatchRows;
            }
            if (batchable) handles.push_back(it->second.handle);
        }
        if (!batchable) {
            results[i] = execute_locked(in);
            continue;
        }
        batch.push_back(i);
        lengths.push_back(static_cast<std::uint32_t>(mine.size()));
        tokens.insert(tokens.end(), mine.begin(), mine.end());
    }
    if (batch.empty()) return results;
    std::vector<std::int32_t> ids(tokens.size());
    try {
        ok(jfh_engine_step_batch(config_.engine, handles.data(), static_cast<std::uint32_t>(handles.size()),
                                 tokens.data(), lengths.data(), ids.data(), nullptr, nullptr));
    } catch (const std::exception& e) {
        for (const std::size_t i : batch) results[i] = ExecutionResult::failure("native_stage_execution_failed", e.what());
        return results;
    }
    std::size_t offset = 0;
    for (std::size_t k = 0; k < batch.size(); ++k) {
        const StageInput& in = inputs[batch[k]];
        const std::size_t n = lengths[k];
        sessions_.at(in.session_id).expected_decode_step += static_cast<int>(n);
        const std::vector<std::int32_t> rows(ids.begin() + static_cast<std::ptrdiff_t>(offset),
                                             ids.begin() + static_cast<std::ptrdiff_t>(offset + n));
        StageOutput out = n > 1 ? rows_output(rows) : token_output(rows[0]);
        out.execution_batch_size = static_cast<int>(batch.size());
        results[batch[k]] = ExecutionResult::success(std::move(out));
        offset += n;
    }
    return results;
}

void HipStageExecutor::close_session(const std::string& session_id) const {
    const std::lock_guard lock(mutex_);
    const auto it = sessions_.find(session_id);
    if (it == sessions_.end()) return;
    jfh_session_destroy(it->second.handle);
    sessions_.erase(it);
}

void HipStageExecutor::rollback_session(const std::string& session_id, int token_count) const {
    const std::lock_guard lock(mutex_);
    if (token_count <= 0) throw std::invalid_argument("rollback token count must be positive");
    const auto it = sessions_.find(session_id);
    if (it == sessions_.end()) throw std::invalid_argument("native stage session not found");
    Session& s = it->second;
    if (token_count >= s.expected_decode_step) throw std::invalid_argument("rollback exceeds the decoded native suffix");
    ok(jfh_session_rollback(s.handle, static_cast<std::uint32_t>(token_count)));
    s.expected_decode_step -= token_count;
}

std::size_t HipStageExecutor::session_count() const {
    const std::lock_guard lock(mutex_);
    return sessions_.size();
}

ExecutionResult HipStageExecutor::prefill(const StageInput& in) const {
    if (sessions_.count(in.session_id) != 0) {
        return ExecutionResult::invalid_input("duplicate_stage_session",
                                              "prefill session already exists on this native stage");
    }
    std::vector<std::int32_t> tokens;
    std::vector<float> act;
    std::size_t count = 0;
    if (config_.position.is_first()) {
        tokens = input_tokens(in);
        count = tokens.size();
    } else {
        act = input_activation(in.payload);
        count = act.size() / params_.n_embd;
    }
    if (count == 0) throw std::invalid_argument("native Qwen2 prefill is outside session capacity");
    const std::size_t capacity = session_capacity(count, in.max_tokens);
    jfh_session* handle = nullptr;
    ok(jfh_session_create(config_.engine, static_cast<std::uint32_t>(capacity), &handle));
    std::unique_ptr<jfh_session, void (*)(jfh_session*)> owned(handle, jfh_session_destroy);
    const bool last = config_.position.is_last();
    std::int32_t token = -1;
    std::vector<float> out_rows(last ? 0 : count * params_.n_embd);
    if (whole_model()) {
        ok(jfh_session_prefill(handle, tokens.data(), static_cast<std::uint32_t>(count), &token, nullptr));
    } else {
        ok(jfh_session_stage_prefill(handle, tokens.empty() ? nullptr : tokens.data(),
                                     act.empty() ? nullptr : act.data(), static_cast<std::uint32_t>(count),
                                     last ? &token : nullptr, last ? nullptr : out_rows.data(), nullptr));
    }
    StageOutput out;
    if (last) {
        out = token_output(token);
    } else {
        out.payload = activation_payload(out_rows);
        out.execution_batch_size = 1;
    }
    if (config_.position.is_first()) {
        out.prompt_tokens = static_cast<int>(tokens.size());
        for (const std::int32_t t : tokens) {
            if (t < 0) throw std::invalid_argument("native tokenizer returned a negative token");
            out.prompt_token_ids.push_back(static_cast<std::uint32_t>(t));
        }
    }
    sessions_.emplace(in.session_id, Session{owned.release(), 1});
    return ExecutionResult::success(std::move(out));
}

ExecutionResult HipStageExecutor::decode(const StageInput& in) const {
    const auto it = sessions_.find(in.session_id);
    if (it == sessions_.end()) {
        return ExecutionResult::invalid_input("stage_session_not_found",
                                              "decode requires an existing native prefill session");
    }
    Session& s = it->second;
    if (in.decode_step != s.expected_decode_step) {
        return ExecutionResult::invalid_input("unexpected_decode_step", "native decode step does not match session state");
    }
    const bool last = config_.position.is_last();
    if (!whole_model()) {
        std::vector<std::int32_t> tokens;
        std::vector<float> act;
        if (config_.position.is_first()) {
            tokens = input_tokens(in);
            if (tokens.size() != 1U) {
                return ExecutionResult::invalid_input("native_multi_token_verification_unsupported",
                                                      "native serving currently accepts one decode token per pass");
            }
        } else {
            act = input_activation(in.payload);
            if (act.size() != params_.n_embd) {
                return ExecutionResult::invalid_input("native_multi_token_verification_unsupported",
                                                      "native decode activation must contain one token row");
            }
        }
        std::int32_t token = -1;
        std::vector<float> out_row(last ? 0 : params_.n_embd);
        ok(jfh_session_stage_decode(s.handle, tokens.empty() ? nullptr : tokens.data(),
                                    act.empty() ? nullptr : act.data(), last ? &token : nullptr,
                                    last ? nullptr : out_row.data(), nullptr));
        ++s.expected_decode_step;
        if (last) return ExecutionResult::success(token_output(token));
        StageOutput out;
        out.payload = activation_payload(out_row);
        out.execution_batch_size = 1;
        return ExecutionResult::success(std::move(out));
    }
    const std::vector<std::int32_t> tokens = input_tokens(in);
    if (tokens.empty() || tokens.size() > static_cast<std::size_t>(config_.speculative_max_tokens + 1)) {
        return ExecutionResult::invalid_input("invalid_verification_width",
                                              "native decode accepts 1..speculative_max_tokens+1 tokens per pass");
    }
    std::vector<std::int32_t> ids(tokens.size());
    if (tokens.size() == 1) {
        ok(jfh_session_decode(s.handle, tokens[0], ids.data(), nullptr));
    } else {
        ok(jfh_session_verify(s.handle, tokens.data(), static_cast<std::uint32_t>(tokens.size()), ids.data(), nullptr,
                              nullptr));
    }
    s.expected_decode_step += static_cast<int>(tokens.size());
    return ExecutionResult::success(tokens.size() > 1 ? rows_output(ids) : token_output(ids[0]));
}

bool HipStageExecutor::assignment_matches(const StageInput& in) const {
    return in.position.index == config_.position.index && in.position.count == config_.position.count &&
           in.layers.start == config_.layers.start && in.layers.end == config_.layers.end;
}

bool HipStageExecutor::whole_model() const { return config_.position.is_first() && config_.position.is_last(); }

std::vector<std::int32_t> HipStageExecutor::input_tokens(const StageInput& in) const {
    if (in.payload.kind == PayloadKind::Text) {
        return config_.tokenizer->tokenize(
            std::string_view(reinterpret_cast<const char*>(in.payload.bytes.data()), in.payload.bytes.size()));
    }
    if (in.payload.kind == PayloadKind::Tokens || in.payload.kind == PayloadKind::SampledToken) {
        return inference::decode_token_ids(in.payload);
    }
    throw std::invalid_argument("native first stage requires text or token input");
}

// f32[sequence_length, hidden_size] (native_stage_executor.cpp:16-45)
std::vector<float> HipStageExecutor::input_activation(const Payload& p) const {
    const std::int64_t hidden = params_.n_embd;
    if (p.kind != PayloadKind::Activation || p.tensor.dtype != "f32" || p.tensor.shape.size() != 2 ||
        p.tensor.shape[0] <= 0 || p.tensor.shape[1] != hidden) {
        throw std::invalid_argument("native activation must be f32[sequence_length, hidden_size]");
    }
    const std::size_t rows = static_cast<std::size_t>(p.tensor.shape[0]);
    if (rows > std::numeric_limits<std::size_t>::max() / static_cast<std::size_t>(hidden) / sizeof(float)) {
        throw std::invalid_argument("native activation shape exceeds addressable memory");
    }
    if (p.bytes.size() != rows * static_cast<std::size_t>(hidden) * sizeof(float)) {
        throw std::invalid_argument("native activation byte count does not match its shape");
    }
    std::vector<float> values(rows * static_cast<std::size_t>(hidden));
    std::memcpy(values.data(), p.bytes.data(), p.bytes.size());
    return values;
}

// native_stage_executor.cpp:47-70
Payload HipStageExecutor::activation_payload(const std::vector<float>& rows) const {
    Payload p;
    p.kind = PayloadKind::Activation;
    p.tensor.dtype = "f32";
    p.tensor.shape = {static_cast<std::int64_t>(rows.size() / params_.n_embd), static_cast<std::int64_t>(params_.n_embd)};
    p.tensor.byte_order = "little";
    p.tensor.layout = "row_major";
    p.bytes.resize(rows.size() * sizeof(float));
    std::memcpy(p.bytes.data(), rows.data(), p.bytes.size());
    return p;
}

// native_stage_executor.cpp:203-212
StageOutput HipStageExecutor::token_output(std::int32_t token) const {
    StageOutput out;
    out.payload = inference::sampled_token_payload(token);
    out.end_of_generation = config_.tokenizer->is_end_token(token);
    if (!out.end_of_generation) {
        out.token_text = config_.tokenizer->token_piece(token);
        out.completion_tokens = 1;
    }
    return out;
}

// llama_cpp_stage_adapter.cpp:350-386: one sampled id per verify row
StageOutput HipStageExecutor::rows_output(const std::vector<std::int32_t>& tokens) const {
    StageOutput out;
    out.verification_width = static_cast<int>(tokens.size());
    for (const std::int32_t t : tokens) {
        const bool eog = config_.tokenizer->is_end_token(t);
        out.token_eog.push_back(eog ? 1 : 0);
        if (!eog) {
            out.token_text += config_.tokenizer->token_piece(t);
            ++out.completion_tokens;
        }
        out.token_text_offsets.push_back(static_cast<std::uint32_t>(out.token_text.size()));
    }
    out.payload = inference::sampled_tokens_payload(tokens);
    return out;
}

// native_stage_executor.cpp:191-201
std::size_t HipStageExecutor::session_capacity(std::size_t prompt_tokens, int max_tokens) const {
    if (max_tokens <= 0) throw std::invalid_argument("native request needs a positive max_tokens");
    const std::size_t decode_inputs = static_cast<std::size_t>(max_tokens - 1);
    if (prompt_tokens > std::numeric_limits<std::size_t>::max() - decode_inputs) {
        throw std::invalid_argument("native session capacity overflow");
    }
    const std::size_t required = prompt_tokens + decode_inputs;
    if (required > static_cast<std::size_t>(config_.ctx_size)) {
        throw std::invalid_argument("native request exceeds configured context size");
    }
    return required;
}

}  // namespace jetsonfabric::runtime::adapters
