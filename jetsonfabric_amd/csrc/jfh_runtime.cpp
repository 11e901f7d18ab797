// Stage contract, HIP stage executor, prompt-lookup drafts and the
// speculative generation loop.
#include "jfh_runtime.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <limits>
#include <map>
#include <stdexcept>
#include <stop_token>
#include <thread>

namespace jfh::runtime {

// ------------------------------------------------------------------ inference
namespace inference {

ExecutionResult ExecutionResult::success(StageOutput output) {
    ExecutionResult r;
    r.ok = true;
    r.output = std::move(output);
    return r;
}

ExecutionResult ExecutionResult::invalid_input(std::string code, std::string message) {
    ExecutionResult r;
    r.error = ExecutionError{ErrorKind::InvalidInput, std::move(code), std::move(message)};
    return r;
}

ExecutionResult ExecutionResult::failure(std::string code, std::string message) {
    ExecutionResult r;
    r.error = ExecutionError{ErrorKind::ExecutionFailure, std::move(code), std::move(message)};
    return r;
}

void Executor::rollback_session(const std::string& session_id, int token_count) const {
    (void) session_id;
    (void) token_count;
    throw std::runtime_error("inference executor does not support KV-cache rollback");
}

namespace {

std::uint64_t dtype_width(const std::string& dtype) {
    if (dtype == "f32" || dtype == "i32" || dtype == "u32") return 4;
    if (dtype == "f16" || dtype == "bf16") return 2;
    return 0;
}

TensorDescriptor token_descriptor(std::size_t count) {
    return TensorDescriptor{"i32", {static_cast<std::int64_t>(count)}, "little", "row_major"};
}

void append_i32(std::vector<std::uint8_t>& out, std::int32_t v) {
    const auto b = static_cast<std::uint32_t>(v);
    for (int i = 0; i < 4; ++i) out.push_back(static_cast<std::uint8_t>(b >> (8 * i)));
}

}  // namespace

// runtime/inference/stage.cpp:95-160
std::string validate_stage_input(const StageInput& input) {
    if (input.session_id.empty()) return "session_id is required";
    if (input.request_id.empty()) return "request_id is required";
    if (input.model_id.empty()) return "model_id is required";
    if (input.position.count <= 0) return "stage count must be greater than zero";
    if (input.position.index < 0 || input.position.index >= input.position.count) {
        return "stage index must be within stage count";
    }
    if (input.layers.end <= input.layers.start) return "layer range end must be greater than start";
    if (input.phase == Phase::Prefill && input.decode_step != 0) return "prefill requires decode_step 0";
    if (input.phase == Phase::Decode && input.decode_step <= 0) return "decode requires a positive decode_step";
    if (input.max_tokens <= 0) return "max_tokens must be greater than zero";
    const Payload& p = input.payload;
    if (p.kind == PayloadKind::Text) {
        if (p.encoding != "utf-8") return "text payload encoding must be utf-8";
        if (!p.tensor.dtype.empty() || !p.tensor.shape.empty()) return "text payload must not declare tensor metadata";
        return "";
    }
    if (!p.encoding.empty()) return "tensor payload must not declare text encoding";
    if (p.tensor.dtype.empty() || p.tensor.shape.empty()) return "tensor payload requires dtype and shape";
    if (p.tensor.byte_order != "little" || p.tensor.layout != "row_major") {
        return "tensor payload requires little byte order and row_major layout";
    }
    const std::uint64_t width = dtype_width(p.tensor.dtype);
    if (width == 0) return "unsupported tensor dtype: " + p.tensor.dtype;
    std::uint64_t count = 1;
    for (const std::int64_t d : p.tensor.shape) {
        if (d <= 0 || count > (std::uint64_t(1) << 40) / static_cast<std::uint64_t>(d)) return "invalid or oversized tensor shape";
        count *= static_cast<std::uint64_t>(d);
    }
    if (count * width != p.bytes.size()) return "tensor shape and dtype do not match payload length";
    if (p.kind == PayloadKind::SampledToken && count != 1) return "sampled_token payload must contain exactly one element";
    if (p.kind == PayloadKind::SampledTokens && count < 2) return "sampled_tokens payload must contain at least two elements";
    return "";
}

// runtime/inference/token_payload.cpp:36-53
std::vector<std::int32_t> decode_token_ids(const Payload& payload) {
    if ((payload.tensor.dtype != "i32" && payload.tensor.dtype != "u32") || payload.tensor.shape.size() != 1 ||
        payload.tensor.shape[0] <= 0 || payload.tensor.byte_order != "little" ||
        payload.tensor.layout != "row_major" || payload.bytes.size() % 4 != 0 ||
        static_cast<std::uint64_t>(payload.tensor.shape[0]) != payload.bytes.size() / 4) {
        throw std::invalid_argument("token payload must be a little-endian i32 or u32 vector");
    }
    std::vector<std::int32_t> tokens(payload.bytes.size() / 4);
    for (std::size_t i = 0; i < tokens.size(); ++i) {
        const std::uint8_t* b = payload.bytes.data() + 4 * i;
        tokens[i] = static_cast<std::int32_t>(std::uint32_t(b[0]) | std::uint32_t(b[1]) << 8 |
                                              std::uint32_t(b[2]) << 16 | std::uint32_t(b[3]) << 24);
    }
    return tokens;
}

Payload tokens_payload(std::span<const std::int32_t> tokens) {
    Payload p;
    p.kind = PayloadKind::Tokens;
    p.tensor = token_descriptor(tokens.size());
    for (const std::int32_t t : tokens) append_i32(p.bytes, t);
    return p;
}

Payload sampled_token_payload(std::int32_t token) {
    Payload p;
    p.kind = PayloadKind::SampledToken;
    p.tensor = token_descriptor(1);
    append_i32(p.bytes, token);
    return p;
}

Payload sampled_tokens_payload(std::span<const std::int32_t> tokens) {
    if (tokens.size() < 2) throw std::invalid_argument("sampled_tokens payload requires at least two tokens");
    Payload p;
    p.kind = PayloadKind::SampledTokens;
    p.tensor = token_descriptor(tokens.size());
    for (const std::int32_t t : tokens) append_i32(p.bytes, t);
    return p;
}

}  // namespace inference

// ------------------------------------------------------------------ tokenization
namespace tokenization {

std::vector<std::int32_t> IdTokenizer::tokenize(std::string_view text) const {
    std::vector<std::int32_t> out;
    std::size_t i = 0;
    while (i < text.size()) {
        while (i < text.size() && (text[i] == ' ' || text[i] == '\n' || text[i] == '\t' || text[i] == ',')) ++i;
        if (i == text.size()) break;
        std::int64_t v = 0;
        std::size_t j = i;
        while (j < text.size() && text[j] >= '0' && text[j] <= '9' && v <= std::numeric_limits<std::int32_t>::max()) {
            v = v * 10 + (text[j] - '0');
            ++j;
        }
        if (j == i || v > std::numeric_limits<std::int32_t>::max()) {
            throw std::invalid_argument("text payload must contain decimal token ids");
        }
        out.push_back(static_cast<std::int32_t>(v));
        i = j;
    }
    return out;
}

std::string IdTokenizer::token_piece(std::int32_t token) const { return std::to_string(token) + " "; }

bool IdTokenizer::is_end_token(std::int32_t token) const {
    return std::find(end_tokens_.begin(), end_tokens_.end(), token) != end_tokens_.end();
}

}  // namespace tokenization

// ------------------------------------------------------------------ speculative
namespace speculative {

PromptLookupDraft::PromptLookupDraft(std::size_t max_ngram, std::size_t min_ngram)
    : max_ngram_(max_ngram), min_ngram_(min_ngram) {
    if (min_ngram == 0 || max_ngram < min_ngram) {
        throw std::invalid_argument("prompt lookup requires 0 < min_ngram <= max_ngram");
    }
}

// Longest suffix n-gram (max..min) that occurred earlier; the most recent
// earlier occurrence wins and the tokens after it are proposed
// (prompt_lookup_draft.cpp:15-44).
std::vector<std::uint32_t> PromptLookupDraft::propose(const std::vector<std::uint32_t>& history,
                                                      std::size_t max_tokens) const {
    if (max_tokens == 0 || history.size() <= min_ngram_) return {};
    const std::size_t n = history.size();
    for (std::size_t g = std::min(max_ngram_, n - 1); g >= min_ngram_; --g) {
        const std::size_t suffix = n - g;
        // candidate windows [c, c+g) entirely before the suffix, scanned right to left
        for (std::size_t c = suffix >= g ? suffix - g + 1 : 0; c-- > 0;) {
            if (!std::equal(history.begin() + static_cast<std::ptrdiff_t>(c),
                            history.begin() + static_cast<std::ptrdiff_t>(c + g),
                            history.begin() + static_cast<std::ptrdiff_t>(suffix))) {
                continue;
            }
            const std::size_t start = c + g;
            const std::size_t count = std::min(max_tokens, n - start);
            return std::vector<std::uint32_t>(history.begin() + static_cast<std::ptrdiff_t>(start),
                                              history.begin() + static_cast<std::ptrdiff_t>(start + count));
        }
        if (g == min_ngram_) break;
    }
    return {};
}

}  // namespace speculative

// ------------------------------------------------------------------ activation codecs
namespace activation {

std::uint16_t f32_to_f16(float value) {
    std::uint32_t x = 0;
    std::memcpy(&x, &value, sizeof(x));
    const std::uint16_t sign = static_cast<std::uint16_t>((x >> 16) & 0x8000U);
    const std::uint32_t ax = x & 0x7FFFFFFFU;
    if (ax > 0x7F800000U) return static_cast<std::uint16_t>(sign | 0x7E00U | ((ax >> 13) & 0x3FFU));  // NaN
    if (ax >= 0x477FF000U) return static_cast<std::uint16_t>(sign | 0x7C00U);  // rounds past 65504: infinity
    if (ax >= 0x38800000U) {
        // normal: rebias the exponent (127 -> 15), round the 13 dropped bits
        // to nearest even; a carry out of the mantissa bumps the exponent
        std::uint32_t m = ax - 0x38000000U;
        m += 0x0FFFU + ((m >> 13) & 1U);
        return static_cast<std::uint16_t>(sign | (m >> 13));
    }
    if (ax < 0x33000000U) return sign;  // below half the smallest subnormal (2^-25)
    // subnormal: value / 2^-24 rounded to nearest even (may reach 0x400, the smallest normal)
    const std::uint32_t e = ax >> 23, mant = (ax & 0x7FFFFFU) | 0x800000U;
    const std::uint32_t shift = 126U - e;  // 14 .. 24
    std::uint32_t q = mant >> shift;
    const std::uint32_t rest = mant & ((1U << shift) - 1U), half = 1U << (shift - 1U);
    if (rest > half || (rest == half && (q & 1U) != 0U)) ++q;
    return static_cast<std::uint16_t>(sign | q);
}

float f16_to_f32(std::uint16_t value) {
    const std::uint32_t sign = static_cast<std::uint32_t>(value & 0x8000U) << 16;
    const std::uint32_t e = (value >> 10) & 0x1FU, m = value & 0x3FFU;
    std::uint32_t bits = 0;
    if (e == 0x1FU) {
        bits = sign | 0x7F800000U | (m << 13);
    } else if (e != 0U) {
        bits = sign | ((e + 112U) << 23) | (m << 13);
    } else {
        const float sub = static_cast<float>(m) * 0x1p-24F;  // exact: m < 2^10
        std::memcpy(&bits, &sub, sizeof(bits));
        bits |= sign;
    }
    float out = 0.0F;
    std::memcpy(&out, &bits, sizeof(out));
    return out;
}

namespace {

constexpr const char* kF32 = "f32";
constexpr const char* kF16 = "f16";

void require_activation(const inference::Payload& p, const char* dtype) {
    if (p.kind != inference::PayloadKind::Activation) {
        throw std::invalid_argument("activation codec requires an activation payload");
    }
    if (p.tensor.dtype != dtype) {
        throw std::invalid_argument(std::string("activation codec expected ") + dtype + " input, got " + p.tensor.dtype);
    }
}

class F32Codec final : public ActivationCodec {
public:
    const std::string& name() const noexcept override {
        static const std::string n = kF32;
        return n;
    }
    inference::Payload encode(inference::Payload p) const override {
        require_activation(p, kF32);
        return p;
    }
    inference::Payload decode(inference::Payload p) const override {
        require_activation(p, kF32);
        return p;
    }
};

// little-endian f32 words <-> little-endian f16 words
class F16Codec final : public ActivationCodec {
public:
    const std::string& name() const noexcept override {
        static const std::string n = kF16;
        return n;
    }
    inference::Payload encode(inference::Payload p) const override {
        require_activation(p, kF32);
        if (p.bytes.size() % 4 != 0) throw std::invalid_argument("f32 activation byte length must be divisible by four");
        std::vector<std::uint8_t> out(p.bytes.size() / 2);
        for (std::size_t i = 0; i < out.size() / 2; ++i) {
            const std::uint8_t* b = p.bytes.data() + 4 * i;
            const std::uint32_t w = static_cast<std::uint32_t>(b[0]) | (static_cast<std::uint32_t>(b[1]) << 8) |
                                    (static_cast<std::uint32_t>(b[2]) << 16) | (static_cast<std::uint32_t>(b[3]) << 24);
            float f = 0.0F;
            std::memcpy(&f, &w, sizeof(f));
            const std::uint16_t h = f32_to_f16(f);
            out[2 * i] = static_cast<std::uint8_t>(h & 0xFFU);
            out[2 * i + 1] = static_cast<std::uint8_t>(h >> 8);
        }
        p.tensor.dtype = kF16;
        p.bytes = std::move(out);
        return p;
    }
    inference::Payload decode(inference::Payload p) const override {
        require_activation(p, kF16);
        if (p.bytes.size() % 2 != 0) throw std::invalid_argument("f16 activation byte length must be divisible by two");
        std::vector<std::uint8_t> out(p.bytes.size() * 2);
        for (std::size_t i = 0; i < p.bytes.size() / 2; ++i) {
            const std::uint16_t h =
                static_cast<std::uint16_t>(p.bytes[2 * i] | (static_cast<std::uint16_t>(p.bytes[2 * i + 1]) << 8));
            const float f = f16_to_f32(h);
            std::uint32_t w = 0;
            std::memcpy(&w, &f, sizeof(w));
            for (int k = 0; k < 4; ++k) out[4 * i + k] = static_cast<std::uint8_t>((w >> (8 * k)) & 0xFFU);
        }
        p.tensor.dtype = kF32;
        p.bytes = std::move(out);
        return p;
    }
};

}  // namespace

void ActivationCodecFactory::register_codec(std::string name, Builder builder) {
    if (name.empty()) throw std::invalid_argument("activation codec name must not be empty");
    if (!builder) throw std::invalid_argument("activation codec builder must not be empty");
    if (!builders_.emplace(std::move(name), std::move(builder)).second) {
        throw std::invalid_argument("activation codec is already registered");
    }
}

bool ActivationCodecFactory::supports(const std::string& name) const { return builders_.count(name) != 0; }

std::shared_ptr<const ActivationCodec> ActivationCodecFactory::create_codec(const std::string& name) const {
    auto it = builders_.find(name);
    if (it == builders_.end()) throw std::invalid_argument("unsupported activation encoding: " + name);
    std::shared_ptr<const ActivationCodec> codec = it->second();
    if (!codec) throw std::runtime_error("activation codec builder returned null: " + name);
    if (codec->name() != name) {
        throw std::runtime_error("activation codec registered as " + name + " returned strategy " + codec->name());
    }
    return codec;
}

std::shared_ptr<const ActivationCodecFactory> make_default_activation_codec_factory() {
    auto f = std::make_shared<ActivationCodecFactory>();
    f->register_codec(kF32, [] { return std::make_shared<F32Codec>(); });
    f->register_codec(kF16, [] { return std::make_shared<F16Codec>(); });
    return f;
}

}  // namespace activation

// ------------------------------------------------------------------ adapter
namespace adapters {

using inference::ExecutionResult;
using inference::Phase;
using inference::PayloadKind;
using inference::StageInput;
using inference::StageOutput;

class HipStageExecutor::Impl {
public:
    using Clock = std::chrono::steady_clock;

    struct SessionState {
        std::unique_ptr<Session> session;
        int expected_decode_step = 1;
        Clock::time_point last_used = Clock::now();
    };

    explicit Impl(HipStageConfig c) : config(std::move(c)) {
        if (!config.engine || !config.tokenizer) throw std::invalid_argument("native executor requires engine and tokenizer");
        if (config.ctx_size <= 0) throw std::invalid_argument("native executor context size must be positive");
        // native_stage_executor.cpp:84-104: a stage runs exactly the engine's resident layers
        const int layers = static_cast<int>(config.engine->params().n_layer);
        const inference::StagePosition& pos = config.position;
        if (pos.count <= 0 || pos.index < 0 || pos.index >= pos.count || config.layers.start < 0 ||
            config.layers.end <= config.layers.start || config.layers.end > layers ||
            (pos.is_first() && config.layers.start != 0) || (pos.is_last() && config.layers.end != layers)) {
            throw std::invalid_argument("native serving stage assignment is invalid");
        }
        if (config.layers.start != static_cast<int>(config.engine->layer_start()) ||
            config.layers.end != static_cast<int>(config.engine->layer_end())) {
            throw std::invalid_argument("native stage exceeds its resident layer range");
        }
        if (static_cast<std::uint32_t>(config.ctx_size) > config.engine->params().n_ctx) {
            throw std::invalid_argument("native context size exceeds model context");
        }
        if (config.speculative_max_tokens < 0 || config.speculative_max_tokens > 8) {
            throw std::invalid_argument("speculative width must be 0..8");
        }
        if (config.session_idle_ttl <= std::chrono::milliseconds::zero() ||
            config.session_reap_interval <= std::chrono::milliseconds::zero()) {
            throw std::invalid_argument("native session expiration intervals must be greater than zero");
        }
        reaper = std::jthread([this](std::stop_token stop) { reap_sessions(stop); });
    }

    // llama_cpp_stage_adapter.cpp:939-967: sessions idle for the TTL are closed
    void prune_expired_locked(Clock::time_point now) {
        for (auto it = sessions.begin(); it != sessions.end();) {
            it = now - it->second.last_used >= config.session_idle_ttl ? sessions.erase(it) : std::next(it);
        }
    }

    void reap_sessions(std::stop_token stop) {
        std::mutex wait_mutex;
        std::condition_variable_any wake;
        while (!stop.stop_requested()) {
            {
                std::unique_lock wait_lock(wait_mutex);
                wake.wait_for(wait_lock, stop, config.session_reap_interval, [] { return false; });
            }
            if (stop.stop_requested()) return;
            std::lock_guard lock(mutex);
            prune_expired_locked(Clock::now());
        }
    }

    // native_stage_executor.cpp:110-140
    ExecutionResult execute(const StageInput& input) {
        std::lock_guard lock(mutex);
        prune_expired_locked(Clock::now());
        return execute_locked(input);
    }

    ExecutionResult execute_locked(const StageInput& input) {
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
        } catch (const Error& e) {
            if (e.code() == Status::InvalidArgument) return ExecutionResult::invalid_input("invalid_native_stage_input", e.what());
            return ExecutionResult::failure("native_stage_execution_failed", e.what());
        } catch (const std::exception& e) {
            return ExecutionResult::failure("native_stage_execution_failed", e.what());
        }
    }

    // Decode inputs of distinct existing sessions run as one multi-sequence
    // engine step; everything else falls back to execute (executor.hpp:20-28).
    std::vector<ExecutionResult> execute_batch(const std::vector<StageInput>& inputs) {
        std::lock_guard lock(mutex);
        prune_expired_locked(Clock::now());
        std::vector<ExecutionResult> results(inputs.size());
        std::vector<std::size_t> batch;
        std::vector<std::vector<std::int32_t>> batch_tokens;
        for (std::size_t i = 0; i < inputs.size(); ++i) {
            const StageInput& in = inputs[i];
            bool batchable = whole_model() && in.phase == Phase::Decode && inference::validate_stage_input(in).empty() &&
                             assignment_matches(in) && batch.size() < static_cast<std::size_t>(gpu::kMaxSeq);
            std::vector<std::int32_t> tokens;
            if (batchable) {
                auto it = sessions.find(in.session_id);
                batchable = it != sessions.end() && in.decode_step == it->second.expected_decode_step;
                for (std::size_t j : batch) batchable = batchable && inputs[j].session_id != in.session_id;
                if (batchable) {
                    try {
                        tokens = input_tokens(in);
                    } catch (const std::exception&) {
                        batchable = false;
                    }
                    batchable = batchable && !tokens.empty() &&
                                tokens.size() <= static_cast<std::size_t>(config.speculative_max_tokens + 1);
                }
            }
            if (batchable) {
                batch.push_back(i);
                batch_tokens.push_back(std::move(tokens));
            } else {
                results[i] = execute_locked(in);
            }
        }
        if (batch.empty()) return results;
        try {
            std::vector<SeqStep> steps;
            std::size_t outs = 0;
            for (std::size_t k = 0; k < batch.size(); ++k) {
                SeqStep st;
                st.session = sessions.at(inputs[batch[k]].session_id).session.get();
                st.tokens = batch_tokens[k].data();
                st.n = static_cast<std::uint32_t>(batch_tokens[k].size());
                st.logits = st.n > 1 ? 2 : 1;
                outs += st.n;
                steps.push_back(st);
            }
            std::vector<std::int32_t> ids(outs);
            config.engine->forward(steps, ids.data(), nullptr, nullptr);
            std::size_t o = 0;
            for (std::size_t k = 0; k < batch.size(); ++k) {
                const std::size_t n = batch_tokens[k].size();
                SessionState& state = sessions.at(inputs[batch[k]].session_id);
                state.expected_decode_step += static_cast<int>(n);
                state.last_used = Clock::now();
                std::vector<std::int32_t> mine(ids.begin() + static_cast<std::ptrdiff_t>(o),
                                               ids.begin() + static_cast<std::ptrdiff_t>(o + n));
                StageOutput out = n > 1 ? rows_output(mine) : token_output(mine[0]);
                out.execution_batch_size = static_cast<int>(batch.size());
                results[batch[k]] = ExecutionResult::success(std::move(out));
                o += n;
            }
        } catch (const std::exception& e) {
            for (std::size_t k : batch) results[k] = ExecutionResult::failure("native_stage_execution_failed", e.what());
        }
        return results;
    }

    void close_session(const std::string& id) {
        std::lock_guard lock(mutex);
        sessions.erase(id);
    }

    // native_stage_executor.cpp:147-162
    void rollback_session(const std::string& id, int n) {
        std::lock_guard lock(mutex);
        if (n <= 0) throw std::invalid_argument("rollback token count must be positive");
        auto it = sessions.find(id);
        if (it == sessions.end()) throw std::invalid_argument("native stage session not found");
        SessionState& state = it->second;
        if (n >= state.expected_decode_step) throw std::invalid_argument("rollback exceeds the decoded native suffix");
        state.session->rollback(static_cast<std::uint32_t>(n));
        state.expected_decode_step -= n;
        state.last_used = Clock::now();
    }

    std::size_t count() {
        std::lock_guard lock(mutex);
        prune_expired_locked(Clock::now());
        return sessions.size();
    }

private:
    bool assignment_matches(const StageInput& in) const {
        return in.position.index == config.position.index && in.position.count == config.position.count &&
               in.layers.start == config.layers.start && in.layers.end == config.layers.end;
    }

    std::vector<std::int32_t> input_tokens(const StageInput& in) const {
        if (in.payload.kind == PayloadKind::Text) {
            return config.tokenizer->tokenize(std::string_view(reinterpret_cast<const char*>(in.payload.bytes.data()),
                                                               in.payload.bytes.size()));
        }
        if (in.payload.kind == PayloadKind::Tokens || in.payload.kind == PayloadKind::SampledToken) {
            return inference::decode_token_ids(in.payload);
        }
        throw std::invalid_argument("native first stage requires text or token input");
    }

    std::size_t session_capacity(std::size_t prompt_tokens, int max_tokens) const {
        const std::size_t required = prompt_tokens + static_cast<std::size_t>(max_tokens - 1);
        if (required > static_cast<std::size_t>(config.ctx_size)) {
            throw std::invalid_argument("native request exceeds configured context size");
        }
        return required;
    }

    // native_stage_executor.cpp:203-212
    StageOutput token_output(std::int32_t token) const {
        StageOutput out;
        out.payload = inference::sampled_token_payload(token);
        out.end_of_generation = config.tokenizer->is_end_token(token);
        if (!out.end_of_generation) {
            out.token_text = config.tokenizer->token_piece(token);
            out.completion_tokens = 1;
        }
        return out;
    }

    // llama_cpp_stage_adapter.cpp:350-386
    StageOutput rows_output(const std::vector<std::int32_t>& tokens) const {
        StageOutput out;
        out.verification_width = static_cast<int>(tokens.size());
        for (const std::int32_t t : tokens) {
            const bool eog = config.tokenizer->is_end_token(t);
            out.token_eog.push_back(eog ? 1 : 0);
            if (!eog) {
                out.token_text += config.tokenizer->token_piece(t);
                ++out.completion_tokens;
            }
            out.token_text_offsets.push_back(static_cast<std::uint32_t>(out.token_text.size()));
        }
        out.payload = inference::sampled_tokens_payload(tokens);
        return out;
    }

    bool whole_model() const { return config.position.is_first() && config.position.is_last(); }

    // native_stage_executor.cpp:16-47: f32 [rows, n_embd] activation payloads
    std::vector<float> input_activation(const StageInput& in) const {
        const std::int64_t H = config.engine->params().n_embd;
        const inference::Payload& p = in.payload;
        if (p.kind != PayloadKind::Activation || p.tensor.dtype != "f32" || p.tensor.shape.size() != 2 ||
            p.tensor.shape[0] <= 0 || p.tensor.shape[1] != H) {
            throw std::invalid_argument("native activation must be f32[sequence_length, hidden_size]");
        }
        const std::size_t rows = static_cast<std::size_t>(p.tensor.shape[0]);
        if (rows > std::numeric_limits<std::size_t>::max() / static_cast<std::size_t>(H) / sizeof(float)) {
            throw std::invalid_argument("native activation shape exceeds addressable memory");
        }
        if (p.bytes.size() != rows * static_cast<std::size_t>(H) * sizeof(float)) {
            throw std::invalid_argument("native activation byte count does not match its shape");
        }
        std::vector<float> rows_f32(rows * static_cast<std::size_t>(H));
        std::memcpy(rows_f32.data(), p.bytes.data(), p.bytes.size());
        return rows_f32;
    }

    StageOutput activation_output(const std::vector<float>& rows) const {
        const std::int64_t H = config.engine->params().n_embd;
        StageOutput out;
        out.payload.kind = PayloadKind::Activation;
        out.payload.tensor.dtype = "f32";
        out.payload.tensor.shape = {static_cast<std::int64_t>(rows.size()) / H, H};
        out.payload.tensor.byte_order = "little";
        out.payload.tensor.layout = "row_major";
        out.payload.bytes.resize(rows.size() * sizeof(float));
        std::memcpy(out.payload.bytes.data(), rows.data(), out.payload.bytes.size());
        out.execution_batch_size = 1;
        return out;
    }

    // A stage of a pipeline (not the whole model): prefill_stage_* / decode_stage_*
    // (native_stage_executor.cpp:226-320)
    ExecutionResult stage_prefill(const StageInput& in) {
        std::vector<std::int32_t> tokens;
        std::vector<float> act;
        std::size_t count = 0;
        if (config.position.is_first()) {
            tokens = input_tokens(in);
            count = tokens.size();
        } else {
            act = input_activation(in);
            count = act.size() / config.engine->params().n_embd;
        }
        const std::size_t capacity = session_capacity(count, in.max_tokens);
        std::unique_ptr<Session> session = config.engine->create_session(static_cast<std::uint32_t>(capacity));
        std::vector<float> out_rows(config.position.is_last() ? 0 : count * config.engine->params().n_embd);
        const std::int32_t token = config.engine->stage_prefill(
            *session, tokens.empty() ? nullptr : tokens.data(), act.empty() ? nullptr : act.data(),
            static_cast<std::uint32_t>(count), out_rows.empty() ? nullptr : out_rows.data());
        StageOutput out = config.position.is_last() ? token_output(token) : activation_output(out_rows);
        if (config.position.is_first()) {
            out.prompt_tokens = static_cast<int>(tokens.size());
            for (const std::int32_t t : tokens) {
                if (t < 0) throw std::invalid_argument("native tokenizer returned a negative token");
                out.prompt_token_ids.push_back(static_cast<std::uint32_t>(t));
            }
        }
        sessions.emplace(in.session_id, SessionState{std::move(session), 1});
        return ExecutionResult::success(std::move(out));
    }

    ExecutionResult stage_decode(const StageInput& in, SessionState& state) {
        std::vector<std::int32_t> tokens;
        std::vector<float> act;
        if (config.position.is_first()) {
            tokens = input_tokens(in);
            if (tokens.size() != 1U) {
                return ExecutionResult::invalid_input("native_multi_token_verification_unsupported",
                                                      "native serving currently accepts one decode token per pass");
            }
        } else {
            act = input_activation(in);
            if (act.size() != config.engine->params().n_embd) {
                return ExecutionResult::invalid_input("native_multi_token_verification_unsupported",
                                                      "native decode activation must contain one token row");
            }
        }
        std::vector<float> out_rows(config.position.is_last() ? 0 : config.engine->params().n_embd);
        const std::int32_t token =
            config.engine->stage_decode(*state.session, tokens.empty() ? nullptr : tokens.data(),
                                        act.empty() ? nullptr : act.data(), out_rows.empty() ? nullptr : out_rows.data());
        ++state.expected_decode_step;
        state.last_used = Clock::now();
        return ExecutionResult::success(config.position.is_last() ? token_output(token) : activation_output(out_rows));
    }

    ExecutionResult prefill(const StageInput& in) {
        if (sessions.count(in.session_id)) {
            return ExecutionResult::invalid_input("duplicate_stage_session", "prefill session already exists on this native stage");
        }
        if (!whole_model()) return stage_prefill(in);
        const std::vector<std::int32_t> tokens = input_tokens(in);
        if (tokens.empty()) throw std::invalid_argument("native Qwen2 prefill is outside session capacity");
        const std::size_t capacity = session_capacity(tokens.size(), in.max_tokens);
        std::unique_ptr<Session> session = config.engine->create_session(static_cast<std::uint32_t>(capacity));
        const std::int32_t token =
            config.engine->prefill(*session, tokens.data(), static_cast<std::uint32_t>(tokens.size()), nullptr);
        StageOutput out = token_output(token);
        out.prompt_tokens = static_cast<int>(tokens.size());
        for (const std::int32_t t : tokens) {
            if (t < 0) throw std::invalid_argument("native tokenizer returned a negative token");
            out.prompt_token_ids.push_back(static_cast<std::uint32_t>(t));
        }
        sessions.emplace(in.session_id, SessionState{std::move(session), 1});
        return ExecutionResult::success(std::move(out));
    }

    ExecutionResult decode(const StageInput& in) {
        auto it = sessions.find(in.session_id);
        if (it == sessions.end()) {
            return ExecutionResult::invalid_input("stage_session_not_found", "decode requires an existing native prefill session");
        }
        SessionState& state = it->second;
        if (in.decode_step != state.expected_decode_step) {
            return ExecutionResult::invalid_input("unexpected_decode_step", "native decode step does not match session state");
        }
        if (!whole_model()) return stage_decode(in, state);
        const std::vector<std::int32_t> tokens = input_tokens(in);
        if (tokens.empty() || tokens.size() > static_cast<std::size_t>(config.speculative_max_tokens + 1)) {
            return ExecutionResult::invalid_input("invalid_verification_width",
                                                  "native decode accepts 1..speculative_max_tokens+1 tokens per pass");
        }
        if (state.session->position() == 0) throw std::invalid_argument("native Qwen2 decode is outside session capacity");
        SeqStep st;
        st.session = state.session.get();
        st.tokens = tokens.data();
        st.n = static_cast<std::uint32_t>(tokens.size());
        st.logits = tokens.size() > 1 ? 2 : 1;
        std::vector<std::int32_t> ids(tokens.size());
        config.engine->forward({st}, ids.data(), nullptr, nullptr);
        state.expected_decode_step += static_cast<int>(tokens.size());
        state.last_used = Clock::now();
        return ExecutionResult::success(tokens.size() > 1 ? rows_output(ids) : token_output(ids[0]));
    }

    HipStageConfig config;
    mutable std::mutex mutex;
    std::unordered_map<std::string, SessionState> sessions;
    std::jthread reaper;  // last: stopped and joined before the sessions go
};

HipStageExecutor::HipStageExecutor(HipStageConfig config) : impl_(std::make_unique<Impl>(std::move(config))) {}
HipStageExecutor::~HipStageExecutor() = default;

inference::ExecutionResult HipStageExecutor::execute(const inference::StageInput& input) const {
    return impl_->execute(input);
}

std::vector<inference::ExecutionResult> HipStageExecutor::execute_batch(
    const std::vector<inference::StageInput>& inputs) const {
    return impl_->execute_batch(inputs);
}

void HipStageExecutor::close_session(const std::string& session_id) const { impl_->close_session(session_id); }

void HipStageExecutor::rollback_session(const std::string& session_id, int token_count) const {
    impl_->rollback_session(session_id, token_count);
}

std::size_t HipStageExecutor::session_count() const { return impl_->count(); }

}  // namespace adapters

// ------------------------------------------------------------------ generation loop
namespace {

struct SampledBatch {
    std::vector<std::uint32_t> tokens;
    std::vector<bool> eog;
};

// generation_runner.cpp:45-84
SampledBatch read_sampled(const inference::StageOutput& out) {
    SampledBatch b;
    const std::vector<std::int32_t> ids = inference::decode_token_ids(out.payload);
    for (const std::int32_t t : ids) {
        if (t < 0) throw std::invalid_argument("sampled token is negative");
        b.tokens.push_back(static_cast<std::uint32_t>(t));
    }
    if (out.payload.kind == inference::PayloadKind::SampledTokens) {
        if (out.token_eog.size() != ids.size()) throw std::invalid_argument("sampled token flags do not match tokens");
        for (const std::uint8_t e : out.token_eog) b.eog.push_back(e != 0);
    } else {
        b.eog.push_back(out.end_of_generation);
    }
    return b;
}

}  // namespace

GenerationResult run_generation(const inference::Executor& executor, const GenerationRequest& request,
                                const speculative::DraftStrategy* draft_strategy, int speculative_max_tokens) {
    using clock = std::chrono::steady_clock;
    GenerationResult result;
    const auto fail = [&](std::string code, std::string message) {
        executor.close_session(request.session_id);
        result.ok = false;
        result.error_code = std::move(code);
        result.error_message = std::move(message);
        return result;
    };
    auto stage_input = [&](inference::Phase phase, int step, std::span<const std::int32_t> tokens) {
        inference::StageInput in;
        in.session_id = request.session_id;
        in.request_id = request.request_id;
        in.model_id = request.model_id;
        in.phase = phase;
        in.decode_step = step;
        in.position = {0, 1};
        in.layers = {0, request.layer_count};
        in.payload = inference::tokens_payload(tokens);
        in.max_tokens = request.max_tokens;
        return in;
    };

    std::vector<std::uint32_t> history;
    std::uint32_t previous = 0;
    bool eog = false;
    bool recover = false;
    int decode_step = 1;
    const auto t0 = clock::now();
    inference::ExecutionResult pre = executor.execute(stage_input(inference::Phase::Prefill, 0, request.prompt));
    if (!pre.ok) return fail(pre.error.code, pre.error.message);
    SampledBatch first;
    try {
        first = read_sampled(pre.output);
    } catch (const std::exception& e) {
        return fail("invalid_sampled_token", e.what());
    }
    if (first.tokens.size() != 1) return fail("invalid_sampled_token", "prefill returned multiple tokens");
    result.time_to_first_token_ms = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
    history = pre.output.prompt_token_ids;
    eog = first.eog[0];
    auto emit = [&](std::uint32_t token) {
        result.sampled_tokens.push_back(token);
        history.push_back(token);
        ++result.completion_tokens;
        previous = token;
    };
    if (!eog) emit(first.tokens[0]);
    if (request.after_prefill) request.after_prefill();

    const auto t1 = clock::now();
    while (result.completion_tokens < request.max_tokens && !eog) {
        const int remaining = request.max_tokens - result.completion_tokens;
        std::vector<std::uint32_t> draft;
        if (draft_strategy && remaining > 1 && !recover) {
            draft = draft_strategy->propose(history, static_cast<std::size_t>(std::min(speculative_max_tokens, remaining - 1)));
        }
        recover = false;
        std::vector<std::int32_t> verify;
        verify.push_back(static_cast<std::int32_t>(previous));
        for (const std::uint32_t t : draft) verify.push_back(static_cast<std::int32_t>(t));
        inference::ExecutionResult pass = executor.execute(stage_input(inference::Phase::Decode, decode_step, verify));
        ++result.target_decode_passes;
        if (!pass.ok) return fail(pass.error.code, pass.error.message);
        SampledBatch target;
        try {
            target = read_sampled(pass.output);
        } catch (const std::exception& e) {
            return fail("invalid_sampled_token", e.what());
        }
        if (target.tokens.size() != verify.size()) {
            return fail("invalid_speculative_verification", "target output count does not match speculative verification input");
        }
        std::size_t accepted = 0;
        while (accepted < draft.size() && !target.eog[accepted] && target.tokens[accepted] == draft[accepted]) ++accepted;
        result.speculative_draft_tokens += static_cast<int>(draft.size());
        result.speculative_accepted_tokens += static_cast<int>(accepted);
        const int rollback = accepted < draft.size() ? static_cast<int>(draft.size() - accepted) : 0;
        if (rollback > 0) {
            try {
                executor.rollback_session(request.session_id, rollback);
            } catch (const std::exception& e) {
                return fail("generation_rollback_failed", e.what());
            }
            recover = true;
        }
        decode_step += static_cast<int>(verify.size()) - rollback;
        const std::size_t outputs = accepted < draft.size() ? accepted + 1 : target.tokens.size();
        for (std::size_t i = 0; i < outputs && result.completion_tokens < request.max_tokens; ++i) {
            if (target.eog[i]) {
                eog = true;
                break;
            }
            emit(target.tokens[i]);
        }
    }
    result.decode_end = clock::now();
    result.decode_ms = std::chrono::duration<double, std::milli>(result.decode_end - t1).count();
    executor.close_session(request.session_id);
    result.ok = true;
    result.finish_reason = eog ? "stop" : "length";
    return result;
}

// ------------------------------------------------------------------ continuous batching
namespace pipeline_parallel {

// Decode steps are combined by the threads that submit them; there is no
// worker thread. A submitted step waits in `arrived` (a pointer to a ticket
// on its caller's stack). The first caller that finds no batch forming leads
// the next one: it waits until max_batch_size steps have arrived or max_wait
// has passed, takes up to max_batch_size of them in arrival order (its own
// step need not be among them when more had queued), runs them as one
// delegate execute_batch without holding the queue lock, writes each ticket's
// result and wakes everyone. A caller whose ticket is still open afterwards
// leads or joins the next batch. Steps arriving while a batch runs queue for
// the next one, so the GPU goes from one batched step to the next.
// Both waits (an open ticket for its batch, a leader for its batch to fill)
// first spin for up to kSpin on atomic copies of the state kept under the
// lock, then block on the condition variable: a batched step is answered
// within microseconds instead of a thread wake-up later, which the next step
// of every sequence in the batch would wait for.
struct ContinuousBatchingExecutor::Impl {
    static constexpr auto kSpin = std::chrono::microseconds(2000);
    struct Ticket {
        const inference::StageInput* input = nullptr;
        inference::ExecutionResult result;
        std::atomic<bool> answered{false};
    };

    // spins until done() or kSpin (or the deadline) has passed; the caller
    // re-checks its condition under the lock before blocking
    template <typename Done>
    static void spin(Done done, std::chrono::steady_clock::time_point deadline) {
        deadline = std::min(deadline, std::chrono::steady_clock::now() + kSpin);
        while (!done() && std::chrono::steady_clock::now() < deadline) std::this_thread::yield();
    }

    std::unique_ptr<inference::Executor> delegate;
    ContinuousBatchingConfig config;
    // delegate calls are serialized: batches, prefills, rollbacks and closes
    std::mutex delegate_turn;
    std::mutex state;
    std::condition_variable changed;
    std::vector<Ticket*> arrived;  // steps no leader has taken yet, oldest first
    bool forming = false;          // a leader is gathering or running a batch
    // copies of arrived.size() and forming, written under the lock, read while spinning
    std::atomic<std::size_t> n_arrived{0};
    std::atomic<bool> forming_now{false};

    Impl(std::unique_ptr<inference::Executor> d, ContinuousBatchingConfig c) : delegate(std::move(d)), config(c) {
        if (!delegate) throw std::invalid_argument("a continuous-batching executor needs a delegate executor");
        if (config.max_batch_size < 2) {
            throw std::invalid_argument("a continuous-batching executor needs max_batch_size >= 2");
        }
        if (config.max_wait < std::chrono::microseconds::zero()) {
            throw std::invalid_argument("a continuous-batching executor needs a non-negative max_wait");
        }
    }

    // Runs the taken steps on the delegate; failures, whatever the delegate
    // throws, become per-step results with the reference's error codes.
    std::vector<inference::ExecutionResult> run_batch(const std::vector<Ticket*>& taken) {
        std::vector<inference::ExecutionResult> out;
        try {
            std::vector<inference::StageInput> inputs;
            inputs.reserve(taken.size());
            for (const Ticket* t : taken) inputs.push_back(*t->input);
            std::lock_guard turn(delegate_turn);
            out = delegate->execute_batch(inputs);
        } catch (const std::exception& e) {
            return std::vector<inference::ExecutionResult>(
                taken.size(), inference::ExecutionResult::failure("continuous_batch_failed", e.what()));
        } catch (...) {
            return std::vector<inference::ExecutionResult>(
                taken.size(), inference::ExecutionResult::failure("continuous_batch_failed",
                                                                   "the delegate threw a non-standard exception"));
        }
        if (out.size() != taken.size()) {
            const std::string why = "the delegate answered " + std::to_string(out.size()) + " of " +
                                    std::to_string(taken.size()) + " batched steps";
            return std::vector<inference::ExecutionResult>(
                taken.size(), inference::ExecutionResult::failure("continuous_batch_result_mismatch", why));
        }
        return out;
    }

    inference::ExecutionResult step(const inference::StageInput& input) {
        Ticket mine;
        mine.input = &input;
        std::unique_lock lock(state);
        arrived.push_back(&mine);
        n_arrived.store(arrived.size(), std::memory_order_release);
        changed.notify_all();  // a gathering leader may now hold a full batch
        while (!mine.answered.load(std::memory_order_acquire)) {
            if (forming) {
                lock.unlock();
                spin([&] { return mine.answered.load(std::memory_order_acquire) ||
                              !forming_now.load(std::memory_order_acquire); },
                     std::chrono::steady_clock::time_point::max());
                lock.lock();
                if (!mine.answered.load(std::memory_order_acquire) && forming) changed.wait(lock);
                continue;
            }
            forming = true;
            forming_now.store(true, std::memory_order_release);
            std::vector<Ticket*> taken;
            try {
                const auto deadline = std::chrono::steady_clock::now() + config.max_wait;
                if (arrived.size() < config.max_batch_size) {
                    lock.unlock();
                    spin([&] { return n_arrived.load(std::memory_order_acquire) >= config.max_batch_size; }, deadline);
                    lock.lock();
                }
                changed.wait_until(lock, deadline, [this] { return arrived.size() >= config.max_batch_size; });
                const std::size_t n = std::min(arrived.size(), config.max_batch_size);
                taken.assign(arrived.begin(), arrived.begin() + static_cast<std::ptrdiff_t>(n));
                arrived.erase(arrived.begin(), arrived.begin() + static_cast<std::ptrdiff_t>(n));
                n_arrived.store(arrived.size(), std::memory_order_release);
                lock.unlock();
                std::vector<inference::ExecutionResult> results = run_batch(taken);
                lock.lock();
                for (std::size_t i = 0; i < n; ++i) {
                    taken[i]->result = std::move(results[i]);
                    taken[i]->answered.store(true, std::memory_order_release);
                }
            } catch (...) {
                // Whatever escaped, no ticket is left waiting for this leader: the
                // steps it took and its own step (still queued or not) are answered
                // with the batch failure, and the next caller leads.
                if (!lock.owns_lock()) lock.lock();
                const auto failed = [] {
                    return inference::ExecutionResult::failure("continuous_batch_failed", "the batch leader failed");
                };
                for (Ticket* t : taken) {
                    if (!t->answered.load(std::memory_order_acquire)) {
                        t->result = failed();
                        t->answered.store(true, std::memory_order_release);
                    }
                }
                const auto it = std::find(arrived.begin(), arrived.end(), &mine);
                if (it != arrived.end()) {
                    arrived.erase(it);
                    n_arrived.store(arrived.size(), std::memory_order_release);
                    mine.result = failed();
                    mine.answered.store(true, std::memory_order_release);
                }
            }
            forming = false;
            forming_now.store(false, std::memory_order_release);
            changed.notify_all();
        }
        return std::move(mine.result);
    }
};

ContinuousBatchingExecutor::ContinuousBatchingExecutor(std::unique_ptr<inference::Executor> delegate,
                                                       ContinuousBatchingConfig config)
    : impl_(std::make_unique<Impl>(std::move(delegate), config)) {}

ContinuousBatchingExecutor::~ContinuousBatchingExecutor() = default;

inference::ExecutionResult ContinuousBatchingExecutor::execute(const inference::StageInput& input) const {
    if (input.phase == inference::Phase::Prefill) {
        // a prompt is not held back to wait for decode steps
        std::lock_guard turn(impl_->delegate_turn);
        return impl_->delegate->execute(input);
    }
    return impl_->step(input);
}

std::vector<inference::ExecutionResult> ContinuousBatchingExecutor::execute_batch(
    const std::vector<inference::StageInput>& inputs) const {
    std::lock_guard turn(impl_->delegate_turn);
    return impl_->delegate->execute_batch(inputs);
}

void ContinuousBatchingExecutor::close_session(const std::string& session_id) const {
    std::lock_guard turn(impl_->delegate_turn);
    impl_->delegate->close_session(session_id);
}

void ContinuousBatchingExecutor::rollback_session(const std::string& session_id, int token_count) const {
    std::lock_guard turn(impl_->delegate_turn);
    impl_->delegate->rollback_session(session_id, token_count);
}

}  // namespace pipeline_parallel

}  // namespace jfh::runtime
