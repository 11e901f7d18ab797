// C ABI of the HIP Qwen2 stage engine (declarations and reference mapping in include/jfh.h).
#include "jfh.h"

#include "jfh_engine.hpp"
#include "jfh_runtime.hpp"
#include "jfh_tokenizer.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>

struct jfh_model {
    std::unique_ptr<jfh::HostModel> model;
    std::vector<std::string> names;  // stable NUL-terminated copies for views
    bool finalized = false;
};

struct jfh_engine {
    std::shared_ptr<jfh::Engine> engine;
};

struct jfh_package {
    std::unique_ptr<jfh::Package> package;
};

struct jfh_session {
    jfh_engine* owner;
    std::unique_ptr<jfh::Session> session;
};

namespace {

jfh_status ok() {
    jfh_status s{};
    s.code = JFH_STATUS_OK;
    return s;
}

jfh_status error(int32_t code, const char* message) {
    jfh_status s{};
    s.code = code;
    std::snprintf(s.message, sizeof(s.message), "%s", message);
    return s;
}

template <typename F>
jfh_status guarded(F&& fn) {
    try {
        fn();
        return ok();
    } catch (const jfh::Error& e) {
        return error(static_cast<int32_t>(e.code()), e.what());
    } catch (const std::invalid_argument& e) {
        return error(JFH_STATUS_INVALID_ARGUMENT, e.what());
    } catch (const std::bad_alloc&) {
        return error(JFH_STATUS_OUT_OF_MEMORY, "host allocation failed");
    } catch (const std::exception& e) {
        return error(JFH_STATUS_DEVICE_ERROR, e.what());
    }
}

void require(bool condition, const char* message) {
    if (!condition) throw jfh::Error(jfh::Status::InvalidArgument, message);
}

void require(bool condition, const std::string& message) { require(condition, message.c_str()); }

void fill_view(const jfh_model* m, size_t index, jfh_tensor_view* out) {
    const jfh::TensorView& t = m->model->tensors()[index];
    out->name = m->names[index].c_str();
    out->type = t.type;
    out->rank = t.rank;
    for (int d = 0; d < 4; ++d) out->shape[d] = t.shape[d];
    out->layer = t.layer;
    out->data = t.data;
    out->size = t.size;
}

void refresh_names(jfh_model* m) {
    m->names.clear();
    for (const jfh::TensorView& t : m->model->tensors()) m->names.push_back(t.name);
    m->finalized = true;
}

jfh::ModelParams to_params(const jfh_model_params& p) {
    jfh::ModelParams q;
    q.n_layer = p.n_layer;
    q.n_embd = p.n_embd;
    q.n_ff = p.n_ff;
    q.n_head = p.n_head;
    q.n_head_kv = p.n_head_kv;
    q.n_ctx = p.n_ctx;
    q.n_vocab = p.n_vocab;
    q.head_dim = p.n_head ? p.n_embd / p.n_head : 0;
    q.rope_base = p.rope_base;
    q.rms_eps = p.rms_eps;
    return q;
}

// A DraftStrategy whose proposals come from a caller's C function
// (jfh_generate_draft); at most max_tokens of them are used.
class CallbackDraft final : public jfh::runtime::speculative::DraftStrategy {
public:
    CallbackDraft(jfh_draft_propose_fn fn, void* user) : fn_(fn), user_(user) {}
    std::vector<std::uint32_t> propose(const std::vector<std::uint32_t>& history,
                                       std::size_t max_tokens) const override {
        std::vector<std::uint32_t> out(max_tokens);
        const uint32_t n = max_tokens ? fn_(user_, history.data(), history.size(), static_cast<uint32_t>(max_tokens),
                                            out.data())
                                      : 0;
        out.resize(std::min<std::size_t>(n, max_tokens));
        return out;
    }

private:
    jfh_draft_propose_fn fn_;
    void* user_;
};

// Generation statistics of one request: the runner's counters and times, the
// rates of GenerationResult and the prefill / buffer metrics of the engine.
void fill_stats(const jfh::Engine& engine, const jfh::runtime::GenerationResult& r, const jfh::PrefillMetrics& pm,
                uint32_t capacity, uint32_t prompt_tokens, jfh_generation_stats& st) {
    st = jfh_generation_stats{};
    st.completion_tokens = static_cast<uint32_t>(r.completion_tokens);
    st.target_decode_passes = static_cast<uint32_t>(r.target_decode_passes);
    st.speculative_draft_tokens = static_cast<uint32_t>(r.speculative_draft_tokens);
    st.speculative_accepted_tokens = static_cast<uint32_t>(r.speculative_accepted_tokens);
    st.time_to_first_token_ms = r.time_to_first_token_ms;
    st.decode_ms = r.decode_ms;
    st.stopped = r.finish_reason == "stop" ? 1U : 0U;
    // the first token comes from the prefill; the decode passes produce the rest
    const double decoded = r.sampled_tokens.empty() ? 0.0 : static_cast<double>(r.sampled_tokens.size() - 1);
    st.inter_token_latency_ms = decoded > 0.0 ? r.decode_ms / decoded : 0.0;
    st.decode_tokens_per_second = decoded > 0.0 && r.decode_ms > 0.0 ? decoded / (r.decode_ms * 1e-3) : 0.0;
    const double total_ms = r.time_to_first_token_ms + r.decode_ms;
    st.end_to_end_tokens_per_second = total_ms > 0.0 ? static_cast<double>(r.sampled_tokens.size()) / (total_ms * 1e-3) : 0.0;
    st.prefill_plan_reused = pm.plan_reused ? 1U : 0U;
    st.prefill_attention_matrix_cores = pm.attention_matrix_cores ? 1U : 0U;
    st.prefill_planning_ms = pm.planning_ms;
    st.prefill_allocation_ms = pm.allocation_ms;
    st.prefill_host_input_ms = pm.host_input_ms;
    st.prefill_compute_ms = pm.compute_ms;
    st.prefill_output_read_ms = pm.output_read_ms;
    const jfh::BufferMetrics bm = engine.buffer_metrics(capacity, prompt_tokens, pm);
    st.kv_cache_bytes = bm.kv_cache_bytes;
    st.prefill_scratch_bytes = bm.prefill_scratch_bytes;
    st.decode_scratch_bytes = bm.decode_scratch_bytes;
    st.prefill_host_input_bytes = bm.prefill_host_input_bytes;
}

// One GenerationRunner loop over a HIP stage executor owning every layer.
void generate_one(jfh_engine* engine, const int32_t* prompt, uint32_t n_prompt, uint32_t max_tokens,
                  uint32_t draft_max, const jfh::runtime::speculative::DraftStrategy* draft, int32_t* out_tokens,
                  uint32_t* out_count, jfh_generation_stats* stats) {
    require(engine && prompt && n_prompt > 0 && max_tokens > 0 && out_tokens && out_count, "generation arguments are required");
    require(draft_max <= 8, "draft length must be 0..8");
    namespace rt = jfh::runtime;
    const jfh::ModelParams& p = engine->engine->params();
    rt::adapters::HipStageConfig cfg;
    cfg.engine = engine->engine;
    cfg.tokenizer = std::make_shared<rt::tokenization::IdTokenizer>(engine->engine->end_tokens());
    cfg.ctx_size = static_cast<int>(std::min<uint64_t>(p.n_ctx, static_cast<uint64_t>(n_prompt) + max_tokens));
    cfg.position = {0, 1};
    cfg.layers = {0, static_cast<int>(p.n_layer)};
    cfg.speculative_max_tokens = static_cast<int>(draft_max);
    rt::adapters::HipStageExecutor executor(cfg);
    rt::GenerationRequest req;
    req.prompt.assign(prompt, prompt + n_prompt);
    req.max_tokens = static_cast<int>(max_tokens);
    req.layer_count = static_cast<int>(p.n_layer);
    const rt::GenerationResult r =
        rt::run_generation(executor, req, draft_max > 0 ? draft : nullptr, static_cast<int>(draft_max));
    if (!r.ok) throw jfh::Error(jfh::Status::InvalidArgument, r.error_code + ": " + r.error_message);
    for (size_t i = 0; i < r.sampled_tokens.size(); ++i) out_tokens[i] = static_cast<int32_t>(r.sampled_tokens[i]);
    *out_count = static_cast<uint32_t>(r.sampled_tokens.size());
    if (stats) {
        fill_stats(*engine->engine, r, jfh::Engine::last_prefill_metrics(), static_cast<uint32_t>(cfg.ctx_size),
                   n_prompt, *stats);
    }
}

}  // namespace

extern "C" {

jfh_status jfh_tensor_type_layout(uint32_t type, uint32_t* block_elements, uint32_t* block_bytes) {
    if (!block_elements || !block_bytes) return error(JFH_STATUS_INVALID_ARGUMENT, "tensor layout outputs are required");
    if (!jfh::type_layout(type, block_elements, block_bytes)) {
        return error(JFH_STATUS_FORMAT_ERROR, "unsupported JFM tensor type");
    }
    return ok();
}

jfh_status jfh_sha256(const void* data, size_t size, uint8_t digest[32]) {
    if ((!data && size) || !digest) return error(JFH_STATUS_INVALID_ARGUMENT, "data and digest are required");
    const auto d = jfh::sha256(data, size);
    std::memcpy(digest, d.data(), 32);
    return ok();
}

jfh_status jfh_package_open(const char* package_path, uint32_t layer_start, uint32_t layer_end, uint32_t verify_hashes,
                            jfh_package** out) {
    return guarded([&] {
        require(package_path && package_path[0] && out, "package path and output are required");
        *out = nullptr;
        jfh::StagePlan plan;
        plan.layer_start = layer_start;
        plan.layer_end = layer_end;
        plan.verify_hashes = verify_hashes != 0;
        auto p = std::make_unique<jfh_package>();
        p->package = jfh::Package::open(package_path, plan);
        *out = p.release();
    });
}

void jfh_package_close(jfh_package* package) { delete package; }

jfh_status jfh_package_get_stats(const jfh_package* package, jfh_package_stats* out) {
    return guarded([&] {
        require(package && out, "package and output are required");
        const jfh::PackageStats& s = package->package->stats();
        *out = jfh_package_stats{s.layer_start, s.layer_end, s.layer_count, 0, s.selected_weight_bytes,
                                 s.total_weight_bytes, s.mapped_bytes, s.selected_tensor_count, s.total_tensor_count};
    });
}

size_t jfh_package_tensor_count(const jfh_package* package) {
    return package ? package->package->tensors().size() : 0;
}

namespace {
void package_view(const jfh::TensorView& t, jfh_tensor_view* out) {
    out->name = t.name.c_str();
    out->type = t.type;
    out->rank = t.rank;
    for (int d = 0; d < 4; ++d) out->shape[d] = t.shape[d];
    out->layer = t.layer;
    out->data = t.data;
    out->size = t.size;
}
}  // namespace

jfh_status jfh_package_tensor_at(const jfh_package* package, size_t index, jfh_tensor_view* out) {
    return guarded([&] {
        require(package && out, "package and output are required");
        const auto& tensors = package->package->tensors();
        if (index >= tensors.size()) throw jfh::Error(jfh::Status::NotFound, "tensor index is out of range");
        package_view(tensors[index], out);
    });
}

jfh_status jfh_package_find_tensor(const jfh_package* package, const char* name, jfh_tensor_view* out) {
    return guarded([&] {
        require(package && name && out, "package, name and output are required");
        const jfh::TensorView* t = package->package->find(name);
        if (!t) throw jfh::Error(jfh::Status::NotFound, std::string("tensor not found: ") + name);
        package_view(*t, out);
    });
}

jfh_status jfh_package_gguf_metadata(const jfh_package* package, const void** data, size_t* size) {
    return guarded([&] {
        require(package && data && size, "package and outputs are required");
        *data = package->package->gguf_metadata();
        *size = package->package->gguf_metadata_size();
        if (!*data) throw jfh::Error(jfh::Status::NotFound, "package has no GGUF metadata");
    });
}

jfh_status jfh_package_source_sha256(const jfh_package* package, uint8_t digest[32]) {
    return guarded([&] {
        require(package && digest, "package and output are required");
        std::memcpy(digest, package->package->source_sha256().data(), 32);
    });
}

jfh_status jfh_model_open_gguf(const char* gguf_path, jfh_model** out) {
    return guarded([&] {
        require(gguf_path && out, "GGUF path and output are required");
        *out = nullptr;
        auto m = std::make_unique<jfh_model>();
        m->model = jfh::HostModel::open_gguf(gguf_path);
        refresh_names(m.get());
        *out = m.release();
    });
}

jfh_status jfh_model_open(const char* package_path, uint32_t layer_start, uint32_t layer_end, uint32_t verify_hashes,
                          jfh_model** out) {
    return guarded([&] {
        require(package_path && out, "package path and output are required");
        *out = nullptr;
        jfh::StagePlan plan;
        plan.layer_start = layer_start;
        plan.layer_end = layer_end;
        plan.verify_hashes = verify_hashes != 0;
        auto m = std::make_unique<jfh_model>();
        m->model = jfh::HostModel::open_package(package_path, plan);
        refresh_names(m.get());
        *out = m.release();
    });
}

jfh_status jfh_model_synthesize(const jfh_synth_spec* spec, jfh_model** out) {
    return guarded([&] {
        require(spec && out, "spec and output are required");
        *out = nullptr;
        jfh::SynthSpec s;
        s.params = to_params(spec->params);
        s.type_linear = spec->type_linear;
        s.type_embd = spec->type_embd;
        s.type_output = spec->type_output;
        s.tied_output = spec->tied_output != 0;
        s.output_bias = spec->output_bias != 0;
        s.seed = spec->seed;
        s.stddev = spec->stddev;
        s.threads = spec->threads;
        auto m = std::make_unique<jfh_model>();
        m->model = jfh::HostModel::synthesize(s);
        refresh_names(m.get());
        *out = m.release();
    });
}

jfh_status jfh_model_create(const jfh_model_params* params, jfh_model** out) {
    return guarded([&] {
        require(params && out, "params and output are required");
        require(params->n_head > 0 && params->n_embd % params->n_head == 0, "heads must divide the embedding");
        *out = nullptr;
        auto m = std::make_unique<jfh_model>();
        m->model = jfh::HostModel::build(to_params(*params));
        *out = m.release();
    });
}

jfh_status jfh_model_add_tensor(jfh_model* model, const char* name, uint32_t type, uint32_t rank,
                                const uint64_t* shape, const void* data, uint64_t size) {
    return guarded([&] {
        require(model && name && shape && (data || size == 0), "model, name, shape and data are required");
        require(!model->finalized, "model is already finalized");
        model->model->add_tensor(name, type, rank, shape, data, size);
    });
}

jfh_status jfh_model_finalize(jfh_model* model) {
    return guarded([&] {
        require(model, "model is required");
        require(!model->finalized, "model is already finalized");
        model->model->finalize();
        refresh_names(model);
    });
}

jfh_status jfh_model_write_package(const jfh_model* model, const char* directory) {
    return guarded([&] {
        require(model && directory && model->finalized, "a finalized model and a directory are required");
        model->model->write_package(directory);
    });
}

jfh_status jfh_model_slice(const jfh_model* model, uint32_t layer_start, uint32_t layer_end, jfh_model** out) {
    return guarded([&] {
        require(model && out && model->finalized, "a finalized model and an output are required");
        *out = nullptr;
        auto m = std::make_unique<jfh_model>();
        m->model = model->model->slice(layer_start, layer_end);
        refresh_names(m.get());
        *out = m.release();
    });
}

void jfh_model_close(jfh_model* model) { delete model; }

jfh_status jfh_model_get_params(const jfh_model* model, jfh_model_params* out) {
    return guarded([&] {
        require(model && out, "model and output are required");
        const jfh::ModelParams& p = model->model->params();
        out->n_layer = p.n_layer;
        out->n_embd = p.n_embd;
        out->n_ff = p.n_ff;
        out->n_head = p.n_head;
        out->n_head_kv = p.n_head_kv;
        out->n_ctx = p.n_ctx;
        out->n_vocab = p.n_vocab;
        out->head_dim = p.head_dim;
        out->rope_base = p.rope_base;
        out->rms_eps = p.rms_eps;
    });
}

jfh_status jfh_model_get_stats(const jfh_model* model, jfh_model_stats* out) {
    return guarded([&] {
        require(model && out && model->finalized, "a finalized model and an output are required");
        const jfh::HostModel& m = *model->model;
        out->layer_start = m.layer_start();
        out->layer_end = m.layer_end();
        out->layer_count = m.params().n_layer;
        out->selected_weight_bytes = m.weight_bytes();
        out->total_weight_bytes = m.total_weight_bytes();
        out->selected_tensor_count = m.tensors().size();
        out->total_tensor_count = m.total_tensor_count();
    });
}

size_t jfh_model_tensor_count(const jfh_model* model) { return model ? model->names.size() : 0; }

jfh_status jfh_model_tensor_at(const jfh_model* model, size_t index, jfh_tensor_view* out) {
    return guarded([&] {
        require(model && out && model->finalized, "a finalized model and an output are required");
        if (index >= model->names.size()) throw jfh::Error(jfh::Status::NotFound, "tensor index is out of range");
        fill_view(model, index, out);
    });
}

jfh_status jfh_model_find_tensor(const jfh_model* model, const char* name, jfh_tensor_view* out) {
    return guarded([&] {
        require(model && name && out && model->finalized, "a finalized model, a name and an output are required");
        for (size_t i = 0; i < model->names.size(); ++i) {
            if (model->names[i] == name) {
                fill_view(model, i, out);
                return;
            }
        }
        throw jfh::Error(jfh::Status::NotFound, std::string("tensor not found: ") + name);
    });
}

jfh_status jfh_model_source_sha256(const jfh_model* model, char hex[65]) {
    return guarded([&] {
        require(model && hex && model->finalized, "a finalized model and an output are required");
        const std::string h = model->model->source_sha256();
        std::snprintf(hex, 65, "%s", h.c_str());
    });
}

jfh_status jfh_engine_create(const jfh_model* model, const jfh_engine_options* options, jfh_engine** out) {
    return guarded([&] {
        require(model && out && model->finalized, "a finalized model and an output are required");
        *out = nullptr;
        jfh::EngineOptions o;
        if (options) {
            o.device = options->device;
            o.use_graphs = options->use_graphs != 0;
        }
        auto e = std::make_unique<jfh_engine>();
        e->engine = std::make_shared<jfh::Engine>(*model->model, o);
        *out = e.release();
    });
}

void jfh_engine_destroy(jfh_engine* engine) { delete engine; }

jfh_status jfh_engine_get_info(const jfh_engine* engine, jfh_engine_info* out) {
    return guarded([&] {
        require(engine && out, "engine and output are required");
        out->weight_bytes = engine->engine->weight_bytes();
        out->prefill_chunk = engine->engine->max_prefill_chunk();
        std::snprintf(out->device_name, sizeof(out->device_name), "%s", engine->engine->device_name().c_str());
        out->layer_start = engine->engine->layer_start();
        out->layer_end = engine->engine->layer_end();
    });
}

jfh_status jfh_engine_get_params(const jfh_engine* engine, jfh_model_params* out) {
    return guarded([&] {
        require(engine && out, "engine and output are required");
        const jfh::ModelParams& p = engine->engine->params();
        *out = jfh_model_params{p.n_layer, p.n_embd, p.n_ff, p.n_head, p.n_head_kv,
                                p.n_ctx,   p.n_vocab, p.head_dim, p.rope_base, p.rms_eps};
    });
}

jfh_status jfh_engine_set_end_tokens(jfh_engine* engine, const int32_t* ids, uint32_t n) {
    return guarded([&] {
        require(engine, "engine is required");
        engine->engine->set_end_tokens(ids, n);
    });
}

jfh_status jfh_session_create(jfh_engine* engine, uint32_t capacity, jfh_session** out) {
    return guarded([&] {
        require(engine && out, "engine and output are required");
        *out = nullptr;
        auto s = std::make_unique<jfh_session>();
        s->owner = engine;
        s->session = engine->engine->create_session(capacity);
        *out = s.release();
    });
}

void jfh_session_destroy(jfh_session* session) { delete session; }

uint32_t jfh_session_capacity(const jfh_session* session) { return session ? session->session->capacity() : 0; }

uint32_t jfh_session_position(const jfh_session* session) { return session ? session->session->position() : 0; }

jfh_status jfh_session_prefill(jfh_session* session, const int32_t* tokens, uint32_t n, int32_t* out_token,
                               float* logits) {
    return guarded([&] {
        require(session && tokens && out_token, "session, tokens and output are required");
        *out_token = session->owner->engine->prefill(*session->session, tokens, n, logits);
    });
}

jfh_status jfh_session_decode(jfh_session* session, int32_t token, int32_t* out_token, float* logits) {
    return guarded([&] {
        require(session && out_token, "session and output are required");
        jfh::Session& s = *session->session;
        // qwen2_architecture.cpp:1050-1054
        if (s.position() == 0 || s.position() >= s.capacity()) {
            throw jfh::Error(jfh::Status::InvalidArgument, "native Qwen2 decode is outside session capacity");
        }
        jfh::SeqStep st;
        st.session = &s;
        st.tokens = &token;
        st.n = 1;
        st.logits = 1;
        session->owner->engine->forward({st}, out_token, nullptr, logits);
    });
}

jfh_status jfh_session_verify(jfh_session* session, const int32_t* tokens, uint32_t n, int32_t* out_tokens,
                              uint32_t* out_accepted, float* logits) {
    return guarded([&] {
        require(session && tokens && out_tokens && n > 0, "session, tokens and outputs are required");
        jfh::Session& s = *session->session;
        if (s.position() == 0) throw jfh::Error(jfh::Status::InvalidArgument, "verification requires a prefilled session");
        jfh::SeqStep st;
        st.session = &s;
        st.tokens = tokens;
        st.n = n;
        st.logits = 2;
        int32_t accepted = 0;
        session->owner->engine->forward({st}, out_tokens, &accepted, logits);
        if (out_accepted) *out_accepted = static_cast<uint32_t>(accepted);
    });
}

jfh_status jfh_session_stage_prefill(jfh_session* session, const int32_t* tokens, const float* activations,
                                     uint32_t n, int32_t* out_token, float* out_activations, float* logits) {
    return guarded([&] {
        require(session, "session is required");
        jfh::Engine& e = *session->owner->engine;
        require(!e.last_stage() || out_token, "the final stage writes a token");
        require(e.last_stage() || !logits, "only the final stage computes logits");
        const int32_t token = e.stage_prefill(*session->session, tokens, activations, n, out_activations, logits);
        if (out_token) *out_token = token;
    });
}

jfh_status jfh_session_stage_decode(jfh_session* session, const int32_t* token, const float* activation,
                                    int32_t* out_token, float* out_activation, float* logits) {
    return guarded([&] {
        require(session, "session is required");
        jfh::Engine& e = *session->owner->engine;
        require(!e.last_stage() || out_token, "the final stage writes a token");
        require(e.last_stage() || !logits, "only the final stage computes logits");
        const int32_t t = e.stage_decode(*session->session, token, activation, out_activation, logits);
        if (out_token) *out_token = t;
    });
}

namespace {

jfh::runtime::inference::Payload activation_payload(const std::string& dtype, const void* data, size_t size) {
    jfh::runtime::inference::Payload p;
    p.kind = jfh::runtime::inference::PayloadKind::Activation;
    p.tensor.dtype = dtype;
    p.tensor.byte_order = "little";
    p.tensor.layout = "row_major";
    const auto* b = static_cast<const uint8_t*>(data);
    p.bytes.assign(b, b + size);
    return p;
}

}  // namespace

jfh_status jfh_activation_encode(const char* codec, const float* values, size_t n, void* out, size_t out_size) {
    return guarded([&] {
        require(codec && (values || n == 0) && (out || out_size == 0), "codec, values and output are required");
        auto c = jfh::runtime::activation::make_default_activation_codec_factory()->create_codec(codec);
        const auto wire = c->encode(activation_payload("f32", values, n * sizeof(float)));
        require(wire.bytes.size() == out_size, "activation output size does not match the encoding");
        if (out_size) std::memcpy(out, wire.bytes.data(), out_size);
    });
}

jfh_status jfh_activation_decode(const char* codec, const void* data, size_t size, float* values, size_t n) {
    return guarded([&] {
        require(codec && (data || size == 0) && (values || n == 0), "codec, data and output are required");
        auto c = jfh::runtime::activation::make_default_activation_codec_factory()->create_codec(codec);
        const auto f32 = c->decode(activation_payload(codec, data, size));
        require(f32.bytes.size() == n * sizeof(float), "activation output size does not match the encoding");
        if (n) std::memcpy(values, f32.bytes.data(), n * sizeof(float));
    });
}

jfh_status jfh_session_rollback(jfh_session* session, uint32_t n) {
    return guarded([&] {
        require(session, "session is required");
        session->session->rollback(n);
    });
}

jfh_status jfh_engine_step_batch(jfh_engine* engine, jfh_session* const* sessions, uint32_t count,
                                 const int32_t* tokens, const uint32_t* lengths, int32_t* out_tokens,
                                 uint32_t* out_accepted, float* logits) {
    return guarded([&] {
        require(engine && sessions && tokens && lengths && out_tokens && count > 0, "batch arguments are required");
        std::vector<jfh::SeqStep> steps;
        size_t offset = 0;
        for (uint32_t i = 0; i < count; ++i) {
            require(sessions[i] && sessions[i]->owner == engine, "session does not belong to this engine");
            require(sessions[i]->session->position() > 0, "batched steps require prefilled sessions");
            jfh::SeqStep st;
            st.session = sessions[i]->session.get();
            st.tokens = tokens + offset;
            st.n = lengths[i];
            st.logits = lengths[i] > 1 ? 2 : 1;
            offset += lengths[i];
            steps.push_back(st);
        }
        std::vector<int32_t> accepted(count);
        engine->engine->forward(steps, out_tokens, accepted.data(), logits);
        if (out_accepted) {
            for (uint32_t i = 0; i < count; ++i) out_accepted[i] = static_cast<uint32_t>(accepted[i]);
        }
    });
}

jfh_status jfh_engine_stage_step_batch(jfh_engine* engine, jfh_session* const* sessions, uint32_t count,
                                       const int32_t* tokens, const float* activations, const uint32_t* lengths,
                                       int32_t* out_tokens, float* out_activations, float* logits) {
    return guarded([&] {
        require(engine && sessions && lengths && count > 0, "batch arguments are required");
        jfh::Engine& e = *engine->engine;
        require(e.first_stage() ? tokens != nullptr && activations == nullptr : tokens == nullptr && activations != nullptr,
                "the first stage takes token ids, later stages activation rows");
        require(e.last_stage() ? out_tokens != nullptr : out_activations != nullptr && logits == nullptr,
                "the last stage writes token ids (and logits), the others activation rows");
        const size_t H = e.params().n_embd;
        std::vector<jfh::SeqStep> steps;
        size_t offset = 0;
        for (uint32_t i = 0; i < count; ++i) {
            require(sessions[i] && sessions[i]->owner == engine, "session does not belong to this engine");
            require(sessions[i]->session->position() > 0, "batched steps require prefilled sessions");
            require(lengths[i] > 0, "every session brings at least one row");
            jfh::SeqStep st;
            st.session = sessions[i]->session.get();
            st.tokens = tokens ? tokens + offset : nullptr;
            st.activations = activations ? activations + offset * H : nullptr;
            st.n = lengths[i];
            st.logits = e.last_stage() ? 2 : 0;
            offset += lengths[i];
            steps.push_back(st);
        }
        e.forward(steps, out_tokens, nullptr, logits, e.last_stage() ? nullptr : out_activations);
    });
}

jfh_status jfh_engine_dequantize(jfh_engine* engine, const char* tensor, uint32_t row0, uint32_t n_rows, float* out) {
    return guarded([&] {
        require(engine && tensor && out, "engine, tensor and output are required");
        engine->engine->dequantize(tensor, row0, n_rows, out);
    });
}

jfh_status jfh_engine_matmul(jfh_engine* engine, const char* tensor, const float* x, uint32_t n_tok, float* y) {
    return guarded([&] {
        require(engine && tensor && x && y, "engine, tensor and buffers are required");
        engine->engine->matmul(tensor, x, n_tok, y);
    });
}

jfh_status jfh_engine_matmul_noalloc(jfh_engine* engine, const char* tensor, const float* x, uint32_t n_tok,
                                     float* y, void* stream) {
    return guarded([&] {
        require(engine && tensor && x && y, "engine, tensor and device buffers are required");
        engine->engine->matmul_noalloc(tensor, x, n_tok, y, static_cast<hipStream_t>(stream));
    });
}

jfh_status jfh_session_read_kv(const jfh_session* session, uint32_t layer, uint32_t n, uint16_t* k, uint16_t* v) {
    return guarded([&] {
        require(session && k && v, "cache read arguments are required");
        session->owner->engine->read_kv(*session->session, layer, n, k, v);
    });
}

jfh_status jfh_session_import_kv(jfh_session* session, uint32_t n, const uint16_t* k, const uint16_t* v) {
    return guarded([&] {
        require(session && k && v, "cache import arguments are required");
        session->owner->engine->import_kv(*session->session, n, k, v);
    });
}

jfh_status jfh_session_time_steps(jfh_session* session, const int32_t* tokens, uint32_t n, uint32_t all_logits,
                                  uint32_t warmup, uint32_t iterations, double* ms_per_step) {
    return guarded([&] {
        require(session && tokens && ms_per_step && n > 0 && iterations > 0, "timing arguments are required");
        jfh::Engine& e = *session->owner->engine;
        jfh::Session& s = *session->session;
        require(s.position() > 0, "timing requires a prefilled session");
        jfh::SeqStep st;
        st.session = &s;
        st.tokens = tokens;
        st.n = n;
        st.logits = all_logits ? 2 : 1;
        std::vector<int32_t> ids(n);
        for (uint32_t i = 0; i < warmup; ++i) {
            e.forward({st}, ids.data(), nullptr, nullptr);
            s.rollback(n);
        }
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
            throw jfh::Error(jfh::Status::DeviceError, "create timing events");
        }
        (void) hipEventRecord(a, e.stream());
        for (uint32_t i = 0; i < iterations; ++i) {
            e.forward({st}, ids.data(), nullptr, nullptr);
            s.rollback(n);
        }
        (void) hipEventRecord(b, e.stream());
        (void) hipEventSynchronize(b);
        float ms = 0.0F;
        (void) hipEventElapsedTime(&ms, a, b);
        (void) hipEventDestroy(a);
        (void) hipEventDestroy(b);
        *ms_per_step = static_cast<double>(ms) / iterations;
    });
}

jfh_status jfh_session_profile_step(jfh_session* session, const int32_t* tokens, uint32_t n, uint32_t all_logits,
                                    uint32_t iterations, jfh_kernel_stat* out, uint32_t capacity, uint32_t* count) {
    return guarded([&] {
        require(session && tokens && out && count && n > 0 && iterations > 0, "profile arguments are required");
        require(session->session->position() > 0, "profiling requires a prefilled session");
        jfh::SeqStep st;
        st.session = session->session.get();
        st.tokens = tokens;
        st.n = n;
        st.logits = all_logits ? 2 : 1;
        const std::vector<jfh::KernelStat> stats = session->owner->engine->profile({st}, iterations);
        const uint32_t k = std::min<uint32_t>(capacity, static_cast<uint32_t>(stats.size()));
        for (uint32_t i = 0; i < k; ++i) {
            std::snprintf(out[i].label, sizeof(out[i].label), "%s", stats[i].label.c_str());
            out[i].launches = stats[i].launches;
            out[i].total_ms = stats[i].total_ms;
            out[i].bytes = stats[i].bytes;
        }
        *count = k;
    });
}

jfh_status jfh_engine_profile_batch(jfh_engine* engine, jfh_session* const* sessions, uint32_t count,
                                    const int32_t* tokens, const uint32_t* lengths, uint32_t all_logits,
                                    uint32_t iterations, jfh_kernel_stat* out, uint32_t capacity, uint32_t* out_count) {
    return guarded([&] {
        require(engine && sessions && tokens && lengths && out && out_count && count > 0 && iterations > 0,
                "profile arguments are required");
        std::vector<jfh::SeqStep> steps(count);
        uint32_t offset = 0;
        for (uint32_t i = 0; i < count; ++i) {
            require(sessions[i] && sessions[i]->owner == engine, "every session must belong to the engine");
            require(lengths[i] > 0, "every session needs rows");
            require(sessions[i]->session->position() > 0, "profiling requires prefilled sessions");
            steps[i].session = sessions[i]->session.get();
            steps[i].tokens = tokens + offset;
            steps[i].n = lengths[i];
            steps[i].logits = all_logits ? 2 : 1;
            offset += lengths[i];
        }
        const std::vector<jfh::KernelStat> stats = engine->engine->profile(steps, iterations);
        const uint32_t k = std::min<uint32_t>(capacity, static_cast<uint32_t>(stats.size()));
        for (uint32_t i = 0; i < k; ++i) {
            std::snprintf(out[i].label, sizeof(out[i].label), "%s", stats[i].label.c_str());
            out[i].launches = stats[i].launches;
            out[i].total_ms = stats[i].total_ms;
            out[i].bytes = stats[i].bytes;
        }
        *out_count = k;
    });
}

struct jfh_tokenizer {
    std::shared_ptr<const jfh::runtime::tokenization::BpeTokenizer> tokenizer;
};

jfh_status jfh_tokenizer_open(const char* path, jfh_tokenizer** out) {
    return guarded([&] {
        require(path && out, "tokenizer path and output are required");
        *out = nullptr;
        auto t = std::make_unique<jfh_tokenizer>();
        t->tokenizer = jfh::runtime::tokenization::BpeTokenizer::open(path);
        *out = t.release();
    });
}

void jfh_tokenizer_destroy(jfh_tokenizer* tokenizer) { delete tokenizer; }

jfh_status jfh_tokenizer_tokenize(const jfh_tokenizer* tokenizer, const char* text, size_t length, int32_t* ids,
                                  uint32_t capacity, uint32_t* out_count) {
    return guarded([&] {
        require(tokenizer && (text || length == 0) && out_count && (ids || capacity == 0), "tokenizer arguments are required");
        const std::vector<int32_t> v = tokenizer->tokenizer->tokenize(std::string_view(text ? text : "", length));
        *out_count = static_cast<uint32_t>(v.size());
        require(v.size() <= capacity, "id buffer holds fewer than the " + std::to_string(v.size()) + " ids");
        std::copy(v.begin(), v.end(), ids);
    });
}

jfh_status jfh_tokenizer_token_piece(const jfh_tokenizer* tokenizer, int32_t token, char* buf, uint32_t capacity,
                                     uint32_t* out_length) {
    return guarded([&] {
        require(tokenizer && out_length && (buf || capacity == 0), "tokenizer arguments are required");
        const std::string piece = tokenizer->tokenizer->token_piece(token);
        *out_length = static_cast<uint32_t>(piece.size());
        require(piece.size() <= capacity, "piece buffer holds fewer than the " + std::to_string(piece.size()) + " bytes");
        std::copy(piece.begin(), piece.end(), buf);
    });
}

jfh_status jfh_tokenizer_is_end_token(const jfh_tokenizer* tokenizer, int32_t token, uint32_t* out) {
    return guarded([&] {
        require(tokenizer && out, "tokenizer arguments are required");
        *out = tokenizer->tokenizer->is_end_token(token) ? 1 : 0;
    });
}

jfh_status jfh_tokenizer_end_tokens(const jfh_tokenizer* tokenizer, int32_t* ids, uint32_t capacity,
                                    uint32_t* out_count) {
    return guarded([&] {
        require(tokenizer && out_count && (ids || capacity == 0), "tokenizer arguments are required");
        const std::vector<int32_t> v = tokenizer->tokenizer->end_tokens();
        *out_count = static_cast<uint32_t>(v.size());
        require(v.size() <= capacity, "id buffer holds fewer than the " + std::to_string(v.size()) + " ids");
        std::copy(v.begin(), v.end(), ids);
    });
}

jfh_status jfh_tokenizer_vocab_size(const jfh_tokenizer* tokenizer, uint32_t* out) {
    return guarded([&] {
        require(tokenizer && out, "tokenizer arguments are required");
        *out = static_cast<uint32_t>(tokenizer->tokenizer->vocab_size());
    });
}

jfh_status jfh_prompt_lookup_propose(const uint32_t* history, size_t n, uint32_t max_ngram, uint32_t min_ngram,
                                     uint32_t max_tokens, uint32_t* out, uint32_t* out_count) {
    return guarded([&] {
        require((history || n == 0) && out_count && (out || max_tokens == 0), "history and outputs are required");
        jfh::runtime::speculative::PromptLookupDraft draft(max_ngram, min_ngram);
        const std::vector<uint32_t> h(history, history + n);
        const std::vector<uint32_t> p = draft.propose(h, max_tokens);
        std::copy(p.begin(), p.end(), out);
        *out_count = static_cast<uint32_t>(p.size());
    });
}

jfh_status jfh_generate(jfh_engine* engine, const int32_t* prompt, uint32_t n_prompt, uint32_t max_tokens,
                        uint32_t draft_max, uint32_t max_ngram, uint32_t min_ngram, int32_t* out_tokens,
                        uint32_t* out_count, jfh_generation_stats* stats) {
    return guarded([&] {
        std::unique_ptr<jfh::runtime::speculative::PromptLookupDraft> draft;
        if (draft_max > 0) draft = std::make_unique<jfh::runtime::speculative::PromptLookupDraft>(max_ngram, min_ngram);
        generate_one(engine, prompt, n_prompt, max_tokens, draft_max, draft.get(), out_tokens, out_count, stats);
    });
}

jfh_status jfh_generate_draft(jfh_engine* engine, const int32_t* prompt, uint32_t n_prompt, uint32_t max_tokens,
                              uint32_t draft_max, jfh_draft_propose_fn propose, void* user, int32_t* out_tokens,
                              uint32_t* out_count, jfh_generation_stats* stats) {
    return guarded([&] {
        require(propose != nullptr || draft_max == 0, "a draft strategy is required");
        const CallbackDraft draft(propose, user);
        generate_one(engine, prompt, n_prompt, max_tokens, draft_max, propose ? &draft : nullptr, out_tokens,
                     out_count, stats);
    });
}

jfh_status jfh_generate_concurrent(jfh_engine* engine, uint32_t n_requests, const int32_t* prompts,
                                   const uint32_t* prompt_lengths, uint32_t max_tokens, uint32_t draft_max,
                                   uint32_t max_ngram, uint32_t min_ngram, uint32_t batch_wait_us,
                                   int32_t* out_tokens, uint32_t* out_counts, jfh_generation_stats* stats,
                                   double* decode_wall_ms) {
    return guarded([&] {
        require(engine && prompts && prompt_lengths && out_tokens && out_counts && max_tokens > 0,
                "generation arguments are required");
        require(n_requests >= 1 && n_requests <= 8, "requests must be 1..8");
        require(draft_max <= 8, "draft length must be 0..8");
        require(n_requests * (draft_max + 1) <= static_cast<uint32_t>(jfh::gpu::kMaxRows),
                "the requests' verify rows must fit one step");
        namespace rt = jfh::runtime;
        const jfh::ModelParams& p = engine->engine->params();
        std::vector<std::vector<int32_t>> req_prompts(n_requests);
        uint64_t longest = 0;
        for (uint32_t i = 0, o = 0; i < n_requests; o += prompt_lengths[i], ++i) {
            require(prompt_lengths[i] > 0, "every request needs a prompt");
            req_prompts[i].assign(prompts + o, prompts + o + prompt_lengths[i]);
            longest = std::max<uint64_t>(longest, prompt_lengths[i]);
        }
        rt::adapters::HipStageConfig cfg;
        cfg.engine = engine->engine;
        cfg.tokenizer = std::make_shared<rt::tokenization::IdTokenizer>(engine->engine->end_tokens());
        cfg.ctx_size = static_cast<int>(std::min<uint64_t>(p.n_ctx, longest + max_tokens));
        cfg.position = {0, 1};
        cfg.layers = {0, static_cast<int>(p.n_layer)};
        cfg.speculative_max_tokens = static_cast<int>(draft_max);
        std::unique_ptr<rt::inference::Executor> executor = std::make_unique<rt::adapters::HipStageExecutor>(cfg);
        if (n_requests > 1) {
            rt::pipeline_parallel::ContinuousBatchingConfig bc;
            bc.max_batch_size = n_requests;
            bc.max_wait = std::chrono::microseconds(batch_wait_us);
            executor = std::make_unique<rt::pipeline_parallel::ContinuousBatchingExecutor>(std::move(executor), bc);
        }
        std::unique_ptr<rt::speculative::PromptLookupDraft> draft;
        if (draft_max > 0) draft = std::make_unique<rt::speculative::PromptLookupDraft>(max_ngram, min_ngram);

        // decode phases start together: the last runner to finish its prefill releases the others
        using clock = std::chrono::steady_clock;
        std::mutex gate_mutex;
        std::condition_variable gate;
        uint32_t waiting = n_requests;
        clock::time_point decode_start;
        auto arrive = [&] {
            std::unique_lock lock(gate_mutex);
            if (--waiting == 0) {
                decode_start = clock::now();
                gate.notify_all();
            } else {
                gate.wait(lock, [&] { return waiting == 0; });
            }
        };
        std::vector<rt::GenerationResult> results(n_requests);
        std::vector<jfh::PrefillMetrics> prefill(n_requests);
        std::vector<std::thread> runners;
        for (uint32_t i = 0; i < n_requests; ++i) {
            runners.emplace_back([&, i] {
                bool arrived = false;
                rt::GenerationRequest req;
                req.session_id = "session-" + std::to_string(i);
                req.request_id = "request-" + std::to_string(i);
                req.prompt = req_prompts[i];
                req.max_tokens = static_cast<int>(max_tokens);
                req.layer_count = static_cast<int>(p.n_layer);
                req.after_prefill = [&] {
                    arrived = true;
                    arrive();
                };
                try {
                    results[i] = rt::run_generation(*executor, req, draft.get(), static_cast<int>(draft_max));
                    prefill[i] = jfh::Engine::last_prefill_metrics();  // the prefill ran on this thread
                } catch (const std::exception& e) {
                    results[i].ok = false;
                    results[i].error_code = "generation_failed";
                    results[i].error_message = e.what();
                }
                if (!arrived) arrive();  // a runner that failed before decoding must not hold the others
            });
        }
        for (std::thread& t : runners) t.join();
        clock::time_point last = decode_start;
        for (uint32_t i = 0; i < n_requests; ++i) {
            const rt::GenerationResult& r = results[i];
            if (!r.ok) throw jfh::Error(jfh::Status::InvalidArgument, r.error_code + ": " + r.error_message);
            for (size_t k = 0; k < r.sampled_tokens.size(); ++k) {
                out_tokens[static_cast<size_t>(i) * max_tokens + k] = static_cast<int32_t>(r.sampled_tokens[k]);
            }
            out_counts[i] = static_cast<uint32_t>(r.sampled_tokens.size());
            if (stats) {
                fill_stats(*engine->engine, r, prefill[i], static_cast<uint32_t>(cfg.ctx_size), prompt_lengths[i],
                           stats[i]);
            }
            // the decode ends with a runner's last token; closing its session (freeing the
            // KV cache) follows and is not decode work, as in the runner's own decode_ms
            last = std::max(last, r.decode_end);
        }
        if (decode_wall_ms) *decode_wall_ms = std::chrono::duration<double, std::milli>(last - decode_start).count();
    });
}

}  // extern "C"
