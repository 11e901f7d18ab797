// HIP Qwen2 stage engine (host side).
#include "jfh_engine.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace jfh {
namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(Status::DeviceError, std::string(what) + ": " + hipGetErrorString(e));
}

[[noreturn]] void fail(Status s, const std::string& m) { throw Error(s, m); }

// NEOX RoPE angles (qwen2_architecture.cpp:499-506): theta starts at the
// position and is multiplied by base^(-2/head_dim) once per rotated pair.
void rope_rows(float base, uint32_t hd, uint32_t begin, uint32_t count, float* out) {
    const float theta_scale = std::pow(base, -2.0F / static_cast<float>(hd));
    for (uint32_t p = 0; p < count; ++p) {
        float theta = static_cast<float>(begin + p);
        float* row = out + static_cast<size_t>(p) * hd;
        for (uint32_t i = 0; i < hd / 2; ++i) {
            row[2 * i] = std::cos(theta);
            row[2 * i + 1] = std::sin(theta);
            theta *= theta_scale;
        }
    }
}

bool quantized(uint32_t type) { return type == kQ4_K || type == kQ6_K || type == kQ8_0 || type == kQ2_K; }

}  // namespace

// ------------------------------------------------------------------ Session
Session::Session(Engine* engine, uint32_t capacity) : engine_(engine), capacity_(capacity) {
    const ModelParams& p = engine->params();
    const size_t elems = static_cast<size_t>(p.n_layer) * p.n_head_kv * capacity * p.head_dim;
    kv_bytes_ = 2 * elems * sizeof(uint16_t);
    hip_check(hipMalloc(&k_, elems * sizeof(uint16_t)), "allocate K cache");
    if (hipMalloc(&v_, elems * sizeof(uint16_t)) != hipSuccess) {
        (void) hipFree(k_);
        fail(Status::OutOfMemory, "allocate V cache");
    }
    hip_check(hipMemsetAsync(k_, 0, elems * sizeof(uint16_t), engine->stream()), "clear K cache");
    hip_check(hipMemsetAsync(v_, 0, elems * sizeof(uint16_t), engine->stream()), "clear V cache");
    hip_check(hipStreamSynchronize(engine->stream()), "clear KV cache");
}

Session::~Session() {
    (void) hipFree(k_);
    (void) hipFree(v_);
}

void Session::rollback(uint32_t n) {
    // qwen2_architecture.cpp:818-823: only the decoded suffix can be removed;
    // cached rows past the position are overwritten by later steps.
    if (n == 0 || n > position_ - prefill_position_) {
        fail(Status::InvalidArgument, "native Qwen2 rollback exceeds the decoded suffix");
    }
    position_ -= n;
}

// ------------------------------------------------------------------ Engine
void* Engine::device_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes == 0 ? 16 : bytes) != hipSuccess) {
        fail(Status::OutOfMemory, "device allocation of " + std::to_string(bytes) + " bytes failed");
    }
    allocations_.push_back(p);
    return p;
}

const float* Engine::upload_f32(const TensorView& t) {
    if (t.type != kF32) fail(Status::FormatError, "tensor must be F32: " + t.name);
    void* p = device_alloc(t.size);
    hip_check(hipMemcpy(p, t.data, t.size, hipMemcpyHostToDevice), "upload tensor");
    weight_bytes_ += t.size;
    return static_cast<const float*>(p);
}

const Engine::DeviceTensor& Engine::upload(const TensorView& t) {
    auto found = tensors_.find(t.name);
    if (found != tensors_.end()) return found->second;
    DeviceTensor d;
    const uint64_t cols = t.shape[0];
    const uint64_t rows = t.size / row_bytes(t.type, cols);
    d.mat.type = t.type;
    d.mat.rows = static_cast<uint32_t>(rows);
    d.mat.cols = static_cast<uint32_t>(cols);
    d.bytes = t.size;
    std::vector<uint8_t> main, aux;
    const uint8_t* src = t.data;
    switch (t.type) {
    case kF32:
    case kF16:
    case kQ4_K:
        d.mat.main_row_bytes = static_cast<uint32_t>(row_bytes(t.type, cols));
        break;
    case kQ6_K: {
        const uint64_t nb = cols / 256;
        d.mat.main_row_bytes = static_cast<uint32_t>(nb * 208);
        d.mat.aux_row_bytes = static_cast<uint32_t>(nb * 2);
        main.resize(rows * nb * 208);
        aux.resize(rows * nb * 2);
        for (uint64_t b = 0; b < rows * nb; ++b) {
            std::memcpy(&main[b * 208], src + b * 210, 208);
            std::memcpy(&aux[b * 2], src + b * 210 + 208, 2);
        }
        break;
    }
    case kQ8_0: {
        const uint64_t nb = cols / 32;
        d.mat.main_row_bytes = static_cast<uint32_t>(nb * 32);
        d.mat.aux_row_bytes = static_cast<uint32_t>(nb * 2);
        main.resize(rows * nb * 32);
        aux.resize(rows * nb * 2);
        for (uint64_t b = 0; b < rows * nb; ++b) {
            std::memcpy(&aux[b * 2], src + b * 34, 2);
            std::memcpy(&main[b * 32], src + b * 34 + 2, 32);
        }
        break;
    }
    case kQ2_K: {
        const uint64_t nb = cols / 256;
        d.mat.main_row_bytes = static_cast<uint32_t>(nb * 80);
        d.mat.aux_row_bytes = static_cast<uint32_t>(nb * 4);
        main.resize(rows * nb * 80);
        aux.resize(rows * nb * 4);
        for (uint64_t b = 0; b < rows * nb; ++b) {
            std::memcpy(&main[b * 80], src + b * 84, 80);
            std::memcpy(&aux[b * 4], src + b * 84 + 80, 4);
        }
        break;
    }
    default:
        fail(Status::FormatError, std::string("unsupported tensor type ") + type_name(t.type) + " for " + t.name);
    }
    const size_t main_bytes = static_cast<size_t>(rows) * d.mat.main_row_bytes;
    d.main = device_alloc(main_bytes);
    hip_check(hipMemcpy(d.main, main.empty() ? static_cast<const void*>(src) : main.data(), main_bytes,
                        hipMemcpyHostToDevice),
              "upload tensor");
    d.mat.main = static_cast<const uint8_t*>(d.main);
    if (!aux.empty()) {
        d.aux = device_alloc(aux.size());
        hip_check(hipMemcpy(d.aux, aux.data(), aux.size(), hipMemcpyHostToDevice), "upload tensor");
        d.mat.aux = static_cast<const uint8_t*>(d.aux);
    }
    weight_bytes_ += t.size;
    return tensors_.emplace(t.name, d).first->second;
}

Engine::Engine(const HostModel& model, const EngineOptions& options) : params_(model.params()), options_(options) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        fail(Status::DeviceError, "no HIP device is available for the native engine");
    }
    if (options.device < 0 || options.device >= count) fail(Status::InvalidArgument, "HIP device index is out of range");
    hip_check(hipSetDevice(options.device), "select device");
    hipDeviceProp_t prop{};
    hip_check(hipGetDeviceProperties(&prop, options.device), "device properties");
    device_name_ = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "create stream");

    if (model.layer_start() != 0 || model.layer_end() != params_.n_layer) {
        fail(Status::InvalidArgument, "the HIP engine holds every model layer on one device");
    }
    const ModelParams& p = params_;
    if (p.head_dim % 2 != 0 || p.head_dim > 128) fail(Status::InvalidArgument, "unsupported head dimension");
    if (p.n_embd % 4 != 0) fail(Status::InvalidArgument, "hidden size must be a multiple of 4");
    const uint32_t G = p.n_head / p.n_head_kv;
    prefill_chunk_ = std::max<uint32_t>(1, std::min<uint32_t>(8, 64 / G));

    embd_ = &upload(model.require("token_embd.weight"));
    output_ = &upload(model.require("output.weight"));
    output_norm_ = upload_f32(model.require("output_norm.weight"));
    if (const TensorView* b = model.find("output.bias")) {
        DeviceTensor& out = tensors_.at("output.weight");
        out.mat.bias = upload_f32(*b);
        output_ = &out;
    }
    for (uint32_t l = 0; l < p.n_layer; ++l) {
        const std::string pre = "blk." + std::to_string(l) + ".";
        Layer L{};
        L.attn_norm = upload_f32(model.require(pre + "attn_norm.weight"));
        L.ffn_norm = upload_f32(model.require(pre + "ffn_norm.weight"));
        L.bq = upload_f32(model.require(pre + "attn_q.bias"));
        L.bk = upload_f32(model.require(pre + "attn_k.bias"));
        L.bv = upload_f32(model.require(pre + "attn_v.bias"));
        L.q = &upload(model.require(pre + "attn_q.weight"));
        L.k = &upload(model.require(pre + "attn_k.weight"));
        L.v = &upload(model.require(pre + "attn_v.weight"));
        L.o = &upload(model.require(pre + "attn_output.weight"));
        L.gate = &upload(model.require(pre + "ffn_gate.weight"));
        L.up = &upload(model.require(pre + "ffn_up.weight"));
        L.down = &upload(model.require(pre + "ffn_down.weight"));
        if (L.q->mat.type != L.k->mat.type || L.q->mat.type != L.v->mat.type || L.gate->mat.type != L.up->mat.type) {
            fail(Status::FormatError, "q/k/v and gate/up of a layer must share one tensor type");
        }
        for (const DeviceTensor* t : {L.q, L.o, L.gate, L.down}) {
            if (quantized(t->mat.type) && t->mat.cols % gpu::kActBlock != 0) {
                fail(Status::FormatError, "quantized matrices need row lengths that are multiples of 256");
            }
        }
        layers_.push_back(L);
    }
    if (quantized(output_->mat.type) && output_->mat.cols % gpu::kActBlock != 0) {
        fail(Status::FormatError, "quantized matrices need row lengths that are multiples of 256");
    }
    quantized_act_ = p.n_embd % gpu::kActBlock == 0 && p.n_ff % gpu::kActBlock == 0;

    const int32_t H = static_cast<int32_t>(p.n_embd), F = static_cast<int32_t>(p.n_ff);
    const int32_t kv = static_cast<int32_t>(p.n_head_kv * p.head_dim);
    kmax_ = (std::max(H, F) + 255) / 256 * 256;
    const size_t R = gpu::kMaxRows;
    h_ = static_cast<float*>(device_alloc(R * H * sizeof(float)));
    act_.q = static_cast<int8_t*>(device_alloc(R * kmax_));
    act_.d = static_cast<float*>(device_alloc(R * (kmax_ / 256) * sizeof(float)));
    act_.s = static_cast<int16_t*>(device_alloc(R * (kmax_ / 16) * sizeof(int16_t)));
    act_.f = static_cast<float*>(device_alloc(R * kmax_ * sizeof(float)));
    act_.stride = kmax_;
    qkv_ = static_cast<float*>(device_alloc(R * (H + 2 * kv) * sizeof(float)));
    q_ = static_cast<float*>(device_alloc(R * H * sizeof(float)));
    ffn_ = static_cast<float*>(device_alloc(R * F * sizeof(float)));
    logits_ = static_cast<float*>(device_alloc(R * static_cast<size_t>(p.n_vocab) * sizeof(float)));
    best_ = static_cast<unsigned long long*>(device_alloc(R * sizeof(unsigned long long)));
    // attention split counters: zero here, and every kernel that uses them leaves them zero
    const size_t n_counters = static_cast<size_t>(gpu::kMaxSeq) * p.n_head_kv;
    counters_ = static_cast<int32_t*>(device_alloc(n_counters * sizeof(int32_t)));
    hip_check(hipMemset(counters_, 0, n_counters * sizeof(int32_t)), "clear attention counters");
    step_dev_ = static_cast<gpu::StepDev*>(device_alloc(sizeof(gpu::StepDev)));
    out_dev_ = static_cast<gpu::StepOut*>(device_alloc(sizeof(gpu::StepOut)));
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&step_host_), sizeof(gpu::StepDev), hipHostMallocDefault),
              "pinned step buffer");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&out_host_), sizeof(gpu::StepOut), hipHostMallocDefault),
              "pinned output buffer");
    std::memset(step_host_, 0, sizeof(gpu::StepDev));
    ensure_capacity(256);
}

Engine::~Engine() {
    for (auto& [key, exec] : graphs_) (void) hipGraphExecDestroy(exec);
    for (void* p : allocations_) (void) hipFree(p);
    if (partial_) (void) hipFree(partial_);
    if (rope_) (void) hipFree(rope_);
    if (step_host_) (void) hipHostFree(step_host_);
    if (out_host_) (void) hipHostFree(out_host_);
    if (stream_) (void) hipStreamDestroy(stream_);
}

void Engine::ensure_capacity(uint32_t capacity) {
    if (capacity <= capacity_max_) return;
    hip_check(hipStreamSynchronize(stream_), "synchronize before resize");
    const ModelParams& p = params_;
    const uint32_t cap = std::min<uint32_t>(p.n_ctx, std::max<uint32_t>(capacity, 256));
    std::vector<float> table(static_cast<size_t>(cap) * p.head_dim);
    rope_rows(p.rope_base, p.head_dim, 0, cap, table.data());
    if (rope_) (void) hipFree(rope_);
    rope_ = nullptr;
    hip_check(hipMalloc(&rope_, table.size() * sizeof(float)), "allocate rope table");
    hip_check(hipMemcpy(rope_, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice), "upload rope table");
    splits_ = gpu::attention_splits(static_cast<int32_t>(cap));
    const size_t partial_floats = static_cast<size_t>(gpu::kMaxRows) * p.n_head * splits_ * (p.head_dim + 2);
    if (partial_) (void) hipFree(partial_);
    partial_ = nullptr;
    hip_check(hipMalloc(&partial_, partial_floats * sizeof(float)), "allocate attention partials");
    capacity_max_ = cap;
    for (auto& [key, exec] : graphs_) (void) hipGraphExecDestroy(exec);
    graphs_.clear();
}

std::unique_ptr<Session> Engine::create_session(uint32_t capacity) {
    if (capacity == 0 || capacity > params_.n_ctx) {
        fail(Status::InvalidArgument, "native Qwen2 cache capacity is outside model context");
    }
    std::lock_guard lock(mutex_);
    ensure_capacity(capacity);
    return std::unique_ptr<Session>(new Session(this, capacity));
}

namespace {

uint64_t mat_bytes(const gpu::DMat& m) { return static_cast<uint64_t>(m.rows) * row_bytes(m.type, m.cols); }

std::string gemv_label(const gpu::GemvArgs& a) {
    const uint32_t t = a.mat[0].type;
    const bool fl = t == kF32 || t == kF16;
    const int nt = a.n_tok > 8 ? 8 : a.n_tok;
    return std::string(fl ? "k_gemv_f<" : "k_gemv_q<") + (fl ? "" : std::to_string(t) + ",") + std::to_string(nt) + ">";
}

// Algorithmic HBM bytes of one matmul launch: encoded weights, the activation
// rows (int8 + scales + sums), bias, and the output rows (read too for residual adds).
double gemv_bytes(const gpu::GemvArgs& a) {
    double w = 0.0, rows = 0.0;
    for (int i = 0; i < a.n_mat; ++i) {
        w += static_cast<double>(mat_bytes(a.mat[i]));
        rows += a.mat[i].rows;
        if (a.mat[i].bias) w += 4.0 * a.mat[i].rows;
    }
    const double K = a.mat[0].cols;
    const double act = a.n_tok * (K + K / 256 * 4 + K / 16 * 2);
    double out = a.n_tok * rows * 4.0;
    if (a.mode == gpu::kSwiGLU) out = a.n_tok * a.mat[0].rows * 4.0;
    if (a.mode == gpu::kAdd) out *= 2.0;
    if (a.mode == gpu::kLogits && !a.store_logits) out = 0.0;
    return w + act + out;
}

}  // namespace

template <typename F>
void Engine::timed(const std::string& label, double bytes, F&& fn) {
    if (!prof_) {
        fn();
        return;
    }
    ProfEvent e;
    e.label = label;
    e.bytes = bytes;
    hip_check(hipEventCreate(&e.begin), "profile event");
    hip_check(hipEventCreate(&e.end), "profile event");
    hip_check(hipEventRecord(e.begin, stream_), "profile event");
    fn();
    hip_check(hipEventRecord(e.end, stream_), "profile event");
    prof_->push_back(e);
}

void Engine::record(int32_t n_rows, int32_t max_len, int32_t n_seq, int32_t n_out, bool store_logits) {
    const ModelParams& p = params_;
    const int32_t H = static_cast<int32_t>(p.n_embd), F = static_cast<int32_t>(p.n_ff);
    const int32_t kv = static_cast<int32_t>(p.n_head_kv * p.head_dim);
    const double n = n_rows;
    const double norm_bytes = n * H * (4.0 + 4.0 + 1.0) + 4.0 * H;
    hipStream_t s = stream_;
    timed("k_embed", n * H * (4.0 + static_cast<double>(row_bytes(embd_->mat.type, H))), [&] {
        gpu::launch_embed(embd_->mat, step_dev_, h_, n_rows, H, best_, gpu::kMaxRows, s);
    });
    for (uint32_t l = 0; l < p.n_layer; ++l) {
        const Layer& L = layers_[l];
        timed("k_norm_quant", norm_bytes, [&] {
            gpu::launch_norm_quant(h_, H, L.attn_norm, p.rms_eps, H, step_dev_, 0, n_rows, quantized_act_, act_, s);
        });
        gpu::GemvArgs qkv;
        qkv.n_mat = 3;
        qkv.mat[0] = L.q->mat;
        qkv.mat[0].bias = L.bq;
        qkv.mat[1] = L.k->mat;
        qkv.mat[1].bias = L.bk;
        qkv.mat[2] = L.v->mat;
        qkv.mat[2].bias = L.bv;
        qkv.mode = gpu::kStore;
        qkv.n_tok = n_rows;
        qkv.x = act_;
        qkv.y = qkv_;
        qkv.y_stride = H + 2 * kv;
        timed(gemv_label(qkv) + ":qkv", gemv_bytes(qkv), [&] { gpu::launch_gemv(qkv, s); });
        timed("k_rope_kv", n * (H + 2 * kv) * 4.0 + n * H * 4.0 + n * 2 * kv * 2.0, [&] {
            gpu::launch_rope_kv(qkv_, n_rows, static_cast<int32_t>(p.n_head), static_cast<int32_t>(p.n_head_kv),
                                static_cast<int32_t>(p.head_dim), rope_, step_dev_, static_cast<int32_t>(l), q_, s);
        });
        timed("k_attention", n * H * 8.0, [&] {
            gpu::launch_attention(q_, step_dev_, n_rows, max_len, n_seq, static_cast<int32_t>(l),
                                  static_cast<int32_t>(p.n_head), static_cast<int32_t>(p.n_head_kv),
                                  static_cast<int32_t>(p.head_dim), splits_, partial_, counters_, act_, s);
        });
        gpu::GemvArgs o;
        o.mat[0] = L.o->mat;
        o.mode = gpu::kAdd;
        o.n_tok = n_rows;
        o.x = act_;
        o.y = h_;
        o.y_stride = H;
        timed(gemv_label(o) + ":attn_output", gemv_bytes(o), [&] { gpu::launch_gemv(o, s); });
        timed("k_norm_quant", norm_bytes, [&] {
            gpu::launch_norm_quant(h_, H, L.ffn_norm, p.rms_eps, H, step_dev_, 0, n_rows, quantized_act_, act_, s);
        });
        gpu::GemvArgs gu;
        gu.n_mat = 2;
        gu.mat[0] = L.gate->mat;
        gu.mat[1] = L.up->mat;
        gu.mode = gpu::kSwiGLU;
        gu.n_tok = n_rows;
        gu.x = act_;
        gu.y = ffn_;
        gu.y_stride = F;
        timed(gemv_label(gu) + ":ffn_gate_up", gemv_bytes(gu), [&] { gpu::launch_gemv(gu, s); });
        timed("k_quant", n * F * (4.0 + 4.0 + 1.0), [&] {
            gpu::launch_quant(ffn_, F, F, n_rows, quantized_act_, act_, s);
        });
        gpu::GemvArgs dn;
        dn.mat[0] = L.down->mat;
        dn.mode = gpu::kAdd;
        dn.n_tok = n_rows;
        dn.x = act_;
        dn.y = h_;
        dn.y_stride = H;
        timed(gemv_label(dn) + ":ffn_down", gemv_bytes(dn), [&] { gpu::launch_gemv(dn, s); });
    }
    if (n_out > 0) {
        timed("k_norm_quant", static_cast<double>(n_out) * H * 9.0 + 4.0 * H, [&] {
            gpu::launch_norm_quant(h_, H, output_norm_, p.rms_eps, H, step_dev_, 1, n_out, quantized_act_, act_, s);
        });
        gpu::GemvArgs head;
        head.mat[0] = output_->mat;
        head.mode = gpu::kLogits;
        head.n_tok = n_out;
        head.x = act_;
        head.y = logits_;
        head.y_stride = static_cast<int32_t>(p.n_vocab);
        head.best = best_;
        head.store_logits = store_logits ? 1 : 0;
        timed(gemv_label(head) + ":output", gemv_bytes(head), [&] { gpu::launch_gemv(head, s); });
        timed("k_finish", 1024.0, [&] { gpu::launch_finish(best_, step_dev_, n_out, out_dev_, s); });
    }
}

std::vector<KernelStat> Engine::profile(const std::vector<SeqStep>& steps, uint32_t iterations) {
    std::vector<ProfEvent> events;
    {
        std::lock_guard lock(mutex_);
        prof_ = &events;
    }
    std::vector<KernelStat> out;
    try {
        const bool graphs = options_.use_graphs;
        options_.use_graphs = false;
        std::vector<int32_t> ids(gpu::kMaxRows);
        for (uint32_t it = 0; it < iterations; ++it) {
            forward(steps, ids.data(), nullptr, nullptr);
            for (const SeqStep& st : steps) st.session->position_ -= st.n;
        }
        options_.use_graphs = graphs;
        std::map<std::string, size_t> index;
        for (const ProfEvent& e : events) {
            float ms = 0.0F;
            hip_check(hipEventElapsedTime(&ms, e.begin, e.end), "profile event time");
            auto it = index.find(e.label);
            if (it == index.end()) {
                it = index.emplace(e.label, out.size()).first;
                KernelStat k;
                k.label = e.label;
                out.push_back(k);
            }
            KernelStat& k = out[it->second];
            k.launches += 1;
            k.total_ms += ms;
            k.bytes += e.bytes;
        }
        for (auto& k : out) {
            k.launches /= iterations;
            k.total_ms /= iterations;
            k.bytes /= iterations;
        }
    } catch (...) {
        prof_ = nullptr;
        for (const ProfEvent& e : events) {
            (void) hipEventDestroy(e.begin);
            (void) hipEventDestroy(e.end);
        }
        throw;
    }
    prof_ = nullptr;
    for (const ProfEvent& e : events) {
        (void) hipEventDestroy(e.begin);
        (void) hipEventDestroy(e.end);
    }
    std::sort(out.begin(), out.end(), [](const KernelStat& a, const KernelStat& b) { return a.total_ms > b.total_ms; });
    return out;
}

void Engine::forward(const std::vector<SeqStep>& steps, int32_t* out_tokens, int32_t* accepted, float* logits) {
    std::lock_guard lock(mutex_);
    const ModelParams& p = params_;
    if (steps.empty() || steps.size() > static_cast<size_t>(gpu::kMaxSeq)) {
        fail(Status::InvalidArgument, "a step needs 1.." + std::to_string(gpu::kMaxSeq) + " sequences");
    }
    const uint32_t G = p.n_head / p.n_head_kv;
    gpu::StepDev& sd = *step_host_;
    int32_t rows = 0, outs = 0, max_len = 0;
    for (size_t si = 0; si < steps.size(); ++si) {
        const SeqStep& st = steps[si];
        Session* s = st.session;
        if (s == nullptr || s->engine_ != this) fail(Status::InvalidArgument, "session does not belong to this engine");
        for (size_t sj = 0; sj < si; ++sj) {
            if (steps[sj].session == s) fail(Status::InvalidArgument, "a session appears twice in one step");
        }
        if (st.n == 0 || st.tokens == nullptr) fail(Status::InvalidArgument, "a sequence step needs at least one token");
        if (static_cast<uint64_t>(s->position_) + st.n > s->capacity_) {
            fail(Status::InvalidArgument, "native Qwen2 step is outside session capacity");
        }
        if (st.n * G > 64) fail(Status::InvalidArgument, "too many rows for one sequence step");
        if (rows + static_cast<int32_t>(st.n) > gpu::kMaxRows) fail(Status::InvalidArgument, "too many token rows in one step");
        sd.seqs[si].k = s->k_;
        sd.seqs[si].v = s->v_;
        sd.seqs[si].capacity = static_cast<int32_t>(s->capacity_);
        sd.seqs[si].row0 = rows;
        sd.seqs[si].len = static_cast<int32_t>(st.n);
        sd.seqs[si].pos0 = static_cast<int32_t>(s->position_);
        for (uint32_t i = 0; i < st.n; ++i) {
            const int32_t tok = st.tokens[i];
            if (tok < 0 || static_cast<uint32_t>(tok) >= p.n_vocab) {
                fail(Status::InvalidArgument, "native token ID is outside model vocabulary");
            }
            sd.token[rows + i] = tok;
            sd.pos[rows + i] = static_cast<int32_t>(s->position_ + i);
            sd.seq[rows + i] = static_cast<int32_t>(si);
        }
        if (st.logits == 1) {
            sd.out_row[outs] = rows + static_cast<int32_t>(st.n) - 1;
            sd.draft[outs] = -1;
            ++outs;
        } else if (st.logits == 2) {
            for (uint32_t i = 0; i < st.n; ++i) {
                sd.out_row[outs] = rows + static_cast<int32_t>(i);
                sd.draft[outs] = i + 1 < st.n ? st.tokens[i + 1] : -1;
                ++outs;
            }
        }
        rows += static_cast<int32_t>(st.n);
        max_len = std::max(max_len, static_cast<int32_t>(st.n));
    }
    sd.n_rows = rows;
    sd.n_seq = static_cast<int32_t>(steps.size());
    sd.n_out = outs;
    const bool store = logits != nullptr && outs > 0;
    hip_check(hipMemcpyAsync(step_dev_, step_host_, sizeof(gpu::StepDev), hipMemcpyHostToDevice, stream_), "upload step");
    if (options_.use_graphs) {
        const uint64_t key = (static_cast<uint64_t>(rows) << 40) | (static_cast<uint64_t>(max_len) << 32) |
                             (static_cast<uint64_t>(steps.size()) << 16) | (static_cast<uint64_t>(outs) << 1) |
                             (store ? 1u : 0u);
        auto it = graphs_.find(key);
        if (it == graphs_.end()) {
            hipGraph_t graph = nullptr;
            hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
            try {
                record(rows, max_len, static_cast<int32_t>(steps.size()), outs, store);
            } catch (...) {
                (void) hipStreamEndCapture(stream_, &graph);
                if (graph) (void) hipGraphDestroy(graph);
                throw;
            }
            hip_check(hipStreamEndCapture(stream_, &graph), "end capture");
            hipGraphExec_t exec = nullptr;
            const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void) hipGraphDestroy(graph);
            hip_check(e, "instantiate step graph");
            it = graphs_.emplace(key, exec).first;
        }
        hip_check(hipGraphLaunch(it->second, stream_), "launch step graph");
    } else {
        record(rows, max_len, static_cast<int32_t>(steps.size()), outs, store);
    }
    if (outs > 0) {
        hip_check(hipMemcpyAsync(out_host_, out_dev_, sizeof(gpu::StepOut), hipMemcpyDeviceToHost, stream_),
                  "download step result");
        if (store) {
            hip_check(hipMemcpyAsync(logits, logits_, static_cast<size_t>(outs) * p.n_vocab * sizeof(float),
                                     hipMemcpyDeviceToHost, stream_),
                      "download logits");
        }
    }
    hip_check(hipStreamSynchronize(stream_), "step");
    for (int32_t i = 0; i < outs; ++i) {
        if (out_tokens) out_tokens[i] = out_host_->token[i];
    }
    if (accepted) {
        for (size_t si = 0; si < steps.size(); ++si) accepted[si] = outs > 0 ? out_host_->accepted[si] : 0;
    }
    for (const SeqStep& st : steps) {
        if (st.session->position_ == 0) st.session->prefill_position_ = st.n;
        st.session->position_ += st.n;
    }
}

int32_t Engine::prefill(Session& s, const int32_t* tokens, uint32_t n, float* logits) {
    if (s.position_ != 0 || n == 0 || n > s.capacity_) {
        fail(Status::InvalidArgument, "native Qwen2 prefill is outside session capacity");
    }
    int32_t token = -1;
    for (uint32_t done = 0; done < n;) {
        const uint32_t len = std::min(prefill_chunk_, n - done);
        const bool last = done + len == n;
        SeqStep st;
        st.session = &s;
        st.tokens = tokens + done;
        st.n = len;
        st.logits = last ? 1 : 0;
        forward({st}, last ? &token : nullptr, nullptr, last ? logits : nullptr);
        done += len;
    }
    s.prefill_position_ = n;
    return token;
}

void Engine::dequantize(const std::string& name, uint32_t row0, uint32_t n_rows, float* out_host) {
    std::lock_guard lock(mutex_);
    auto it = tensors_.find(name);
    if (it == tensors_.end()) fail(Status::NotFound, "tensor is not resident as a matrix: " + name);
    const gpu::DMat& m = it->second.mat;
    if (n_rows == 0 || static_cast<uint64_t>(row0) + n_rows > m.rows) fail(Status::InvalidArgument, "row range is outside the tensor");
    float* dev = nullptr;
    const size_t bytes = static_cast<size_t>(n_rows) * m.cols * sizeof(float);
    hip_check(hipMalloc(&dev, bytes), "allocate dequant output");
    try {
        gpu::launch_dequant_rows(m, static_cast<int32_t>(row0), static_cast<int32_t>(n_rows), dev, stream_);
        hip_check(hipMemcpyAsync(out_host, dev, bytes, hipMemcpyDeviceToHost, stream_), "download dequant");
        hip_check(hipStreamSynchronize(stream_), "dequant");
    } catch (...) {
        (void) hipFree(dev);
        throw;
    }
    (void) hipFree(dev);
}

void Engine::matmul(const std::string& name, const float* x_host, uint32_t n_tok, float* y_host) {
    std::lock_guard lock(mutex_);
    auto it = tensors_.find(name);
    if (it == tensors_.end()) fail(Status::NotFound, "tensor is not resident as a matrix: " + name);
    const gpu::DMat& m = it->second.mat;
    if (n_tok == 0 || n_tok > static_cast<uint32_t>(gpu::kMaxRows) || m.cols > static_cast<uint32_t>(kmax_)) {
        fail(Status::InvalidArgument, "matmul shape is outside the engine workspace");
    }
    hip_check(hipMemcpy2DAsync(act_.f, static_cast<size_t>(kmax_) * sizeof(float), x_host, m.cols * sizeof(float),
                               m.cols * sizeof(float), n_tok, hipMemcpyHostToDevice, stream_),
              "upload activations");
    const bool q = quantized(m.type);
    gpu::launch_quant(act_.f, kmax_, static_cast<int32_t>(m.cols), static_cast<int32_t>(n_tok), q, act_, stream_);
    float* y = nullptr;
    const size_t bytes = static_cast<size_t>(n_tok) * m.rows * sizeof(float);
    hip_check(hipMalloc(&y, bytes), "allocate matmul output");
    gpu::GemvArgs a;
    a.mat[0] = m;
    a.mat[0].bias = nullptr;
    a.mode = gpu::kStore;
    a.n_tok = static_cast<int32_t>(n_tok);
    a.x = act_;
    a.y = y;
    a.y_stride = static_cast<int32_t>(m.rows);
    try {
        gpu::launch_gemv(a, stream_);
        hip_check(hipMemcpyAsync(y_host, y, bytes, hipMemcpyDeviceToHost, stream_), "download matmul");
        hip_check(hipStreamSynchronize(stream_), "matmul");
    } catch (...) {
        (void) hipFree(y);
        throw;
    }
    (void) hipFree(y);
}

}  // namespace jfh
