// HIP Qwen2 stage engine (host side).
#include "jfh_engine.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstring>

namespace jfh {
namespace {

// Token rows up to which matmuls normalize their input in the prologue (from
// 3 rows on, the rows are normalized and quantized once, as the token-quad
// matrix-core path takes int8 rows).
constexpr int32_t kNormedPrologueRows = 2;

// Logits rows from which the head runs in the wide matmul (below: token quads).
constexpr int32_t kWideHeadFromRows = gpu::kQuadGroupRows + 1;

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

// The last prefill's metrics per calling thread (Engine::last_prefill_metrics).
thread_local PrefillMetrics t_last_prefill;

// ------------------------------------------------------------------ Session
Session::Session(Engine* engine, uint32_t capacity)
    : engine_(engine), capacity_(capacity), stride_((std::max<uint32_t>(capacity, 16) + 15) / 16 * 16) {
    const ModelParams& p = engine->params();
    const size_t elems = static_cast<size_t>(engine->resident_layers()) * p.n_head_kv * stride_ * p.head_dim;
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

namespace {

// Codes of one 256-value GGML block of a row, as unsigned 2/6-bit codes (Q2_K, Q6_K).
void q6k_codes(const uint8_t* blk, uint8_t* code) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t h = qh[32 * n + l];
            code[128 * n + l] = static_cast<uint8_t>((ql[64 * n + l] & 0xF) | ((h & 3) << 4));
            code[128 * n + l + 32] = static_cast<uint8_t>((ql[64 * n + l + 32] & 0xF) | (((h >> 2) & 3) << 4));
            code[128 * n + l + 64] = static_cast<uint8_t>((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4));
            code[128 * n + l + 96] = static_cast<uint8_t>((ql[64 * n + l + 32] >> 4) | (((h >> 6) & 3) << 4));
        }
    }
}

void q2k_codes(const uint8_t* blk, uint8_t* code) {
    const uint8_t* qs = blk + 16;
    for (int n = 0; n < 2; ++n) {
        for (int r = 0; r < 4; ++r) {
            for (int l = 0; l < 32; ++l) code[128 * n + 32 * r + l] = static_cast<uint8_t>((qs[32 * n + l] >> (2 * r)) & 3);
        }
    }
}

}  // namespace

// One 16-row x 256-value tile (gfx950 layout, jfh_kernels.hpp) from the
// rows' GGML blocks; absent rows (nullptr) are zero. Lane l = i + 16 g of a
// wave owns row i's values 64 g .. 64 g + 63.
void build_tile(uint32_t type, const uint8_t* const* blk, uint8_t* tile) {
    std::memset(tile, 0, gpu::tile_bytes(type));
    auto lane_chunk = [&](uint32_t base, uint32_t chunk, uint32_t lane) { return tile + base + (chunk * 64 + lane) * 16; };
    switch (type) {
    case kQ4_K:
        for (uint32_t i = 0; i < 16; ++i) {
            if (!blk[i]) continue;
            // header: d, dmin, then the eight 6-bit scale/min pairs regrouped
            // per lane group g into 24-bit fields (sc 2g | sc 2g+1 | m 2g |
            // m 2g+1) at bit 24 g of the 12 scale bytes
            std::memcpy(tile + 16 * i, blk[i], 4);
            const uint8_t* q = blk[i] + 4;
            int sc[8], mn[8];
            for (int j = 0; j < 8; ++j) {
                if (j < 4) {
                    sc[j] = q[j] & 63;
                    mn[j] = q[j + 4] & 63;
                } else {
                    sc[j] = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
                    mn[j] = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
                }
            }
            uint8_t packed[12] = {};
            for (uint32_t g = 0; g < 4; ++g) {
                const uint32_t f = static_cast<uint32_t>(sc[2 * g]) | (static_cast<uint32_t>(sc[2 * g + 1]) << 6) |
                                   (static_cast<uint32_t>(mn[2 * g]) << 12) | (static_cast<uint32_t>(mn[2 * g + 1]) << 18);
                for (uint32_t b = 0; b < 3; ++b) packed[3 * g + b] = static_cast<uint8_t>(f >> (8 * b));
            }
            std::memcpy(tile + 16 * i + 4, packed, 12);
            for (uint32_t g = 0; g < 4; ++g) {
                for (uint32_t c = 0; c < 2; ++c) std::memcpy(lane_chunk(256, c, i + 16 * g), blk[i] + 16 + 32 * g + 16 * c, 16);
            }
        }
        return;
    case kQ6_K:
        for (uint32_t i = 0; i < 16; ++i) {
            if (!blk[i]) continue;
            std::memcpy(tile + 2 * i, blk[i] + 208, 2);
            std::memcpy(tile + 32 + 16 * i, blk[i] + 192, 16);
            uint8_t code[256];
            q6k_codes(blk[i], code);
            for (uint32_t g = 0; g < 4; ++g) {
                const uint8_t* v = code + 64 * g;
                uint32_t dw[12] = {};
                for (uint32_t k = 0; k < 8; ++k) {
                    for (uint32_t e = 0; e < 4; ++e) {
                        dw[k] |= static_cast<uint32_t>((v[8 * k + e] & 0xF) | ((v[8 * k + 4 + e] & 0xF) << 4)) << (8 * e);
                    }
                }
                for (uint32_t m = 0; m < 4; ++m) {
                    for (uint32_t e = 0; e < 4; ++e) {
                        uint32_t hb = 0;
                        for (uint32_t r = 0; r < 4; ++r) hb |= static_cast<uint32_t>(v[16 * m + 4 * r + e] >> 4) << (2 * r);
                        dw[8 + m] |= hb << (8 * e);
                    }
                }
                for (uint32_t c = 0; c < 3; ++c) std::memcpy(lane_chunk(288, c, i + 16 * g), dw + 4 * c, 16);
            }
        }
        return;
    case kQ8_0:
        for (uint32_t i = 0; i < 16; ++i) {
            if (!blk[i]) continue;
            for (uint32_t j = 0; j < 8; ++j) std::memcpy(tile + 16 * i + 2 * j, blk[i] + 34 * j, 2);
            for (uint32_t g = 0; g < 4; ++g) {
                for (uint32_t c = 0; c < 4; ++c) {
                    const uint8_t* b = blk[i] + 34 * (2 * g + c / 2) + 2 + 16 * (c % 2);
                    std::memcpy(lane_chunk(256, c, i + 16 * g), b, 16);
                }
            }
        }
        return;
    case kQ2_K:
        for (uint32_t i = 0; i < 16; ++i) {
            if (!blk[i]) continue;
            std::memcpy(tile + 4 * i, blk[i] + 80, 4);
            std::memcpy(tile + 64 + 16 * i, blk[i], 16);
            uint8_t code[256];
            q2k_codes(blk[i], code);
            for (uint32_t g = 0; g < 4; ++g) {
                const uint8_t* v = code + 64 * g;
                uint32_t dw[4] = {};
                for (uint32_t m = 0; m < 4; ++m) {
                    for (uint32_t e = 0; e < 4; ++e) {
                        for (uint32_t r = 0; r < 4; ++r) {
                            dw[m] |= static_cast<uint32_t>(v[16 * m + 4 * r + e]) << (8 * e + 2 * r);
                        }
                    }
                }
                std::memcpy(lane_chunk(320, 0, i + 16 * g), dw, 16);
            }
        }
        return;
    default:
        fail(Status::FormatError, std::string("unsupported tensor type ") + type_name(type) + " for a device matrix");
    }
}

uint32_t Engine::device_row(const TensorRef& r, uint32_t row) {
    switch (r.kind) {
    case 1: {
        // q/k heads: physical row 2i holds head row i, 2i + 1 holds head row i + head_dim/2
        const uint32_t hd = r.head_dim, head = row / hd, i = row % hd;
        const uint32_t within = i < hd / 2 ? 2 * i : 2 * (i - hd / 2) + 1;
        return r.offset + head * hd + within;
    }
    case 2:
        return (row / gpu::kGluGroup) * 2 * gpu::kGluGroup + row % gpu::kGluGroup;
    case 3:
        return (row / gpu::kGluGroup) * 2 * gpu::kGluGroup + gpu::kGluGroup + row % gpu::kGluGroup;
    default:
        return r.offset + row;
    }
}

const Engine::DeviceTensor& Engine::upload_rows(const std::string& key, uint32_t type, uint64_t cols,
                                                const std::vector<RowSource>& rows, const float* bias) {
    DeviceTensor d;
    d.mat.type = type;
    d.mat.rows = static_cast<uint32_t>(rows.size());
    d.mat.cols = static_cast<uint32_t>(cols);
    const uint64_t src_rb = row_bytes(type, cols);
    std::vector<uint8_t> data;
    const uint32_t TB = gpu::tile_bytes(type);
    if (TB == 0) {
        if (type != kF32 && type != kF16) {
            fail(Status::FormatError, std::string("unsupported tensor type ") + type_name(type) + " for a device matrix");
        }
        d.mat.row_bytes = static_cast<uint32_t>(src_rb);
        data.resize(rows.size() * src_rb);
        for (size_t r = 0; r < rows.size(); ++r) {
            std::memcpy(data.data() + r * src_rb, rows[r].tensor->data + static_cast<uint64_t>(rows[r].row) * src_rb, src_rb);
        }
    } else {
        if (cols % 256 != 0) fail(Status::FormatError, "quantized matrices need row lengths that are multiples of 256");
        const uint64_t nb = cols / 256, n_rg = (rows.size() + 15) / 16;
        const uint64_t blk_bytes = src_rb / nb;  // one 256-value block (8 Q8_0 blocks)
        data.resize(n_rg * nb * TB);
        for (uint64_t rg = 0; rg < n_rg; ++rg) {
            for (uint64_t b = 0; b < nb; ++b) {
                const uint8_t* src[16];
                for (uint32_t i = 0; i < 16; ++i) {
                    const uint64_t r = rg * 16 + i;
                    src[i] = r < rows.size()
                                 ? rows[r].tensor->data + static_cast<uint64_t>(rows[r].row) * src_rb + b * blk_bytes
                                 : nullptr;
                }
                build_tile(type, src, data.data() + (rg * nb + b) * TB);
            }
        }
    }
    d.bytes = rows.size() * src_rb;
    void* mp = device_alloc(data.size());
    hip_check(hipMemcpy(mp, data.data(), data.size(), hipMemcpyHostToDevice), "upload matrix");
    d.mat.data = static_cast<const uint8_t*>(mp);
    if (bias) {
        void* bp = device_alloc(rows.size() * sizeof(float));
        hip_check(hipMemcpy(bp, bias, rows.size() * sizeof(float), hipMemcpyHostToDevice), "upload bias");
        d.mat.bias = static_cast<const float*>(bp);
    }
    return matrices_.emplace(key, d).first->second;
}

void Engine::add_ref(const TensorView& t, const DeviceTensor& dev, uint32_t offset, uint32_t kind) {
    TensorRef r;
    r.dev = &dev;
    r.rows = static_cast<uint32_t>(t.size / row_bytes(t.type, t.shape[0]));
    r.offset = offset;
    r.kind = kind;
    r.head_dim = params_.head_dim;
    refs_[t.name] = r;
    weight_bytes_ += t.size;
}

const Engine::DeviceTensor& Engine::upload_single(const TensorView& t) {
    const uint64_t cols = t.shape[0];
    const uint32_t rows = static_cast<uint32_t>(t.size / row_bytes(t.type, cols));
    std::vector<RowSource> order(rows);
    for (uint32_t r = 0; r < rows; ++r) order[r] = {&t, r};
    const DeviceTensor& d = upload_rows(t.name, t.type, cols, order, nullptr);
    add_ref(t, d, 0, 0);
    return d;
}

const Engine::TensorRef& Engine::find_ref(const std::string& name) const {
    auto it = refs_.find(name);
    if (it == refs_.end()) fail(Status::NotFound, "tensor is not resident as a matrix: " + name);
    return it->second;
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
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
        fail(Status::DeviceError, "the native engine's kernels are built for gfx950 only; device is " + device_name_);
    }
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "create stream");
    for (hipEvent_t* e : {&ev_begin_, &ev_compute_, &ev_output_}) hip_check(hipEventCreate(e), "create timing event");
    hip_check(hipEventCreateWithFlags(&ev_order_, hipEventDisableTiming), "create ordering event");
    try {
        gpu::scratch_setup(options.device);
    } catch (const std::exception& e) {
        fail(Status::DeviceError, e.what());
    }

    // a pipeline stage holds the model's layer range [layer_start, layer_end)
    // (engine.c:181-196): the first stage the embedding, the last the head
    layer_start_ = model.layer_start();
    layer_end_ = model.layer_end();
    if (layer_start_ >= layer_end_ || layer_end_ > params_.n_layer) {
        fail(Status::InvalidArgument, "native Qwen2 layer range is invalid");
    }
    const ModelParams& p = params_;
    if (p.head_dim % 2 != 0 || p.head_dim > 128) fail(Status::InvalidArgument, "unsupported head dimension");
    if (p.n_embd % 4 != 0) fail(Status::InvalidArgument, "hidden size must be a multiple of 4");
    const uint32_t G = p.n_head / p.n_head_kv;
    const uint32_t attn_rows = static_cast<uint32_t>(gpu::attention_max_rows(static_cast<int32_t>(p.head_dim)));
    prefill_chunk_ = std::max<uint32_t>(1, std::min<uint32_t>(gpu::kMaxRows, attn_rows / G));

    if (p.head_dim % 4 != 0) fail(Status::InvalidArgument, "head dimension must be a multiple of 4");
    if (p.n_ff % gpu::kGluGroup != 0) fail(Status::InvalidArgument, "feed-forward length must be a multiple of 8");
    if (first_stage()) embd_ = &upload_single(model.require("token_embd.weight"));
    if (last_stage()) {
        output_norm_ = upload_f32(model.require("output_norm.weight"));
        const TensorView& out = model.require("output.weight");
        std::vector<float> bias;
        if (const TensorView* b = model.find("output.bias")) {
            if (b->type != kF32) fail(Status::FormatError, "tensor must be F32: " + b->name);
            bias.assign(reinterpret_cast<const float*>(b->data), reinterpret_cast<const float*>(b->data) + b->size / 4);
            weight_bytes_ += b->size;
        }
        const uint32_t rows = static_cast<uint32_t>(out.size / row_bytes(out.type, out.shape[0]));
        if (!bias.empty() && bias.size() != rows) fail(Status::FormatError, "output.bias does not match output.weight");
        std::vector<RowSource> order(rows);
        for (uint32_t r = 0; r < rows; ++r) order[r] = {&out, r};
        output_ = &upload_rows(out.name, out.type, out.shape[0], order, bias.empty() ? nullptr : bias.data());
        add_ref(out, *output_, 0, 0);
    }
    const uint32_t Hq = p.n_head * p.head_dim, KV = p.n_head_kv * p.head_dim;
    for (uint32_t l = layer_start_; l < layer_end_; ++l) {
        const std::string pre = "blk." + std::to_string(l) + ".";
        Layer L{};
        L.attn_norm = upload_f32(model.require(pre + "attn_norm.weight"));
        L.ffn_norm = upload_f32(model.require(pre + "ffn_norm.weight"));
        const TensorView& wq = model.require(pre + "attn_q.weight");
        const TensorView& wk = model.require(pre + "attn_k.weight");
        const TensorView& wv = model.require(pre + "attn_v.weight");
        const TensorView& gate = model.require(pre + "ffn_gate.weight");
        const TensorView& up = model.require(pre + "ffn_up.weight");
        if (wq.type != wk.type || wq.type != wv.type || gate.type != up.type) {
            fail(Status::FormatError, "q/k/v and gate/up of a layer must share one tensor type");
        }
        // fused q|k|v rows (q and k in RoPE pair order) with their biases
        std::vector<RowSource> order(Hq + 2 * KV);
        std::vector<float> bias(Hq + 2 * KV);
        const TensorView* parts[3] = {&wq, &wk, &wv};
        const char* bias_names[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
        const uint32_t offsets[3] = {0, Hq, Hq + KV}, counts[3] = {Hq, KV, KV}, kinds[3] = {1, 1, 0};
        for (int i = 0; i < 3; ++i) {
            const TensorView& b = model.require(pre + bias_names[i]);
            if (b.type != kF32 || b.size != counts[i] * 4) fail(Status::FormatError, "bias shape mismatch: " + b.name);
            TensorRef ref;
            ref.offset = offsets[i];
            ref.kind = kinds[i];
            ref.head_dim = p.head_dim;
            for (uint32_t r = 0; r < counts[i]; ++r) {
                const uint32_t dr = device_row(ref, r);
                order[dr] = {parts[i], r};
                bias[dr] = reinterpret_cast<const float*>(b.data)[r];
            }
            weight_bytes_ += b.size;
        }
        L.qkv = &upload_rows(pre + "attn_qkv", wq.type, wq.shape[0], order, bias.data());
        for (int i = 0; i < 3; ++i) add_ref(*parts[i], *L.qkv, offsets[i], kinds[i]);
        // gate/up interleaved in groups of kGluGroup rows
        std::vector<RowSource> glu(2 * p.n_ff);
        for (uint32_t r = 0; r < p.n_ff; ++r) {
            TensorRef g, u;
            g.kind = 2;
            u.kind = 3;
            glu[device_row(g, r)] = {&gate, r};
            glu[device_row(u, r)] = {&up, r};
        }
        L.gate_up = &upload_rows(pre + "ffn_gate_up", gate.type, gate.shape[0], glu, nullptr);
        add_ref(gate, *L.gate_up, 0, 2);
        add_ref(up, *L.gate_up, 0, 3);
        L.o = &upload_single(model.require(pre + "attn_output.weight"));
        L.down = &upload_single(model.require(pre + "ffn_down.weight"));
        for (const DeviceTensor* t : {L.qkv, L.o, L.gate_up, L.down}) {
            if (quantized(t->mat.type) && t->mat.cols % gpu::kActBlock != 0) {
                fail(Status::FormatError, "quantized matrices need row lengths that are multiples of 256");
            }
        }
        layers_.push_back(L);
    }
    if (output_ && quantized(output_->mat.type) && output_->mat.cols % gpu::kActBlock != 0) {
        fail(Status::FormatError, "quantized matrices need row lengths that are multiples of 256");
    }

    const int32_t H = static_cast<int32_t>(p.n_embd), F = static_cast<int32_t>(p.n_ff);
    const size_t R = gpu::kMaxRows;
    h_ = static_cast<float*>(device_alloc(R * H * sizeof(float)));
    q_ = static_cast<float*>(device_alloc(R * Hq * sizeof(float)));
    attn_ = static_cast<float*>(device_alloc(R * Hq * sizeof(float)));
    ffn_ = static_cast<float*>(device_alloc(R * F * sizeof(float)));
    if (last_stage()) logits_ = static_cast<float*>(device_alloc(R * static_cast<size_t>(p.n_vocab) * sizeof(float)));
    best_ = static_cast<unsigned long long*>(device_alloc(R * sizeof(unsigned long long)));
    // argmax slots start cleared; k_embed and k_finish clear them for every step
    hip_check(hipMemset(best_, 0, R * sizeof(unsigned long long)), "clear argmax slots");
    // int8 rows with room for the scales of 32-value blocks (the block size is the consumer's)
    auto act8 = [&](int32_t K, int32_t blk) {
        gpu::Act8 a;
        a.K = K;
        a.blk = blk;
        a.q = static_cast<int8_t*>(device_alloc(R * K));
        a.d = static_cast<float*>(device_alloc(R * (K / gpu::kActBlock32) * sizeof(float)));
        a.s = static_cast<int16_t*>(device_alloc(R * (K / 16) * sizeof(int16_t)));
        return a;
    };
    if (quantized(layers_[0].o->mat.type) && Hq % 256 == 0) xq_attn_ = act8(Hq, gpu::act_block(layers_[0].o->mat.type));
    if (quantized(layers_[0].down->mat.type) && F % 256 == 0) xq_ffn_ = act8(F, gpu::act_block(layers_[0].down->mat.type));
    if ((quantized(layers_[0].qkv->mat.type) || quantized(layers_[0].gate_up->mat.type)) && H % 256 == 0) {
        xq_norm_ = act8(H, gpu::kActBlock);
    }
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
    for (hipEvent_t e : {ev_begin_, ev_compute_, ev_output_, ev_order_}) {
        if (e) (void) hipEventDestroy(e);
    }
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
    attn_capacity_ = static_cast<int32_t>(cap);
    const size_t partial_floats = gpu::attention_partial_floats(gpu::kMaxRows, static_cast<int32_t>(p.n_head),
                                                                static_cast<int32_t>(p.head_dim), splits_);
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
    const auto t0 = std::chrono::steady_clock::now();
    std::unique_ptr<Session> s(new Session(this, capacity));
    s->prefill_metrics_.allocation_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return s;
}

namespace {

uint64_t mat_bytes(const gpu::DMat& m) { return static_cast<uint64_t>(m.rows) * row_bytes(m.type, m.cols); }

std::string gemv_label(const gpu::GemvArgs& a) {
    const uint32_t t = a.mat.type;
    const bool fl = t == kF32 || t == kF16;
    // int8 or normalized rows of the quantized formats run in token quads (4, 8 or 16 slots)
    const bool quads = quantized(t) && (a.xq.q != nullptr || a.x.gain != nullptr) && a.n_tok >= gpu::kQuadMinRows;
    const int nt = a.n_tok > (quads ? gpu::kQuadGroupRows : 8) ? (quads ? gpu::kQuadGroupRows : 8) : a.n_tok;
    const int slot = quads ? (nt <= 4 ? 4 : nt <= 8 ? 8 : gpu::kQuadGroupRows)
                           : nt <= 2 ? nt : nt <= 4 ? 4 : nt <= 6 ? 6 : 8;
    if (fl) return "k_gemv_f<" + std::to_string(nt) + ">";
    // template arguments of the launched kernel: type, token slots, input kind
    // (0 int8 rows, 1 RMS-normalized float rows, 2 float rows)
    const int in = a.xq.q ? 0 : a.x.gain ? 1 : 2;
    return "k_mm<" + std::to_string(t) + "," + std::to_string(slot) + "," + std::to_string(in) + ">";
}

// Algorithmic HBM bytes of one matmul launch: encoded weights and bias, the
// float activation rows (and norm gain), and what the epilogue writes (and
// reads back for residual adds).
double gemv_bytes(const gpu::GemvArgs& a) {
    const double rows = a.mat.rows, K = a.mat.cols, n = a.n_tok;
    double w = static_cast<double>(mat_bytes(a.mat)) + (a.mat.bias ? 4.0 * rows : 0.0);
    double in = a.xq.q ? n * K * (1.0 + 4.0 / a.xq.blk + 2.0 / 16.0) : n * K * 4.0 + (a.x.gain ? K * 4.0 : 0.0);
    double out = n * rows * 4.0;
    switch (a.mode) {
    case gpu::kAdd: out *= 2.0; break;
    case gpu::kSwiGLU: out = n * rows / 2 * 4.0; break;
    case gpu::kLogits: out = a.store_logits ? out : 0.0; break;
    case gpu::kQKV: {
        const double hq = static_cast<double>(a.qkv.n_head) * a.qkv.head_dim;
        out = n * hq * 4.0 + n * (rows - hq) * 2.0;
        break;
    }
    default: break;
    }
    return w + in + out;
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
    prof_->push_back(e);
    gpu::set_launch_events(e.begin, e.end);
    try {
        fn();
    } catch (...) {
        gpu::set_launch_events(nullptr, nullptr);
        throw;
    }
    gpu::set_launch_events(nullptr, nullptr);
}

void Engine::record(int32_t n_rows, int32_t max_len, int32_t n_seq, int32_t n_out, bool store_logits) {
    const ModelParams& p = params_;
    const int32_t H = static_cast<int32_t>(p.n_embd), F = static_cast<int32_t>(p.n_ff);
    const int32_t Hq = static_cast<int32_t>(p.n_head * p.head_dim);
    const double n = n_rows;
    hipStream_t s = stream_;
    // the first stage embeds token ids; later stages find their input rows in h_
    if (first_stage()) {
        timed("k_embed", n * H * 4.0 + n * static_cast<double>(row_bytes(embd_->mat.type, H)), [&] {
            gpu::launch_embed(embd_->mat, step_dev_, h_, n_rows, H, best_, gpu::kMaxRows, s);
        });
    }
    // Steps of a format's wide_min_rows rows or more run its matrices in the
    // wide matmul with int8 rows quantized once per step (same codes as the
    // decode prologue, same results per row); shorter ones in token-quad
    // groups. The head goes wide only beyond one token-quad group: below,
    // the quads' row groups per work-group merge the argmax more cheaply.
    auto matmul = [&](gpu::GemvArgs& a, const char* role) {
        const int32_t min_rows = gpu::wide_min_rows(a.mat.type);
        const int32_t from = a.mode == gpu::kLogits ? std::max(min_rows, kWideHeadFromRows) : min_rows;
        if (min_rows > 0 && a.n_tok >= from && a.n_tok <= gpu::kWideRows && a.xq.q != nullptr) {
            timed("k_mm_wide<" + std::to_string(a.mat.type) + ">:" + role, gemv_bytes(a),
                  [&] { gpu::launch_gemv_wide(a, s); });
        } else {
            timed(gemv_label(a) + ":" + role, gemv_bytes(a), [&] { gpu::launch_gemv(a, s); });
        }
    };
    // Normalized rows of multi-row steps are quantized once into xq_norm_
    // (the same codes the matmul prologue would stage): a draft-verify group
    // then stages int8 rows instead of normalizing them in every work-group.
    // The block size is the consuming matrix's (32 values for Q8_0, else 256).
    auto normed = [&](gpu::GemvArgs& a, const float* gain) {
        const int32_t blk = gpu::act_block(a.mat.type);
        if (n_rows > kNormedPrologueRows && quantized(a.mat.type) && xq_norm_.q) {
            gpu::Act8 xq = xq_norm_;
            xq.blk = blk;
            timed("k_quantize_norm", n * H * 9.1,
                  [&] { gpu::launch_quantize_norm(h_, H, nullptr, gain, p.rms_eps, n_rows, xq, s); });
            a.xq = xq;
        } else {
            a.x = {h_, H, nullptr, gain, p.rms_eps};
            a.ablk = blk;
        }
    };
    // attention split slots this step shape can fill (a prefill chunk: few long splits)
    const int32_t slots = gpu::attention_slots(splits_, attn_capacity_, n_rows, n_seq);
    // l: the resident layer (its slot in the sessions' caches)
    for (uint32_t l = 0; l < layers_.size(); ++l) {
        const Layer& L = layers_[l];
        gpu::GemvArgs qkv;
        qkv.mat = L.qkv->mat;
        qkv.mode = gpu::kQKV;
        qkv.n_tok = n_rows;
        normed(qkv, L.attn_norm);
        qkv.qkv.step = step_dev_;
        qkv.qkv.rope = rope_;
        qkv.qkv.q = q_;
        qkv.qkv.layer = static_cast<int32_t>(l);
        qkv.qkv.n_head = static_cast<int32_t>(p.n_head);
        qkv.qkv.n_head_kv = static_cast<int32_t>(p.n_head_kv);
        qkv.qkv.head_dim = static_cast<int32_t>(p.head_dim);
        matmul(qkv, "qkv");
        timed("k_attention", attn_kv_bytes_ + n * Hq * 4.0, [&] {
            gpu::launch_attention(q_, step_dev_, max_len, n_seq, static_cast<int32_t>(l), static_cast<int32_t>(p.n_head),
                                  static_cast<int32_t>(p.n_head_kv), static_cast<int32_t>(p.head_dim), splits_, partial_, s,
                                  slots);
        });
        timed("k_attention_merge", n * Hq * 4.0 * (slots + 1.0) + (xq_attn_.q ? n * Hq * 1.1 : 0.0), [&] {
            gpu::launch_attention_merge(partial_, step_dev_, n_rows, static_cast<int32_t>(p.n_head),
                                        static_cast<int32_t>(p.head_dim), splits_, attn_, xq_attn_, s, slots);
        });
        gpu::GemvArgs o;
        o.mat = L.o->mat;
        o.mode = gpu::kAdd;
        o.n_tok = n_rows;
        if (xq_attn_.q && quantized(o.mat.type)) o.xq = xq_attn_;
        else o.x = {attn_, Hq, nullptr, nullptr, 0.0F};
        o.y = h_;
        o.y_stride = H;
        matmul(o, "attn_output");
        gpu::GemvArgs gu;
        gu.mat = L.gate_up->mat;
        gu.mode = gpu::kSwiGLU;
        gu.n_tok = n_rows;
        normed(gu, L.ffn_norm);
        gu.y = ffn_;
        gu.y_stride = F;
        matmul(gu, "ffn_gate_up");
        // The down projection reads the SwiGLU rows quantized once by
        // k_quantize: the codes its float prologue would stage, where every
        // work-group would quantize the whole row again (slower, also for a
        // single row).
        const bool int8_down = xq_ffn_.q && quantized(L.down->mat.type);
        if (int8_down) {
            timed("k_quantize", n * F * 5.1, [&] { gpu::launch_quantize(ffn_, F, n_rows, xq_ffn_, s); });
        }
        gpu::GemvArgs dn;
        dn.mat = L.down->mat;
        dn.mode = gpu::kAdd;
        dn.n_tok = n_rows;
        if (int8_down) {
            dn.xq = xq_ffn_;
        } else {
            dn.x = {ffn_, F, nullptr, nullptr, 0.0F};
            dn.ablk = gpu::act_block(dn.mat.type);
        }
        dn.y = h_;
        dn.y_stride = H;
        matmul(dn, "ffn_down");
    }
    if (n_out > 0) {
        gpu::GemvArgs head;
        head.mat = output_->mat;
        head.mode = gpu::kLogits;
        head.n_tok = n_out;
        const int32_t* out_rows =
            reinterpret_cast<const int32_t*>(reinterpret_cast<const char*>(step_dev_) + offsetof(gpu::StepDev, out_row));
        const int32_t head_blk = gpu::act_block(head.mat.type);
        if (n_out > kNormedPrologueRows && quantized(head.mat.type) && xq_norm_.q) {
            // several logits rows (draft verify, batches): normalized and quantized once
            gpu::Act8 xq = xq_norm_;
            xq.blk = head_blk;
            timed("k_quantize_norm", n_out * H * 9.1, [&] {
                gpu::launch_quantize_norm(h_, H, out_rows, output_norm_, p.rms_eps, n_out, xq, s);
            });
            head.xq = xq;
        } else {
            head.x = {h_, H, out_rows, output_norm_, p.rms_eps};
            head.ablk = head_blk;
        }
        head.y = logits_;
        head.y_stride = static_cast<int32_t>(p.n_vocab);
        head.best = best_;
        head.store_logits = store_logits ? 1 : 0;
        matmul(head, "output");
        timed("k_finish", 1024.0, [&] { gpu::launch_finish(best_, step_dev_, n_out, out_dev_, s); });
    }
}

void Engine::read_kv(const Session& s, uint32_t layer, uint32_t n, uint16_t* k, uint16_t* v) {
    std::lock_guard lock(mutex_);
    const ModelParams& p = params_;
    if (layer < layer_start_ || layer >= layer_end_ || n > s.position_) {
        fail(Status::InvalidArgument, "cache rows are outside the session");
    }
    layer -= layer_start_;  // the resident layer
    hip_check(hipStreamSynchronize(stream_), "synchronize before cache read");
    const size_t hd = p.head_dim, rows = static_cast<size_t>(n) * hd, stride = s.stride_;
    // V tiles of 16 positions, [position / 16][dim][position % 16] -> [position][dim]
    const size_t tiled = (static_cast<size_t>(n) + 15) / 16 * 16 * hd;
    std::vector<uint16_t> vt(tiled);
    for (uint32_t h = 0; h < p.n_head_kv; ++h) {
        const size_t base = (static_cast<size_t>(layer) * p.n_head_kv + h) * stride * hd;
        hip_check(hipMemcpy(k + h * rows, s.k_ + base, rows * sizeof(uint16_t), hipMemcpyDeviceToHost), "read K cache");
        hip_check(hipMemcpy(vt.data(), s.v_ + base, tiled * sizeof(uint16_t), hipMemcpyDeviceToHost), "read V cache");
        for (size_t i = 0; i < n; ++i) {
            for (size_t d = 0; d < hd; ++d) v[h * rows + i * hd + d] = vt[(i & ~size_t{15}) * hd + d * 16 + (i & 15)];
        }
    }
}

void Engine::import_kv(Session& s, uint32_t n, const uint16_t* k, const uint16_t* v) {
    std::lock_guard lock(mutex_);
    const ModelParams& p = params_;
    if (n == 0 || n > s.capacity_) fail(Status::InvalidArgument, "imported cache rows exceed the session capacity");
    hip_check(hipStreamSynchronize(stream_), "synchronize before cache import");
    const size_t hd = p.head_dim, rows = static_cast<size_t>(n) * hd, stride = s.stride_;
    // [position][dim] -> V tiles of 16 positions, [position / 16][dim][position % 16]
    // (positions past n in the last tile are zeros: never read below the session length)
    const size_t tiled = (static_cast<size_t>(n) + 15) / 16 * 16 * hd;
    std::vector<uint16_t> vt(tiled);
    for (uint32_t l = 0; l < resident_layers(); ++l) {
        for (uint32_t h = 0; h < p.n_head_kv; ++h) {
            const size_t idx = static_cast<size_t>(l) * p.n_head_kv + h;
            hip_check(hipMemcpy(s.k_ + idx * stride * hd, k + idx * rows, rows * sizeof(uint16_t),
                                hipMemcpyHostToDevice), "import K cache");
            std::fill(vt.begin(), vt.end(), uint16_t{0});
            for (size_t i = 0; i < n; ++i) {
                for (size_t d = 0; d < hd; ++d) vt[(i & ~size_t{15}) * hd + d * 16 + (i & 15)] = v[idx * rows + i * hd + d];
            }
            hip_check(hipMemcpy(s.v_ + idx * stride * hd, vt.data(), tiled * sizeof(uint16_t), hipMemcpyHostToDevice),
                      "import V cache");
        }
    }
    s.position_ = n;
    s.prefill_position_ = n;
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

void Engine::require_full_model() const {
    if (!first_stage() || !last_stage()) {
        fail(Status::InvalidArgument, "full-model native inference requires every model layer");
    }
}

void Engine::set_end_tokens(const int32_t* ids, uint32_t n) {
    if (n > static_cast<uint32_t>(gpu::kMaxEndTokens)) {
        fail(Status::InvalidArgument, "at most " + std::to_string(gpu::kMaxEndTokens) + " end-of-generation ids");
    }
    if (n > 0 && ids == nullptr) fail(Status::InvalidArgument, "end-of-generation ids are required");
    std::vector<int32_t> next;
    for (uint32_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || static_cast<uint32_t>(ids[i]) >= params_.n_vocab) {
            fail(Status::InvalidArgument, "end-of-generation id is outside model vocabulary");
        }
        next.push_back(ids[i]);
    }
    std::lock_guard lock(mutex_);
    end_tokens_ = std::move(next);
}

std::vector<int32_t> Engine::end_tokens() const {
    std::lock_guard lock(mutex_);
    return end_tokens_;
}

void Engine::forward(const std::vector<SeqStep>& steps, int32_t* out_tokens, int32_t* accepted, float* logits,
                     float* act_out, PrefillMetrics* metrics) {
    using clock = std::chrono::steady_clock;
    const auto ms_since = [](clock::time_point t) { return std::chrono::duration<double, std::milli>(clock::now() - t).count(); };
    std::lock_guard lock(mutex_);
    const auto t_input = clock::now();
    const ModelParams& p = params_;
    if (!last_stage() && act_out == nullptr) fail(Status::InvalidArgument, "a non-final stage needs an activation output");
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
        if (st.n == 0 || (st.tokens == nullptr) == (st.activations == nullptr)) {
            fail(Status::InvalidArgument, "a sequence step needs token ids or activation rows");
        }
        // token ids only enter the first stage, logits only leave the last
        if ((st.tokens != nullptr && !first_stage()) || (st.logits != 0 && !last_stage())) require_full_model();
        if (st.activations != nullptr && first_stage()) {
            fail(Status::InvalidArgument, "the first native stage does not accept activations");
        }
        if (static_cast<uint64_t>(s->position_) + st.n > s->capacity_) {
            fail(Status::InvalidArgument, "native Qwen2 step is outside session capacity");
        }
        if (st.n * G > static_cast<uint32_t>(gpu::attention_max_rows(static_cast<int32_t>(p.head_dim)))) {
            fail(Status::InvalidArgument, "too many rows for one sequence step");
        }
        if (rows + static_cast<int32_t>(st.n) > gpu::kMaxRows) fail(Status::InvalidArgument, "too many token rows in one step");
        sd.seqs[si].k = s->k_;
        sd.seqs[si].v = s->v_;
        sd.seqs[si].capacity = static_cast<int32_t>(s->stride_);
        sd.seqs[si].row0 = rows;
        sd.seqs[si].len = static_cast<int32_t>(st.n);
        sd.seqs[si].pos0 = static_cast<int32_t>(s->position_);
        for (uint32_t i = 0; i < st.n; ++i) {
            const int32_t tok = st.tokens ? st.tokens[i] : 0;
            if (st.tokens && (tok < 0 || static_cast<uint32_t>(tok) >= p.n_vocab)) {
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
                sd.draft[outs] = i + 1 < st.n && st.tokens ? st.tokens[i + 1] : -1;
                ++outs;
            }
        }
        rows += static_cast<int32_t>(st.n);
        max_len = std::max(max_len, static_cast<int32_t>(st.n));
    }
    sd.n_rows = rows;
    attn_kv_bytes_ = 0.0;
    for (size_t si = 0; si < steps.size(); ++si) {
        attn_kv_bytes_ += 2.0 * p.n_head_kv * p.head_dim * 2.0 * (sd.seqs[si].pos0 + sd.seqs[si].len);
    }
    sd.n_seq = static_cast<int32_t>(steps.size());
    sd.n_out = outs;
    sd.n_end = static_cast<int32_t>(end_tokens_.size());
    std::copy(end_tokens_.begin(), end_tokens_.end(), sd.end_token);
    const bool store = logits != nullptr && outs > 0;
    hip_check(hipMemcpyAsync(step_dev_, step_host_, sizeof(gpu::StepDev), hipMemcpyHostToDevice, stream_), "upload step");
    // input rows of a later stage: the previous stage's residual stream
    uint64_t input_bytes = sizeof(gpu::StepDev);
    for (size_t si = 0; si < steps.size(); ++si) {
        if (steps[si].activations == nullptr) continue;
        const size_t bytes = static_cast<size_t>(steps[si].n) * p.n_embd * sizeof(float);
        hip_check(hipMemcpyAsync(h_ + static_cast<size_t>(sd.seqs[si].row0) * p.n_embd, steps[si].activations, bytes,
                                 hipMemcpyHostToDevice, stream_),
                  "upload stage activations");
        input_bytes += bytes;
    }
    if (metrics) {
        metrics->host_input_ms += ms_since(t_input);
        metrics->host_input_bytes += input_bytes;
        metrics->attention_matrix_cores = p.head_dim == 64 || p.head_dim == 128;
        ++metrics->steps;
    }
    if (options_.use_graphs) {
        const uint64_t key = (static_cast<uint64_t>(rows) << 40) | (static_cast<uint64_t>(max_len) << 32) |
                             (static_cast<uint64_t>(steps.size()) << 16) | (static_cast<uint64_t>(outs) << 1) |
                             (store ? 1u : 0u);
        auto it = graphs_.find(key);
        if (it == graphs_.end()) {
            const auto t_plan = clock::now();
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
            if (metrics) {
                metrics->planning_ms += ms_since(t_plan);
                metrics->plan_reused = false;
            }
        }
        if (metrics) hip_check(hipEventRecord(ev_begin_, stream_), "time step");
        hip_check(hipGraphLaunch(it->second, stream_), "launch step graph");
    } else {
        if (metrics) hip_check(hipEventRecord(ev_begin_, stream_), "time step");
        record(rows, max_len, static_cast<int32_t>(steps.size()), outs, store);
    }
    if (metrics) hip_check(hipEventRecord(ev_compute_, stream_), "time step");
    if (outs > 0) {
        hip_check(hipMemcpyAsync(out_host_, out_dev_, sizeof(gpu::StepOut), hipMemcpyDeviceToHost, stream_),
                  "download step result");
        if (store) {
            hip_check(hipMemcpyAsync(logits, logits_, static_cast<size_t>(outs) * p.n_vocab * sizeof(float),
                                     hipMemcpyDeviceToHost, stream_),
                      "download logits");
        }
    }
    if (!last_stage()) {
        hip_check(hipMemcpyAsync(act_out, h_, static_cast<size_t>(rows) * p.n_embd * sizeof(float),
                                 hipMemcpyDeviceToHost, stream_),
                  "download stage activations");
    }
    if (metrics) hip_check(hipEventRecord(ev_output_, stream_), "time step");
    hip_check(hipStreamSynchronize(stream_), "step");
    if (metrics) {
        float compute = 0.0F, output = 0.0F;
        hip_check(hipEventElapsedTime(&compute, ev_begin_, ev_compute_), "step time");
        hip_check(hipEventElapsedTime(&output, ev_compute_, ev_output_), "step time");
        metrics->compute_ms += compute;
        metrics->output_read_ms += output;
    }
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

PrefillMetrics Engine::last_prefill_metrics() { return t_last_prefill; }

uint64_t Engine::scratch_bytes_per_row() const {
    const ModelParams& p = params_;
    const uint64_t H = p.n_embd, Hq = static_cast<uint64_t>(p.n_head) * p.head_dim, F = p.n_ff;
    auto act8 = [](const gpu::Act8& a) { return a.q ? a.K + a.K / 32 * 4 + a.K / 16 * 2 : 0; };
    uint64_t b = (H + 2 * Hq + F) * sizeof(float) + act8(xq_attn_) + act8(xq_ffn_) + act8(xq_norm_);
    b += gpu::attention_partial_floats(1, static_cast<int32_t>(p.n_head), static_cast<int32_t>(p.head_dim), splits_) *
         sizeof(float);
    if (logits_) b += static_cast<uint64_t>(p.n_vocab) * sizeof(float);
    return b;
}

BufferMetrics Engine::buffer_metrics(uint32_t capacity, uint32_t prompt_tokens, const PrefillMetrics& prefill) const {
    const ModelParams& p = params_;
    BufferMetrics m;
    const uint64_t stride = (std::max<uint32_t>(capacity, 16) + 15) / 16 * 16;  // as Session allocates
    m.kv_cache_bytes = 2ull * resident_layers() * p.n_head_kv * stride * p.head_dim * sizeof(uint16_t);
    m.prefill_scratch_bytes = scratch_bytes_per_row() * std::min<uint64_t>(prefill_chunk_, std::max<uint32_t>(1, prompt_tokens));
    m.decode_scratch_bytes = scratch_bytes_per_row();
    m.prefill_host_input_bytes = prefill.host_input_bytes;
    return m;
}

int32_t Engine::prefill(Session& s, const int32_t* tokens, uint32_t n, float* logits) {
    require_full_model();
    if (s.position_ != 0 || n == 0 || n > s.capacity_) {
        fail(Status::InvalidArgument, "native Qwen2 prefill is outside session capacity");
    }
    int32_t token = -1;
    PrefillMetrics m;
    m.allocation_ms = s.prefill_metrics_.allocation_ms;
    for (uint32_t done = 0; done < n;) {
        const uint32_t len = std::min(prefill_chunk_, n - done);
        const bool last = done + len == n;
        SeqStep st;
        st.session = &s;
        st.tokens = tokens + done;
        st.n = len;
        st.logits = last ? 1 : 0;
        forward({st}, last ? &token : nullptr, nullptr, last ? logits : nullptr, nullptr, &m);
        done += len;
    }
    s.prefill_position_ = n;
    s.prefill_metrics_ = m;
    t_last_prefill = m;
    return token;
}

int32_t Engine::stage_prefill(Session& s, const int32_t* tokens, const float* activations, uint32_t n,
                              float* act_out, float* logits) {
    if (first_stage() && activations != nullptr) {
        fail(Status::InvalidArgument, "the first native stage does not accept activations");
    }
    if (!first_stage() && tokens != nullptr) fail(Status::InvalidArgument, "only the first native stage accepts tokens");
    if (first_stage() && tokens == nullptr) fail(Status::InvalidArgument, "the first native stage requires token input");
    if (!first_stage() && (activations == nullptr || n == 0)) {
        fail(Status::InvalidArgument, "native stage activation shape is invalid");
    }
    if (!last_stage() && act_out == nullptr) fail(Status::InvalidArgument, "a non-final stage needs an activation output");
    if (s.position_ != 0 || n == 0 || n > s.capacity_) {
        fail(Status::InvalidArgument, "native Qwen2 prefill is outside session capacity");
    }
    const size_t H = params_.n_embd;
    int32_t token = -1;
    PrefillMetrics m;
    m.allocation_ms = s.prefill_metrics_.allocation_ms;
    for (uint32_t done = 0; done < n;) {
        const uint32_t len = std::min(prefill_chunk_, n - done);
        const bool last = done + len == n;
        SeqStep st;
        st.session = &s;
        st.tokens = tokens ? tokens + done : nullptr;
        st.activations = activations ? activations + done * H : nullptr;
        st.n = len;
        st.logits = last && last_stage() ? 1 : 0;
        forward({st}, st.logits ? &token : nullptr, nullptr, st.logits ? logits : nullptr,
                act_out ? act_out + done * H : nullptr, &m);
        done += len;
    }
    s.prefill_position_ = n;
    s.prefill_metrics_ = m;
    t_last_prefill = m;
    return token;
}

int32_t Engine::stage_decode(Session& s, const int32_t* token, const float* activation, float* act_out,
                             float* logits) {
    if (first_stage() && activation != nullptr) {
        fail(Status::InvalidArgument, "the first native stage does not accept decode activations");
    }
    if (!first_stage() && token != nullptr) {
        fail(Status::InvalidArgument, "only the first native stage accepts decode tokens");
    }
    if (first_stage() && token == nullptr) fail(Status::InvalidArgument, "the first native stage requires token input");
    if (!first_stage() && activation == nullptr) fail(Status::InvalidArgument, "native stage activation shape is invalid");
    if (!last_stage() && act_out == nullptr) fail(Status::InvalidArgument, "a non-final stage needs an activation output");
    if (s.position_ == 0 || s.position_ >= s.capacity_) {
        fail(Status::InvalidArgument, "native Qwen2 decode is outside session capacity");
    }
    SeqStep st;
    st.session = &s;
    st.tokens = token;
    st.activations = activation;
    st.n = 1;
    st.logits = last_stage() ? 1 : 0;
    int32_t out = -1;
    forward({st}, st.logits ? &out : nullptr, nullptr, st.logits ? logits : nullptr, act_out);
    return out;
}

void Engine::dequantize(const std::string& name, uint32_t row0, uint32_t n_rows, float* out_host) {
    std::lock_guard lock(mutex_);
    const TensorRef& ref = find_ref(name);
    const gpu::DMat& m = ref.dev->mat;
    if (n_rows == 0 || static_cast<uint64_t>(row0) + n_rows > ref.rows) {
        fail(Status::InvalidArgument, "row range is outside the tensor");
    }
    float* dev = nullptr;
    const size_t bytes = static_cast<size_t>(n_rows) * m.cols * sizeof(float);
    hip_check(hipMalloc(&dev, bytes), "allocate dequant output");
    try {
        for (uint32_t i = 0; i < n_rows; ++i) {
            gpu::launch_dequant_rows(m, static_cast<int32_t>(device_row(ref, row0 + i)), 1,
                                     dev + static_cast<size_t>(i) * m.cols, stream_);
        }
        hip_check(hipMemcpyAsync(out_host, dev, bytes, hipMemcpyDeviceToHost, stream_), "download dequant");
        hip_check(hipStreamSynchronize(stream_), "dequant");
    } catch (...) {
        (void) hipFree(dev);
        throw;
    }
    (void) hipFree(dev);
}

namespace {

// Bytes of the int8 copy of n_tok rows of K values (codes, one scale per blk
// values, one sum per 16).
size_t act8_bytes(size_t n_tok, size_t K, size_t blk) {
    return n_tok * K + n_tok * (K / blk) * sizeof(float) + n_tok * (K / 16) * 2;
}

gpu::Act8 act8_at(uint8_t* base, size_t n_tok, size_t K, int32_t blk) {
    gpu::Act8 xq;
    xq.K = static_cast<int32_t>(K);
    xq.blk = blk;
    xq.q = reinterpret_cast<int8_t*>(base);
    xq.d = reinterpret_cast<float*>(base + n_tok * K);
    xq.s = reinterpret_cast<int16_t*>(base + n_tok * K + n_tok * (K / blk) * sizeof(float));
    return xq;
}

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

// Quantized formats from 3 rows on are quantized once (xq, n_tok x K, in
// blocks of the weight type's act_block) and run on the matrix-core paths a
// step takes (token quads up to 8 rows, the wide kernel beyond, where the
// format has one); y_full receives the whole device matrix's output rows,
// n_tok x rows.
bool Engine::matmul_staged(const gpu::DMat& m, uint32_t n_tok) {
    return n_tok >= 3 && quantized(m.type) && m.cols % 256 == 0;
}

void Engine::run_matmul(const gpu::DMat& m, const float* x, uint32_t n_tok, float* y_full, const gpu::Act8& xq) {
    const int32_t min_rows = gpu::wide_min_rows(m.type);
    const bool wide = min_rows > 0 && static_cast<int32_t>(n_tok) >= min_rows &&
                      static_cast<int32_t>(n_tok) <= gpu::kWideRows && m.cols % 256 == 0;
    gpu::GemvArgs a;
    a.mat = m;
    a.mat.bias = nullptr;
    a.mode = gpu::kStore;
    a.n_tok = static_cast<int32_t>(n_tok);
    a.y = y_full;
    a.y_stride = static_cast<int32_t>(m.rows);
    if (matmul_staged(m, n_tok)) {
        gpu::launch_quantize(x, static_cast<int32_t>(m.cols), static_cast<int32_t>(n_tok), xq, stream_);
        a.xq = xq;
        if (wide) gpu::launch_gemv_wide(a, stream_);
        else gpu::launch_gemv(a, stream_);
    } else {
        a.x = {x, static_cast<int32_t>(m.cols), nullptr, nullptr, 0.0F};
        a.ablk = gpu::act_block(m.type);
        gpu::launch_gemv(a, stream_);
    }
}

void Engine::matmul(const std::string& name, const float* x_host, uint32_t n_tok, float* y_host) {
    std::lock_guard lock(mutex_);
    const TensorRef& ref = find_ref(name);
    const gpu::DMat& m = ref.dev->mat;
    if (n_tok == 0 || n_tok > static_cast<uint32_t>(gpu::kMaxRows)) {
        fail(Status::InvalidArgument, "matmul shape is outside the engine workspace");
    }
    // the whole device matrix runs through the kernels; the tensor's rows are gathered afterwards
    const size_t x_bytes = static_cast<size_t>(n_tok) * m.cols * sizeof(float);
    const size_t y_bytes = static_cast<size_t>(n_tok) * m.rows * sizeof(float);
    float *x = nullptr, *y = nullptr;
    hip_check(hipMalloc(&x, x_bytes), "allocate matmul input");
    if (hipMalloc(&y, y_bytes) != hipSuccess) {
        (void) hipFree(x);
        fail(Status::OutOfMemory, "allocate matmul output");
    }
    std::vector<float> full(static_cast<size_t>(n_tok) * m.rows);
    uint8_t* xq_mem = nullptr;
    auto release = [&] {
        (void) hipFree(x);
        (void) hipFree(y);
        if (xq_mem) (void) hipFree(xq_mem);
    };
    try {
        hip_check(hipMemcpyAsync(x, x_host, x_bytes, hipMemcpyHostToDevice, stream_), "upload activations");
        gpu::Act8 xq;
        const int32_t blk = gpu::act_block(m.type);
        if (matmul_staged(m, n_tok)) {
            hip_check(hipMalloc(&xq_mem, act8_bytes(n_tok, m.cols, blk)), "allocate int8 rows");
            xq = act8_at(xq_mem, n_tok, m.cols, blk);
        }
        run_matmul(m, x, n_tok, y, xq);
        hip_check(hipMemcpyAsync(full.data(), y, y_bytes, hipMemcpyDeviceToHost, stream_), "download matmul");
        hip_check(hipStreamSynchronize(stream_), "matmul");
    } catch (...) {
        release();
        throw;
    }
    release();
    for (uint32_t t = 0; t < n_tok; ++t) {
        for (uint32_t r = 0; r < ref.rows; ++r) {
            y_host[static_cast<size_t>(t) * ref.rows + r] = full[static_cast<size_t>(t) * m.rows + device_row(ref, r)];
        }
    }
}

void Engine::matmul_noalloc(const std::string& name, const float* x_dev, uint32_t n_tok, float* y_dev,
                            hipStream_t after) {
    std::lock_guard lock(mutex_);
    const TensorRef& ref = find_ref(name);
    const gpu::DMat& m = ref.dev->mat;
    if (n_tok == 0 || n_tok > static_cast<uint32_t>(gpu::kMaxRows)) {
        fail(Status::InvalidArgument, "matmul shape is outside the engine workspace");
    }
    // staging in the GPU's static scratch: [int8 rows][the device matrix's output rows]
    const int32_t blk = gpu::act_block(m.type);
    const size_t xq_bytes = matmul_staged(m, n_tok) ? round256(act8_bytes(n_tok, m.cols, blk)) : 0;
    const size_t y_bytes = round256(static_cast<size_t>(n_tok) * m.rows * sizeof(float));
    if (xq_bytes + y_bytes > gpu::kScratchBytes) {
        fail(Status::InvalidArgument, "allocation-free matmul of " + name + " over " + std::to_string(n_tok) +
                                          " rows needs " + std::to_string(xq_bytes + y_bytes) +
                                          " bytes of staging; the static scratch holds " +
                                          std::to_string(gpu::kScratchBytes));
    }
    uint8_t* base = static_cast<uint8_t*>(gpu::scratch_address(options_.device));
    if (base == nullptr) fail(Status::DeviceError, "the device's static scratch was not set up");
    std::lock_guard use(gpu::scratch_lock(options_.device));
    // x may still be written by work on the caller's stream
    hip_check(hipEventRecord(ev_order_, after), "order after the caller's stream");
    hip_check(hipStreamWaitEvent(stream_, ev_order_, 0), "order after the caller's stream");
    gpu::Act8 xq;
    if (xq_bytes) xq = act8_at(base, n_tok, m.cols, blk);
    float* y_full = reinterpret_cast<float*>(base + xq_bytes);
    run_matmul(m, x_dev, n_tok, y_full, xq);
    gpu::launch_gather_rows(y_full, static_cast<int32_t>(m.rows), y_dev, static_cast<int32_t>(ref.rows),
                            static_cast<int32_t>(n_tok), static_cast<int32_t>(ref.offset),
                            static_cast<int32_t>(ref.kind), static_cast<int32_t>(ref.head_dim), stream_);
    hip_check(hipStreamSynchronize(stream_), "allocation-free matmul");
}

}  // namespace jfh
