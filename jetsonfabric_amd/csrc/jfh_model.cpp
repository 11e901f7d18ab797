// Host-resident Qwen2 model, synthetic weights and block quantizers.
#include "jfh_model.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

namespace jfh {
namespace {

[[noreturn]] void fail(Status s, const std::string& m) { throw Error(s, m); }

uint64_t fnv1a(const std::string& s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) { h ^= c; h *= 1099511628211ull; }
    return h;
}

uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Two standard normals for elements 2p and 2p+1 of a stream: Box-Muller on
// one 64-bit draw of a counter-based generator.
void normal_pair(uint64_t key, uint64_t p, float* a, float* b) {
    const uint64_t r = splitmix(key + p * 0xD1B54A32D192ED03ull);
    const float u1 = (static_cast<float>(r & 0xFFFFFFu) + 0.5F) * (1.0F / 16777216.0F);
    const float u2 = static_cast<float>((r >> 32) & 0xFFFFFFu) * (1.0F / 16777216.0F);
    const float rad = std::sqrt(-2.0F * std::log(u1));
    const float ang = 6.28318530718F * u2;
    *a = rad * std::cos(ang);
    *b = rad * std::sin(ang);
}

float roundf_half_away(float x) { return std::round(x); }

void q8_0_block(const float* x, uint8_t* o) {
    float amax = 0;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
    const uint16_t dh = f32_to_f16(amax / 127.0F);
    const float d = f16_to_f32(dh);
    o[0] = uint8_t(dh); o[1] = uint8_t(dh >> 8);
    for (int i = 0; i < 32; ++i) {
        float q = d > 0 ? roundf_half_away(x[i] / d) : 0.0F;
        q = std::min(127.0F, std::max(-127.0F, q));
        o[2 + i] = uint8_t(int8_t(q));
    }
}

void q4_k_block(const float* x, uint8_t* o) {
    float scale[8], minv[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float mn = 0, mx = -INFINITY;
        for (int l = 0; l < 32; ++l) { mn = std::min(mn, x[32 * j + l]); mx = std::max(mx, x[32 * j + l]); }
        scale[j] = (mx - mn) / 15.0F;
        minv[j] = -mn;
        max_scale = std::max(max_scale, scale[j]);
        max_min = std::max(max_min, minv[j]);
    }
    const uint16_t dh = f32_to_f16(max_scale / 63.0F), mh = f32_to_f16(max_min / 63.0F);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0 ? std::min(63, int(roundf_half_away(scale[j] / d))) : 0;
        m[j] = dmin > 0 ? std::min(63, int(roundf_half_away(minv[j] / dmin))) : 0;
    }
    std::memset(o, 0, 144);
    o[0] = uint8_t(dh); o[1] = uint8_t(dh >> 8); o[2] = uint8_t(mh); o[3] = uint8_t(mh >> 8);
    uint8_t* s = o + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = uint8_t(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = uint8_t(m[j] | ((m[j + 4] >> 4) << 6));
        s[j + 8] = uint8_t((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qs = o + 16;
    for (int i = 0; i < 256; ++i) {
        const int j = i / 32;
        const float d1 = d * float(sc[j]), m1 = dmin * float(m[j]);
        int q = d1 > 0 ? int(roundf_half_away((x[i] + m1) / d1)) : 0;
        q = std::min(15, std::max(0, q));
        const int pair = i / 64, within = i % 64;
        if (within < 32) qs[32 * pair + within] |= uint8_t(q);
        else qs[32 * pair + within - 32] |= uint8_t(q << 4);
    }
}

void q6_k_block(const float* x, uint8_t* o) {
    float sg[16], max_s = 0;
    for (int g = 0; g < 16; ++g) {
        float amax = 0;
        for (int l = 0; l < 16; ++l) amax = std::max(amax, std::fabs(x[16 * g + l]));
        sg[g] = amax / 31.0F;
        max_s = std::max(max_s, sg[g]);
    }
    const uint16_t dh = f32_to_f16(max_s / 127.0F);
    const float d = f16_to_f32(dh);
    std::memset(o, 0, 210);
    uint8_t* ql = o;
    uint8_t* qh = o + 128;
    int8_t* scales = reinterpret_cast<int8_t*>(o + 192);
    for (int g = 0; g < 16; ++g) scales[g] = int8_t(d > 0 ? std::min(127, int(roundf_half_away(sg[g] / d))) : 0);
    for (int i = 0; i < 256; ++i) {
        const float ds = d * float(scales[i / 16]);
        int q = ds > 0 ? int(roundf_half_away(x[i] / ds)) : 0;
        q = std::min(31, std::max(-32, q)) + 32;
        const int half = i / 128, within = i % 128, quarter = within / 32, l = within % 32;
        uint8_t* lo = ql + 64 * half;
        switch (quarter) {
        case 0: lo[l] |= uint8_t(q & 0xF); break;
        case 1: lo[l + 32] |= uint8_t(q & 0xF); break;
        case 2: lo[l] |= uint8_t((q & 0xF) << 4); break;
        default: lo[l + 32] |= uint8_t((q & 0xF) << 4); break;
        }
        qh[32 * half + l] |= uint8_t((q >> 4) << (2 * quarter));
    }
    o[208] = uint8_t(dh); o[209] = uint8_t(dh >> 8);
}

void q2_k_block(const float* x, uint8_t* o) {
    float scale[16], minv[16], max_scale = 0, max_min = 0;
    for (int g = 0; g < 16; ++g) {
        float mn = 0, mx = -INFINITY;
        for (int l = 0; l < 16; ++l) { mn = std::min(mn, x[16 * g + l]); mx = std::max(mx, x[16 * g + l]); }
        scale[g] = (mx - mn) / 3.0F;
        minv[g] = -mn;
        max_scale = std::max(max_scale, scale[g]);
        max_min = std::max(max_min, minv[g]);
    }
    const uint16_t dh = f32_to_f16(max_scale / 15.0F), mh = f32_to_f16(max_min / 15.0F);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    std::memset(o, 0, 84);
    int sc[16], m[16];
    for (int g = 0; g < 16; ++g) {
        sc[g] = d > 0 ? std::min(15, int(roundf_half_away(scale[g] / d))) : 0;
        m[g] = dmin > 0 ? std::min(15, int(roundf_half_away(minv[g] / dmin))) : 0;
        o[g] = uint8_t(sc[g] | (m[g] << 4));
    }
    uint8_t* qs = o + 16;
    for (int i = 0; i < 256; ++i) {
        const int g = i / 16;
        const float dl = d * float(sc[g]), ml = dmin * float(m[g]);
        int q = dl > 0 ? int(roundf_half_away((x[i] + ml) / dl)) : 0;
        q = std::min(3, std::max(0, q));
        const int half = i / 128, within = i % 128, shift = within / 32, part = (within % 32) / 16, l = within % 16;
        qs[32 * half + 16 * part + l] |= uint8_t(q << (2 * shift));
    }
    o[80] = uint8_t(dh); o[81] = uint8_t(dh >> 8); o[82] = uint8_t(mh); o[83] = uint8_t(mh >> 8);
}

template <typename F>
void parallel_rows(int64_t rows, int threads, F&& fn) {
    if (threads <= 0) threads = int(std::max(1u, std::thread::hardware_concurrency()));
    threads = int(std::min<int64_t>(threads, std::max<int64_t>(1, rows)));
    if (threads == 1) { fn(0, rows); return; }
    std::vector<std::thread> pool;
    const int64_t per = (rows + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        const int64_t a = t * per, b = std::min(rows, a + per);
        if (a >= b) break;
        pool.emplace_back([&, a, b] { fn(a, b); });
    }
    for (auto& th : pool) th.join();
}

}  // namespace

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return uint16_t(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return uint16_t(sign | 0x7C00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return sign;
        const uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u, shift = 126u - e;
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), mid = 1u << (shift - 1u);
        if (rem > mid || (rem == mid && (h & 1u))) ++h;
        return uint16_t(sign | h);
    }
    uint32_t h = (a >> 13) - (112u << 10);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return uint16_t(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int k = -1;
            do { ++k; m <<= 1; } while (!(m & 0x400u));
            bits = sign | (uint32_t(127 - 15 - k) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

size_t row_bytes(uint32_t type, uint64_t n) {
    uint32_t be = 0, bb = 0;
    if (!type_layout(type, &be, &bb) || n % be != 0) fail(Status::InvalidArgument, "row length does not fit the block size");
    return size_t(n / be * bb);
}

void quantize_row(uint32_t type, const float* x, uint8_t* out, int64_t n) {
    switch (type) {
    case kF32: std::memcpy(out, x, size_t(n) * 4); return;
    case kF16:
        for (int64_t i = 0; i < n; ++i) { const uint16_t h = f32_to_f16(x[i]); out[2 * i] = uint8_t(h); out[2 * i + 1] = uint8_t(h >> 8); }
        return;
    case kQ8_0: for (int64_t b = 0; b < n / 32; ++b) q8_0_block(x + 32 * b, out + 34 * b); return;
    case kQ4_K: for (int64_t b = 0; b < n / 256; ++b) q4_k_block(x + 256 * b, out + 144 * b); return;
    case kQ6_K: for (int64_t b = 0; b < n / 256; ++b) q6_k_block(x + 256 * b, out + 210 * b); return;
    case kQ2_K: for (int64_t b = 0; b < n / 256; ++b) q2_k_block(x + 256 * b, out + 84 * b); return;
    default: fail(Status::InvalidArgument, "cannot quantize to tensor type " + std::to_string(type));
    }
}

ModelParams parse_qwen2_params(const uint8_t* gguf, size_t size) {
    const auto kv = parse_gguf_kv(gguf, size);
    auto find = [&](const char* key) -> const GgufValue* {
        auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    };
    auto req_u32 = [&](const char* key) {
        const GgufValue* v = find(key);
        if (!v) fail(Status::FormatError, std::string("missing GGUF metadata key ") + key);
        if (v->kind != GgufValue::U32) fail(Status::FormatError, std::string("GGUF metadata key is not uint32: ") + key);
        return v->u32;
    };
    auto req_f32 = [&](const char* key) {
        const GgufValue* v = find(key);
        if (!v) fail(Status::FormatError, std::string("missing GGUF metadata key ") + key);
        if (v->kind != GgufValue::F32) fail(Status::FormatError, std::string("GGUF metadata key is not float32: ") + key);
        return v->f32;
    };
    const GgufValue* arch = find("general.architecture");
    if (!arch) fail(Status::FormatError, "missing GGUF metadata key general.architecture");
    if (arch->kind != GgufValue::Str || arch->str != "qwen2") {
        fail(Status::FormatError, "native execution currently supports only qwen2 GGUF models");
    }
    if (const GgufValue* t = find("qwen2.rope.scaling.type")) {
        if (t->kind != GgufValue::Str) fail(Status::FormatError, "Qwen2 RoPE scaling type is not a string");
        if (t->str != "none" && t->str != "linear") fail(Status::FormatError, "native Qwen2 does not support RoPE scaling type " + t->str);
    }
    if (const GgufValue* f = find("qwen2.rope.scaling.factor")) {
        if (f->kind != GgufValue::F32 || std::fabs(f->f32 - 1.0F) > 1.0e-6F) {
            fail(Status::FormatError, "native Qwen2 does not support scaled RoPE factors");
        }
    }
    ModelParams p;
    p.n_layer = req_u32("qwen2.block_count");
    p.n_embd = req_u32("qwen2.embedding_length");
    p.n_ff = req_u32("qwen2.feed_forward_length");
    p.n_head = req_u32("qwen2.attention.head_count");
    p.n_head_kv = req_u32("qwen2.attention.head_count_kv");
    p.n_ctx = req_u32("qwen2.context_length");
    p.head_dim = p.n_head ? p.n_embd / p.n_head : 0;
    uint32_t rope_dims = p.head_dim;
    if (const GgufValue* v = find("qwen2.rope.dimension_count")) {
        if (v->kind != GgufValue::U32) fail(Status::FormatError, "GGUF metadata key is not uint32: qwen2.rope.dimension_count");
        rope_dims = v->u32;
    }
    p.rope_base = req_f32("qwen2.rope.freq_base");
    p.rms_eps = req_f32("qwen2.attention.layer_norm_rms_epsilon");
    if (p.n_layer == 0 || p.n_embd == 0 || p.n_ff == 0 || p.n_head == 0 || p.n_head_kv == 0 || p.n_ctx == 0) {
        fail(Status::FormatError, "Qwen2 metadata dimensions must be positive");
    }
    if (p.n_embd % p.n_head != 0 || p.n_head % p.n_head_kv != 0) {
        fail(Status::FormatError, "Qwen2 attention dimensions are inconsistent");
    }
    if (rope_dims != p.head_dim || p.rms_eps <= 0.0F || p.rope_base <= 0.0F) {
        fail(Status::FormatError, "Qwen2 RoPE or RMS metadata is unsupported");
    }
    return p;
}

std::unique_ptr<HostModel> HostModel::open_package(const std::string& dir, const StagePlan& plan) {
    auto m = std::unique_ptr<HostModel>(new HostModel());
    m->package_ = Package::open(dir, plan);
    m->params_ = parse_qwen2_params(m->package_->gguf_metadata(), m->package_->gguf_metadata_size());
    m->tensors_ = m->package_->tensors();
    m->layer_start_ = m->package_->stats().layer_start;
    m->layer_end_ = m->package_->stats().layer_end;
    m->total_weight_bytes_ = m->package_->stats().total_weight_bytes;
    m->total_tensor_count_ = m->package_->stats().total_tensor_count;
    m->source_sha256_ = hex(m->package_->source_sha256().data(), 32);
    if (m->package_->stats().layer_count != m->params_.n_layer) {
        fail(Status::FormatError, "package layer count does not match qwen2.block_count");
    }
    m->finalize();
    return m;
}

std::unique_ptr<HostModel> HostModel::open_gguf(const std::string& path) {
    auto m = std::unique_ptr<HostModel>(new HostModel());
    m->gguf_file_ = MappedFile::open(path);
    const uint8_t* data = m->gguf_file_->data();
    const uint64_t size = m->gguf_file_->size();
    m->params_ = parse_qwen2_params(data, size_t(size));
    const GgufLayout layout = parse_gguf_layout(data, size_t(size));
    if (layout.data_offset > size) fail(Status::FormatError, "GGUF data section starts past end of file");
    m->gguf_data_offset_ = layout.data_offset;
    for (const GgufTensorInfo& t : layout.tensors) {
        TensorView v;
        v.name = t.name;
        v.type = jfm_type_from_ggml(t.type);
        if (v.type == UINT32_MAX) fail(Status::FormatError, "unsupported GGUF tensor type for " + t.name);
        v.rank = t.rank;
        uint64_t rows = 1;
        for (uint32_t d = 0; d < 4; ++d) {
            v.shape[d] = d < t.rank ? t.shape[d] : 1;
            if (v.shape[d] == 0) fail(Status::FormatError, "tensor has an invalid shape: " + t.name);
            if (d > 0) rows *= v.shape[d];
        }
        uint32_t be = 0, bb = 0;
        if (!type_layout(v.type, &be, &bb) || v.shape[0] % be != 0) {
            fail(Status::FormatError, "tensor rows are not whole blocks: " + t.name);
        }
        v.size = row_bytes(v.type, v.shape[0]) * rows;
        if (t.offset % layout.alignment != 0 || t.offset > size - layout.data_offset ||
            v.size > size - layout.data_offset - t.offset) {
            fail(Status::FormatError, "tensor exceeds the source GGUF: " + t.name);
        }
        v.data = data + layout.data_offset + t.offset;
        if (t.name.rfind("blk.", 0) == 0) {
            const uint32_t layer = uint32_t(std::stoul(t.name.substr(4, t.name.find('.', 4) - 4)));
            if (layer >= m->params_.n_layer) fail(Status::FormatError, "tensor block exceeds model block count: " + t.name);
            v.layer = int32_t(layer);
        }
        m->tensors_.push_back(v);
    }
    if (!m->find("output.weight")) {
        fail(Status::FormatError, "tied output embeddings are not supported by JFM v2; output.weight is required");
    }
    m->gguf_sha_ = sha256(data, size_t(size));
    m->source_sha256_ = hex(m->gguf_sha_.data(), 32);
    m->layer_start_ = 0;
    m->layer_end_ = m->params_.n_layer;
    m->finalize();
    return m;
}

std::unique_ptr<HostModel> HostModel::build(const ModelParams& params) {
    auto m = std::unique_ptr<HostModel>(new HostModel());
    m->params_ = params;
    if (m->params_.n_head) m->params_.head_dim = params.n_embd / params.n_head;
    m->layer_start_ = 0;
    m->layer_end_ = params.n_layer;
    return m;
}

std::unique_ptr<HostModel> HostModel::slice(uint32_t start, uint32_t end) const {
    if (start >= end || start < layer_start_ || end > layer_end_) {
        fail(Status::InvalidArgument, "native Qwen2 layer range is invalid");
    }
    auto m = build(params_);
    m->layer_start_ = start;
    m->layer_end_ = end;
    for (const TensorView& t : tensors_) {
        const bool keep = t.layer >= 0 ? static_cast<uint32_t>(t.layer) >= start && static_cast<uint32_t>(t.layer) < end
                          : t.name == "token_embd.weight" ? start == 0
                                                          : end == params_.n_layer;
        if (keep) m->add_tensor(t.name, t.type, t.rank, t.shape, t.data, t.size);
    }
    m->source_sha256_ = source_sha256_;
    m->keep_digest_ = true;
    m->total_weight_bytes_ = total_weight_bytes();
    m->total_tensor_count_ = total_tensor_count();
    m->finalize();
    return m;
}

void HostModel::add_tensor(const std::string& name, uint32_t type, uint32_t rank, const uint64_t* shape,
                           const void* data, uint64_t size) {
    if (package_) fail(Status::InvalidArgument, "cannot add tensors to a package-backed model");
    if (rank == 0 || rank > 4) fail(Status::InvalidArgument, "tensor rank must be 1..4: " + name);
    TensorView v;
    v.name = name;
    v.type = type;
    v.rank = rank;
    uint64_t rows = 1;
    for (uint32_t d = 0; d < 4; ++d) {
        v.shape[d] = d < rank ? shape[d] : 1;
        if (d > 0) rows *= v.shape[d];
    }
    if (row_bytes(type, v.shape[0]) * rows != size) fail(Status::InvalidArgument, "tensor byte size does not match its shape: " + name);
    if (name.rfind("blk.", 0) == 0) v.layer = std::stoi(name.substr(4, name.find('.', 4) - 4));
    owned_.emplace_back(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + size);
    v.data = owned_.back().data();
    v.size = size;
    tensors_.push_back(v);
}

const TensorView* HostModel::find(const std::string& name) const {
    for (const TensorView& t : tensors_) if (t.name == name) return &t;
    return nullptr;
}

const TensorView& HostModel::require(const std::string& name) const {
    const TensorView* t = find(name);
    if (!t) fail(Status::NotFound, "native Qwen2 tensor is missing: " + name);
    return *t;
}

uint64_t HostModel::weight_bytes() const {
    uint64_t b = 0;
    for (const TensorView& t : tensors_) b += t.size;
    return b;
}

void HostModel::finalize() {
    std::sort(tensors_.begin(), tensors_.end(), [](const TensorView& a, const TensorView& b) { return a.name < b.name; });
    for (size_t i = 1; i < tensors_.size(); ++i) {
        if (tensors_[i - 1].name == tensors_[i].name) fail(Status::FormatError, "duplicate tensor name " + tensors_[i].name);
    }
    const ModelParams& p = params_;
    const uint64_t H = p.n_embd, kv = uint64_t(p.head_dim) * p.n_head_kv, F = p.n_ff;
    auto shape = [&](const std::string& name, std::initializer_list<uint64_t> expected) {
        const TensorView& t = require(name);
        if (t.rank != expected.size()) fail(Status::FormatError, "native Qwen2 tensor has wrong rank: " + name);
        size_t d = 0;
        for (uint64_t e : expected) {
            if (t.shape[d++] != e) fail(Status::FormatError, "native Qwen2 tensor has wrong shape: " + name);
        }
    };
    const bool first = layer_start_ == 0, last = layer_end_ == p.n_layer;
    if (layer_start_ >= layer_end_ || layer_end_ > p.n_layer) fail(Status::InvalidArgument, "native Qwen2 layer range is invalid");
    // vocabulary from the embedding or the output head (TensorStore::vocabulary_size,
    // tensor_store.cpp:211-220); a middle stage holds neither and has none
    const TensorView* vocab_src = find(first ? "token_embd.weight" : "output.weight");
    if (!vocab_src) vocab_src = find("output.weight");
    if ((first || last) && (!vocab_src || vocab_src->rank != 2)) {
        fail(Status::FormatError, "native Qwen2 vocabulary tensor is missing");
    }
    params_.n_vocab = vocab_src && vocab_src->rank == 2 ? uint32_t(vocab_src->shape[1]) : 0;
    const uint64_t V = params_.n_vocab;
    if (first) shape("token_embd.weight", {H, V});
    if (last) {
        shape("output_norm.weight", {H});
        shape("output.weight", {H, V});
        if (find("output.bias")) shape("output.bias", {V});
    }
    for (uint32_t l = layer_start_; l < layer_end_; ++l) {
        const std::string pre = "blk." + std::to_string(l) + ".";
        shape(pre + "attn_norm.weight", {H});
        shape(pre + "attn_q.weight", {H, H});
        shape(pre + "attn_q.bias", {H});
        shape(pre + "attn_k.weight", {H, kv});
        shape(pre + "attn_k.bias", {kv});
        shape(pre + "attn_v.weight", {H, kv});
        shape(pre + "attn_v.bias", {kv});
        shape(pre + "attn_output.weight", {H, H});
        shape(pre + "ffn_norm.weight", {H});
        shape(pre + "ffn_gate.weight", {H, F});
        shape(pre + "ffn_up.weight", {H, F});
        shape(pre + "ffn_down.weight", {F, H});
    }
    if (!package_ && !gguf_file_ && !keep_digest_) {
        source_sha256_ = hex(source_digest(gguf_header(), blobs()).first.data(), 32);
    }
}

std::vector<uint8_t> HostModel::gguf_header() const {
    if (gguf_file_) return std::vector<uint8_t>(gguf_file_->data(), gguf_file_->data() + gguf_data_offset_);
    if (package_) {
        return std::vector<uint8_t>(package_->gguf_metadata(), package_->gguf_metadata() + package_->gguf_metadata_size());
    }
    const ModelParams& p = params_;
    auto u32 = [](uint32_t v) { GgufValue g; g.kind = GgufValue::U32; g.u32 = v; return g; };
    auto f32 = [](float v) { GgufValue g; g.kind = GgufValue::F32; g.f32 = v; return g; };
    GgufValue arch;
    arch.kind = GgufValue::Str;
    arch.str = "qwen2";
    std::vector<std::pair<std::string, GgufValue>> kv = {
        {"general.architecture", arch},
        {"qwen2.block_count", u32(p.n_layer)},
        {"qwen2.context_length", u32(p.n_ctx)},
        {"qwen2.embedding_length", u32(p.n_embd)},
        {"qwen2.feed_forward_length", u32(p.n_ff)},
        {"qwen2.attention.head_count", u32(p.n_head)},
        {"qwen2.attention.head_count_kv", u32(p.n_head_kv)},
        {"qwen2.rope.dimension_count", u32(p.head_dim)},
        {"qwen2.rope.freq_base", f32(p.rope_base)},
        {"qwen2.attention.layer_norm_rms_epsilon", f32(p.rms_eps)},
    };
    std::vector<GgufTensorInfo> infos;
    uint64_t off = 0;
    for (const TensorView& t : tensors_) {
        GgufTensorInfo i;
        i.name = t.name;
        i.type = t.type;
        i.rank = t.rank;
        std::copy(t.shape, t.shape + 4, i.shape);
        off = (off + 31) / 32 * 32;
        i.offset = off;
        off += t.size;
        infos.push_back(i);
    }
    return write_gguf_header(kv, infos);
}

std::vector<TensorBlob> HostModel::blobs() const {
    std::vector<TensorBlob> blobs;
    for (const TensorView& t : tensors_) {
        TensorBlob b;
        b.name = t.name;
        b.type = t.type;
        b.rank = t.rank;
        std::copy(t.shape, t.shape + 4, b.shape);
        b.data = t.data;
        b.size = t.size;
        blobs.push_back(b);
    }
    return blobs;
}

void HostModel::write_package(const std::string& dir) const {
    if (layer_start_ != 0 || layer_end_ != params_.n_layer) fail(Status::InvalidArgument, "only a full model can be written as a package");
    if (gguf_file_) {
        // the manifest records the imported file itself
        const std::pair<std::array<uint8_t, 32>, uint64_t> source{gguf_sha_, gguf_file_->size()};
        jfh::write_package(dir, params_.n_layer, gguf_header(), blobs(), &source);
        return;
    }
    jfh::write_package(dir, params_.n_layer, gguf_header(), blobs());
}

std::unique_ptr<HostModel> HostModel::synthesize(const SynthSpec& spec) {
    ModelParams p = spec.params;
    if (p.n_head == 0 || p.n_embd % p.n_head != 0) fail(Status::InvalidArgument, "synthetic model heads do not divide the embedding");
    p.head_dim = p.n_embd / p.n_head;
    auto m = build(p);
    m->params_.n_vocab = p.n_vocab;
    const uint64_t H = p.n_embd, kv = uint64_t(p.head_dim) * p.n_head_kv, F = p.n_ff, V = p.n_vocab;
    if (spec.tied_output && spec.type_embd != spec.type_output) {
        fail(Status::InvalidArgument, "tied output requires the embedding and output types to match");
    }
    auto gen = [&](const std::string& name, uint32_t type, uint64_t cols, uint64_t rows, int kind) {
        // kind 0: N(0, stddev); 1: constant 1.0
        const size_t rb = row_bytes(type, cols);
        std::vector<uint8_t> bytes(rb * rows);
        const uint64_t key = spec.seed ^ fnv1a(name);
        parallel_rows(int64_t(rows), spec.threads, [&](int64_t a, int64_t b) {
            std::vector<float> row(cols + 1);
            for (int64_t r = a; r < b; ++r) {
                if (kind == 1) {
                    std::fill(row.begin(), row.end(), 1.0F);
                } else {
                    const uint64_t base = uint64_t(r) * cols;  // cols is even for every tensor here
                    for (uint64_t c = 0; c < cols; c += 2) {
                        float x0, x1;
                        normal_pair(key, (base + c) / 2, &x0, &x1);
                        row[c] = spec.stddev * x0;
                        row[c + 1] = spec.stddev * x1;
                    }
                }
                quantize_row(type, row.data(), bytes.data() + size_t(r) * rb, int64_t(cols));
            }
        });
        const uint64_t shape[2] = {cols, rows};
        m->add_tensor(name, type, rows == 1 ? 1 : 2, shape, bytes.data(), bytes.size());
    };
    gen("token_embd.weight", spec.type_embd, H, V, 0);
    for (uint32_t l = 0; l < p.n_layer; ++l) {
        const std::string pre = "blk." + std::to_string(l) + ".";
        gen(pre + "attn_norm.weight", kF32, H, 1, 1);
        gen(pre + "attn_q.weight", spec.type_linear, H, H, 0);
        gen(pre + "attn_q.bias", kF32, H, 1, 0);
        gen(pre + "attn_k.weight", spec.type_linear, H, kv, 0);
        gen(pre + "attn_k.bias", kF32, kv, 1, 0);
        gen(pre + "attn_v.weight", spec.type_linear, H, kv, 0);
        gen(pre + "attn_v.bias", kF32, kv, 1, 0);
        gen(pre + "attn_output.weight", spec.type_linear, H, H, 0);
        gen(pre + "ffn_norm.weight", kF32, H, 1, 1);
        gen(pre + "ffn_gate.weight", spec.type_linear, H, F, 0);
        gen(pre + "ffn_up.weight", spec.type_linear, H, F, 0);
        gen(pre + "ffn_down.weight", spec.type_linear, F, H, 0);
    }
    gen("output_norm.weight", kF32, H, 1, 1);
    if (spec.tied_output) {
        const TensorView& e = m->require("token_embd.weight");
        const std::vector<uint8_t> copy(e.data, e.data + e.size);
        const uint64_t shape[2] = {H, V};
        m->add_tensor("output.weight", spec.type_output, 2, shape, copy.data(), copy.size());
    } else {
        gen("output.weight", spec.type_output, H, V, 0);
    }
    if (spec.output_bias) gen("output.bias", kF32, V, 1, 0);
    m->finalize();
    return m;
}

}  // namespace jfh
