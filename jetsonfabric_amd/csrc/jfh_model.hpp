// Host-resident Qwen2 model: tensors from a JFM v2 package or generated
// synthetically, plus the hyper-parameters the stage engine needs.
//
// Mirrors the reference's TensorStore + Qwen2HParams pair
// (runtime/engines/native/src/tensor_store.cpp:57-116,
//  runtime/engines/native/src/qwen2_metadata.cpp:90-125,
//  runtime/engines/native/src/qwen2_architecture.cpp:80-118).
#pragma once

#include "jfh_format.hpp"

#include <memory>
#include <string>
#include <vector>

namespace jfh {

struct ModelParams {
    uint32_t n_layer = 0;
    uint32_t n_embd = 0;
    uint32_t n_ff = 0;
    uint32_t n_head = 0;
    uint32_t n_head_kv = 0;
    uint32_t n_ctx = 0;
    uint32_t n_vocab = 0;
    uint32_t head_dim = 0;
    float rope_base = 0.0F;
    float rms_eps = 0.0F;
};

// Synthetic model recipe: every weight is N(0, stddev) from a counter-based
// generator keyed by (seed xor FNV-1a(tensor name), element index), quantized
// with this library's quantizers. Norm gains are 1.0, biases N(0, stddev) F32.
struct SynthSpec {
    ModelParams params;
    uint32_t type_linear = kQ4_K;
    uint32_t type_embd = kQ4_K;
    uint32_t type_output = kQ6_K;
    bool tied_output = false;  // output.weight = byte copy of token_embd.weight
    bool output_bias = false;
    uint64_t seed = 1234;
    float stddev = 0.02F;
    int threads = 0;  // 0 = hardware concurrency
};

class HostModel {
public:
    static std::unique_ptr<HostModel> open_package(const std::string& dir, const StagePlan& plan);
    static std::unique_ptr<HostModel> synthesize(const SynthSpec& spec);
    // A qwen2 GGUF file (memory-mapped) as a model, for writing its JFM v2
    // package (jf_model_compile.cpp:549-645): tensors of the types this
    // engine runs, output.weight required, source SHA-256 of the whole file.
    static std::unique_ptr<HostModel> open_gguf(const std::string& path);
    // Starts an empty model; tensors are added with add_tensor (bytes are copied).
    static std::unique_ptr<HostModel> build(const ModelParams& params);
    // The tensors of layers [start, end) of this model (plus the embedding
    // for a first stage and the output norm and head for a last one) as a
    // model of its own, as jf_model_open selects a package's layer range
    // (engine.c:513-757). Bytes are copied; the source digest is kept.
    std::unique_ptr<HostModel> slice(uint32_t start, uint32_t end) const;

    void add_tensor(const std::string& name, uint32_t type, uint32_t rank, const uint64_t* shape,
                    const void* data, uint64_t size);
    // Validates names and shapes (qwen2_architecture.cpp:80-118) once all tensors are present.
    void finalize();

    const ModelParams& params() const { return params_; }
    const TensorView* find(const std::string& name) const;
    const TensorView& require(const std::string& name) const;
    const std::vector<TensorView>& tensors() const { return tensors_; }
    uint32_t layer_start() const { return layer_start_; }
    uint32_t layer_end() const { return layer_end_; }
    uint64_t weight_bytes() const;
    // Weight bytes and tensors of the whole model this one selects a layer
    // range of (its package, or the model it was sliced from); equal to its
    // own otherwise (jf_model_stats::total_*, engine.h:74-83).
    uint64_t total_weight_bytes() const { return total_weight_bytes_ != 0 ? total_weight_bytes_ : weight_bytes(); }
    uint64_t total_tensor_count() const { return total_tensor_count_ != 0 ? total_tensor_count_ : tensors_.size(); }
    std::string source_sha256() const { return source_sha256_; }

    // GGUF header bytes for the model's metadata (written or as loaded).
    std::vector<uint8_t> gguf_header() const;
    // Tensors as package blobs, in model order.
    std::vector<TensorBlob> blobs() const;
    void write_package(const std::string& dir) const;

private:
    HostModel() = default;
    void index();

    ModelParams params_;
    std::unique_ptr<Package> package_;
    std::shared_ptr<const MappedFile> gguf_file_;  // imported GGUF
    uint64_t gguf_data_offset_ = 0;
    std::array<uint8_t, 32> gguf_sha_{};
    std::vector<std::vector<uint8_t>> owned_;
    std::vector<TensorView> tensors_;
    uint32_t layer_start_ = 0;
    uint32_t layer_end_ = 0;
    std::string source_sha256_;
    bool keep_digest_ = false;  // a slice keeps its source model's digest
    uint64_t total_weight_bytes_ = 0;  // 0: this model is whole
    uint64_t total_tensor_count_ = 0;
};

// Parses and validates qwen2.* GGUF keys (qwen2_metadata.cpp:90-125).
ModelParams parse_qwen2_params(const uint8_t* gguf, size_t size);

// Quantizers used for synthetic weights (any valid block is acceptable input
// to the engine; these are simple min/max fits, not GGML's search).
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);
void quantize_row(uint32_t type, const float* x, uint8_t* out, int64_t n);
size_t row_bytes(uint32_t type, uint64_t n);

}  // namespace jfh
