// HIP Qwen2 stage engine: device-resident weights, sessions owning F16 KV
// caches, and batched forward steps (prefill chunks, decode, draft verify).
//
// Replaces the reference's Qwen2Architecture/Qwen2Session/ForwardGraph
// (runtime/engines/native/src/qwen2_architecture.cpp:120-1212) and
// TensorStore (tensor_store.cpp:57-196) for one GPU holding a model's layers
// or one pipeline stage's layer range (LayerRange, model_architecture.hpp:15-21).
#pragma once

#include "jfh_kernels.hpp"
#include "jfh_model.hpp"

#include <hip/hip_runtime_api.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace jfh {

// Builds one 16-row x 256-value device tile of a quantized type from the 16
// rows' GGML blocks (nullptr rows are zero); tile holds gpu::tile_bytes(type).
void build_tile(uint32_t type, const uint8_t* const* blocks, uint8_t* tile);

struct EngineOptions {
    int device = 0;
    bool use_graphs = true;
};

class Engine;

// KV-cache owner; position bookkeeping follows Qwen2Session
// (qwen2_architecture.cpp:800-823, 1040-1054).
// Host-side breakdown of a prefill (PrefillMetrics, native_inference.hpp:71-78):
// graph capture and instantiation of step shapes met for the first time
// (planning), building and uploading the step descriptors (host input), the
// device time of the step graphs (compute, HIP events around each launch) and
// of the result copies (output read).
struct PrefillMetrics {
    bool plan_reused = true;         // every prefill step shape's graph existed already
    bool attention_matrix_cores = false;  // attention on MFMA (head dim 64 or 128)
    double planning_ms = 0.0;
    double allocation_ms = 0.0;      // the session's KV cache allocation and clearing
    double host_input_ms = 0.0;
    double compute_ms = 0.0;
    double output_read_ms = 0.0;
    uint64_t host_input_bytes = 0;   // step descriptors and activation rows uploaded
    uint32_t steps = 0;              // prefill chunks
};

// Device buffers a generation uses (ExecutionBufferMetrics, native_inference.hpp:80-85).
struct BufferMetrics {
    uint64_t kv_cache_bytes = 0;          // the session's F16 K/V cache
    uint64_t prefill_scratch_bytes = 0;   // workspace rows of one prefill chunk
    uint64_t decode_scratch_bytes = 0;    // workspace of one decode row
    uint64_t prefill_host_input_bytes = 0;
};

class Session {
public:
    ~Session();
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    uint32_t capacity() const { return capacity_; }
    uint32_t position() const { return position_; }
    uint32_t prefill_position() const { return prefill_position_; }
    void rollback(uint32_t n);
    uint64_t kv_bytes() const { return kv_bytes_; }
    // Metrics of the session's prefill (zero before it).
    const PrefillMetrics& prefill_metrics() const { return prefill_metrics_; }

private:
    friend class Engine;
    Session(Engine* engine, uint32_t capacity);

    Engine* engine_;
    uint32_t capacity_;
    uint32_t stride_;  // allocated positions per (layer, kv head): capacity rounded up to 16
    uint32_t position_ = 0;
    uint32_t prefill_position_ = 0;
    uint16_t* k_ = nullptr;  // [resident layer][kv head][stride][head_dim]
    uint16_t* v_ = nullptr;  // [resident layer][kv head][stride / 16][head_dim][16] (16-position tiles)
    uint64_t kv_bytes_ = 0;
    PrefillMetrics prefill_metrics_;
};

// One sequence's share of a batched step.
struct SeqStep {
    Session* session = nullptr;
    const int32_t* tokens = nullptr;     // first stage: token ids, or
    const float* activations = nullptr;  // later stages: f32 [n][n_embd] input rows
    uint32_t n = 0;
    // 0: no logits, 1: last row, 2: every row (draft verify)
    int logits = 1;
};

// Per-kernel device time of one step, measured with HIP events attached to
// the kernel dispatches of an un-graphed step (averaged over iterations).
struct KernelStat {
    std::string label;
    double launches = 0.0;   // launches per step
    double total_ms = 0.0;   // device ms per step
    double bytes = 0.0;      // algorithmic HBM bytes per step
};

class Engine {
public:
    Engine(const HostModel& model, const EngineOptions& options);
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    const ModelParams& params() const { return params_; }
    uint64_t weight_bytes() const { return weight_bytes_; }
    // The resident layer range [layer_start, layer_end): the first stage
    // embeds token ids, the last one holds the output head.
    uint32_t layer_start() const { return layer_start_; }
    uint32_t layer_end() const { return layer_end_; }
    uint32_t resident_layers() const { return layer_end_ - layer_start_; }
    bool first_stage() const { return layer_start_ == 0; }
    bool last_stage() const { return layer_end_ == params_.n_layer; }
    // Fails unless this engine holds every layer (full-model entry points).
    void require_full_model() const;
    hipStream_t stream() const { return stream_; }
    const std::string& device_name() const { return device_name_; }

    std::unique_ptr<Session> create_session(uint32_t capacity);

    // End-of-generation ids (at most gpu::kMaxEndTokens, each inside the
    // vocabulary): a verify row's draft token is accepted only while the
    // greedy id it is compared with is none of them, as the reference runner
    // stops acceptance at an end token. Replaces the previous set; empty by
    // default.
    void set_end_tokens(const int32_t* ids, uint32_t n);
    std::vector<int32_t> end_tokens() const;

    // Runs token rows for several sessions in one pass. Positions advance by
    // each sequence's row count. out_tokens receives one greedy id per logits
    // row (sequence order); accepted (optional) one accepted-draft count per
    // sequence; logits (optional) n_logits_rows x vocab floats. A stage
    // that is not the last one computes no logits: act_out receives the
    // residual-stream rows after its last layer, f32 [rows][n_embd].
    // metrics (optional) accumulates the step's host and device times.
    void forward(const std::vector<SeqStep>& steps, int32_t* out_tokens, int32_t* accepted, float* logits,
                 float* act_out = nullptr, PrefillMetrics* metrics = nullptr);

    // Prefill of arbitrary length: runs the prompt in chunks and returns the
    // greedy token of the last row (and its logits if requested).
    int32_t prefill(Session& s, const int32_t* tokens, uint32_t n, float* logits);

    // One pipeline stage's prefill (n rows at position 0) or decode (one row)
    // (Qwen2Session::prefill_stage_* / decode_stage_*,
    // qwen2_architecture.cpp:909-947, 977-1027): token ids into the first
    // stage, activations into the others; the last stage returns the greedy
    // id of the last row, the others write every row's activations to
    // act_out and return -1. The last stage also writes the last row's
    // logits to `logits` when it is set.
    int32_t stage_prefill(Session& s, const int32_t* tokens, const float* activations, uint32_t n, float* act_out,
                          float* logits = nullptr);
    int32_t stage_decode(Session& s, const int32_t* token, const float* activation, float* act_out,
                         float* logits = nullptr);

    // Parity entry points: dequantize rows of a device tensor; multiply a
    // device matrix with host activations through the same kernels.
    void dequantize(const std::string& name, uint32_t row0, uint32_t n_rows, float* out_host);
    void matmul(const std::string& name, const float* x_host, uint32_t n_tok, float* y_host);
    // The same matmul on device rows (x_dev [n_tok][cols], y_dev [n_tok][rows])
    // with its staging in the GPU's static scratch: no device allocation. It
    // runs after the work enqueued on `after` (the caller's stream) and
    // returns with y_dev written.
    void matmul_noalloc(const std::string& name, const float* x_dev, uint32_t n_tok, float* y_dev, hipStream_t after);

    // Runs the step `iterations` times without graphs, timing every kernel
    // launch; sessions are restored to their starting positions.
    std::vector<KernelStat> profile(const std::vector<SeqStep>& steps, uint32_t iterations);

    // Parity entry points: K/V rows [0, n) of one layer out of a session
    // ([kv_head][n][head_dim] f16), and of every layer ([layer][kv_head][n]
    // [head_dim]) into one, which then stands at position n as after a
    // prefill of n tokens.
    void read_kv(const Session& s, uint32_t layer, uint32_t n, uint16_t* k, uint16_t* v);
    void import_kv(Session& s, uint32_t n, const uint16_t* k, const uint16_t* v);

    uint32_t max_prefill_chunk() const { return prefill_chunk_; }

    // Workspace bytes one token row of a step uses (residual, queries,
    // attention and SwiGLU outputs, their int8 copies, attention partials).
    uint64_t scratch_bytes_per_row() const;
    // Buffer metrics of a session of `capacity` positions whose prefill ran
    // `prompt_tokens` tokens with the given metrics.
    BufferMetrics buffer_metrics(uint32_t capacity, uint32_t prompt_tokens, const PrefillMetrics& prefill) const;
    // The prefill metrics of the last prefill the calling thread ran on any
    // engine (a generation runner's executor closes its session when done).
    static PrefillMetrics last_prefill_metrics();

private:
    friend class Session;
    struct DeviceTensor {
        gpu::DMat mat;
        uint64_t bytes = 0;  // encoded GGML bytes of the rows it holds
    };
    // Where a model tensor's rows live: rows of a (possibly fused) device matrix.
    struct TensorRef {
        const DeviceTensor* dev = nullptr;
        uint32_t rows = 0;     // rows of the model tensor
        uint32_t offset = 0;   // first device row
        uint32_t kind = 0;     // 0 contiguous, 1 RoPE pair order per head, 2 GLU gate rows, 3 GLU up rows
        uint32_t head_dim = 0;
    };
    struct RowSource {
        const TensorView* tensor;
        uint32_t row;
    };
    struct Layer {
        const DeviceTensor *qkv, *o, *gate_up, *down;
        const float *attn_norm, *ffn_norm;
    };

    static uint32_t device_row(const TensorRef& r, uint32_t row);
    static bool matmul_staged(const gpu::DMat& m, uint32_t n_tok);
    void run_matmul(const gpu::DMat& m, const float* x, uint32_t n_tok, float* y_full, const gpu::Act8& xq);
    const DeviceTensor& upload_rows(const std::string& key, uint32_t type, uint64_t cols,
                                    const std::vector<RowSource>& rows, const float* bias);
    const DeviceTensor& upload_single(const TensorView& t);
    void add_ref(const TensorView& t, const DeviceTensor& dev, uint32_t offset, uint32_t kind);
    const TensorRef& find_ref(const std::string& name) const;
    const float* upload_f32(const TensorView& t);
    void ensure_capacity(uint32_t capacity);
    void record(int32_t n_rows, int32_t max_len, int32_t n_seq, int32_t n_out, bool store_logits);
    template <typename F>
    void timed(const std::string& label, double bytes, F&& fn);

    struct ProfEvent {
        std::string label;
        double bytes = 0.0;
        hipEvent_t begin = nullptr;
        hipEvent_t end = nullptr;
    };
    std::vector<ProfEvent>* prof_ = nullptr;
    hipEvent_t ev_begin_ = nullptr, ev_compute_ = nullptr, ev_output_ = nullptr;  // prefill step timing
    hipEvent_t ev_order_ = nullptr;  // orders the allocation-free matmul after the caller's stream
    double attn_kv_bytes_ = 0.0;  // K/V bytes one layer's attention reads in the step being recorded
    void* device_alloc(size_t bytes);

    ModelParams params_;
    EngineOptions options_;
    std::string device_name_;
    hipStream_t stream_ = nullptr;
    std::map<std::string, DeviceTensor> matrices_;
    std::map<std::string, TensorRef> refs_;
    std::vector<void*> allocations_;
    std::vector<Layer> layers_;
    uint32_t layer_start_ = 0, layer_end_ = 0;
    const DeviceTensor* embd_ = nullptr;    // first stage only
    const DeviceTensor* output_ = nullptr;  // last stage only
    const float* output_norm_ = nullptr;
    uint64_t weight_bytes_ = 0;
    uint32_t prefill_chunk_ = 8;

    // workspace
    float* h_ = nullptr;       // residual stream [row][n_embd]
    float* q_ = nullptr;       // roped queries [row][n_embd]
    float* attn_ = nullptr;    // attention output [row][n_embd]
    float* ffn_ = nullptr;     // SwiGLU output [row][n_ff]
    float* logits_ = nullptr;
    unsigned long long* best_ = nullptr;
    gpu::StepDev* step_dev_ = nullptr;
    gpu::StepOut* out_dev_ = nullptr;
    gpu::StepDev* step_host_ = nullptr;  // pinned
    gpu::StepOut* out_host_ = nullptr;   // pinned
    float* partial_ = nullptr;
    float* rope_ = nullptr;
    uint32_t capacity_max_ = 0;
    int32_t splits_ = 0;
    int32_t attn_capacity_ = 0;  // the positions the rope table and attention splits are sized for
    // int8 staging copies of the attention output and the SwiGLU output
    // (set when the consuming matrix is quantized)
    gpu::Act8 xq_attn_;
    gpu::Act8 xq_ffn_;
    // normalized int8 rows of wide steps (the QKV and gate/up inputs)
    gpu::Act8 xq_norm_;

    // captured step graphs keyed by (rows, seqs, outs, store_logits)
    std::map<uint64_t, hipGraphExec_t> graphs_;
    std::vector<int32_t> end_tokens_;
    mutable std::mutex mutex_;
};

}  // namespace jfh
