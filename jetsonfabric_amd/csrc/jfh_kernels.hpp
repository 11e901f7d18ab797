// Host-visible launch interface of the gfx950 kernels that implement the
// Qwen2 stage forward (runtime/engines/native/src/qwen2_architecture.cpp:522-598).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace jfh::gpu {

constexpr int kMaxRows = 64;   // token rows of one step (sum over sequences)
constexpr int kMaxSeq = 16;    // sequences of one batched step
constexpr int kActBlock = 256; // activation quantization block (values)

// A weight matrix in device memory. Quantized types are stored as a 16-byte
// aligned main plane [rows][blocks][main_block_bytes] plus an aux plane
// [rows][blocks][aux_block_bytes] holding the f16 scales that do not fit the
// alignment: Q4_K main 144 / aux 0 (GGML bytes verbatim), Q6_K main 208
// (ql|qh|scales) / aux 2 (d), Q8_0 main 32 (qs) / aux 2 (d), Q2_K main 80
// (scales|qs) / aux 4 (d, dmin). F32/F16 are verbatim with no aux plane.
struct DMat {
    const uint8_t* main = nullptr;
    const uint8_t* aux = nullptr;
    const float* bias = nullptr;  // optional f32 [rows]
    uint32_t type = 0;
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t main_row_bytes = 0;
    uint32_t aux_row_bytes = 0;
};

// Per-sequence cache description for a step.
struct SeqDev {
    uint16_t* k;     // [layers][kv_heads][capacity][head_dim] f16
    uint16_t* v;
    int32_t capacity;
    int32_t row0;    // first step row of the sequence
    int32_t len;     // rows of the sequence in this step
    int32_t pos0;    // position of its first row
};

// Step description in device memory, rewritten before every launch sequence.
struct StepDev {
    int32_t n_rows;
    int32_t n_seq;
    int32_t n_out;                 // rows that produce logits
    int32_t pad;
    int32_t token[kMaxRows];
    int32_t pos[kMaxRows];
    int32_t seq[kMaxRows];
    int32_t out_row[kMaxRows];     // step row of each logits row
    int32_t draft[kMaxRows];       // token the logits row is compared with (-1: none)
    SeqDev seqs[kMaxSeq];
};

// Result block copied back to the host after a step.
struct StepOut {
    int32_t token[kMaxRows];       // argmax of each logits row (first max)
    int32_t accepted[kMaxSeq];     // accepted draft prefix per sequence
};

// Activation buffers for quantized matmuls: int8 values, one f32 scale per
// 256 values and the int16 sum of every 16 values; plus the float copy used
// by F32/F16 weights. Row stride is `stride` values.
struct Act {
    int8_t* q;
    float* d;
    int16_t* s;
    float* f;
    int32_t stride;
};

enum GemvMode : int32_t { kStore = 0, kAdd = 1, kSwiGLU = 2, kLogits = 3 };

struct GemvArgs {
    DMat mat[3];
    int32_t n_mat = 1;
    int32_t mode = kStore;
    int32_t n_tok = 1;
    const Act* act = nullptr;        // host copy of the act descriptor (by value below)
    Act x{};
    float* y = nullptr;               // output [tok][y_stride]
    int32_t y_stride = 0;
    unsigned long long* best = nullptr;  // kLogits: packed (value, -index) per token
    int32_t store_logits = 0;
};

// Launchers (all asynchronous on `stream`).
void launch_embed(const DMat& table, const StepDev* step, float* h, int32_t n_rows, int32_t H,
                  unsigned long long* best, int32_t n_best, hipStream_t stream);
void launch_norm_quant(const float* h, int32_t h_stride, const float* gain, float eps, int32_t H,
                       const StepDev* step, int32_t select_out, int32_t n_rows, bool quantize, Act x,
                       hipStream_t stream);
void launch_quant(const float* src, int32_t src_stride, int32_t K, int32_t n_rows, bool quantize, Act x,
                  hipStream_t stream);
void launch_gemv(const GemvArgs& a, hipStream_t stream);
void launch_rope_kv(const float* qkv, int32_t n_rows, int32_t n_head, int32_t n_head_kv, int32_t head_dim,
                    const float* rope, const StepDev* step, int32_t layer, float* qout, hipStream_t stream);
// Split-K flash attention writing out.f rows, then the int8 quantization of
// those rows. `splits` is fixed per capacity (attention_splits); `counters`
// holds kMaxSeq * n_head_kv zero-initialized ints that the kernel resets.
void launch_attention(const float* q, const StepDev* step, int32_t n_rows, int32_t max_len, int32_t n_seq,
                      int32_t layer, int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits,
                      float* partial, int32_t* counters, Act out, hipStream_t stream);
int32_t attention_splits(int32_t capacity);
void launch_finish(const unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out,
                   hipStream_t stream);
void launch_dequant_rows(const DMat& m, int32_t row0, int32_t n_rows, float* out, hipStream_t stream);

// Bytes of LDS the gemv kernel needs for `n_tok` tokens (for validation).
int32_t gemv_chunk_values(int32_t n_tok, int32_t K);

}  // namespace jfh::gpu
