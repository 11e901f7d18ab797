// Host-visible launch interface of the gfx950 kernels that implement the
// Qwen2 stage forward (runtime/engines/native/src/qwen2_architecture.cpp:522-598).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace jfh::gpu {

constexpr int kMaxRows = 64;   // token rows of one step (sum over sequences)
constexpr int kMaxSeq = 16;    // sequences of one batched step
constexpr int kActBlock = 256; // activation quantization block (values)
constexpr int kMaxAttnQGroups = 8;  // query groups of 8 rows per kv head in one step

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

enum GemvMode : int32_t {
    kStore = 0,   // y = W x + bias
    kAdd = 1,     // y += W x (residual)
    kSwiGLU = 2,  // rows interleaved [gate x kGluGroup][up x kGluGroup]: y = silu(gate) * up
    kLogits = 3,  // y = W x + bias (optional store) and the greedy argmax per token
    kQKV = 4,     // fused q|k|v rows: bias, NEOX RoPE of q and k, q to qkv.q, k and v to the f16 cache
};

// Gate/up rows are interleaved in groups of this many rows per matrix.
constexpr int kGluGroup = 8;

// Float activation rows feeding a matmul. With `gain` set the rows are
// RMS-normalized over their full length and multiplied by the gain first;
// with `gather` set token t reads row gather[t].
struct XIn {
    const float* x = nullptr;
    int32_t stride = 0;
    const int32_t* gather = nullptr;
    const float* gain = nullptr;
    float eps = 0.0F;
};

// kQKV epilogue: q/k rows of every head are stored pair-interleaved
// (physical row 2i = head row i, 2i + 1 = head row i + head_dim/2) so one
// work-group holds both halves of every rotated pair.
struct QkvOut {
    const StepDev* step = nullptr;
    const float* rope = nullptr;  // [position][head_dim/2] (cos, sin)
    float* q = nullptr;           // [token][n_head * head_dim]
    int32_t row0 = 0;             // step row of the first token
    int32_t layer = 0;
    int32_t n_head = 0;
    int32_t n_head_kv = 0;
    int32_t head_dim = 0;
};

struct GemvArgs {
    DMat mat;
    int32_t mode = kStore;
    int32_t n_tok = 1;
    XIn x;
    float* y = nullptr;               // output [tok][y_stride]
    int32_t y_stride = 0;
    unsigned long long* best = nullptr;  // kLogits: packed (value, -index) per token
    int32_t store_logits = 0;
    QkvOut qkv;
};

// Launchers (all asynchronous on `stream`).
void launch_embed(const DMat& table, const StepDev* step, float* h, int32_t n_rows, int32_t H,
                  unsigned long long* best, int32_t n_best, hipStream_t stream);
// Matmul of up to kMaxRows token rows (in groups of 8) against one matrix.
void launch_gemv(const GemvArgs& a, hipStream_t stream);
// Split-K causal GQA flash attention over the f16 caches of the step's
// sequences, writing float rows out[row][n_head * head_dim]. `splits` is
// fixed per capacity (attention_splits); `counters` holds
// kMaxSeq * n_head_kv * kMaxAttnQGroups zero-initialized ints that the kernel
// leaves zero.
void launch_attention(const float* q, const StepDev* step, int32_t max_len, int32_t n_seq, int32_t layer,
                      int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits, float* partial,
                      int32_t* counters, float* out, hipStream_t stream);
int32_t attention_splits(int32_t capacity);
// Floats of the attention split scratch for `rows` token rows.
size_t attention_partial_floats(int32_t rows, int32_t n_head, int32_t head_dim, int32_t splits);
void launch_finish(const unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out,
                   hipStream_t stream);
void launch_dequant_rows(const DMat& m, int32_t row0, int32_t n_rows, float* out, hipStream_t stream);

}  // namespace jfh::gpu
