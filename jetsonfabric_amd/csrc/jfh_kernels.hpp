// Host-visible launch interface of the gfx950 kernels that implement the
// Qwen2 stage forward (runtime/engines/native/src/qwen2_architecture.cpp:522-598).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

namespace jfh::gpu {

// Token rows of one step (a prefill chunk is at most this long).
constexpr int kMaxRows = 256;
// Token groups of at least this many rows (int8 or RMS-normalized input) of
// the quantized formats (Q4_K, Q6_K, Q8_0, Q2_K) run as token quads on matrix
// cores.
constexpr int kQuadMinRows = 2;        // token rows of one step (sum over sequences)
// Token rows per matrix-core launch of the token-quad matmul (longer steps
// run in groups of this many rows).
constexpr int kQuadGroupRows = 16;
constexpr int kMaxSeq = 16;         // sequences of one batched step
constexpr int kActBlock = 256;      // activation quantization block of K-quant inputs (values)
constexpr int kActBlock32 = 32;     // activation block of Q8_0 inputs
constexpr int kTileRows = 16;       // rows of one weight tile
constexpr int kMaxAttnQGroups = 8;  // query groups of 8 rows per kv head in one step
constexpr int kMaxEndTokens = 16;   // end-of-generation ids the on-GPU acceptance stops at

// Bytes of one weight tile (16 rows x 256 values) of a quantized type, 0 for
// float types. The tile holds the 16 rows' GGML blocks rearranged so that
// lane l of a wave (row i = l % 16, group g = l / 16) owns row i's values
// 64 g .. 64 g + 63 and reads their codes with 16-byte loads that cover
// 1 KiB of contiguous memory per wave (chunk c of lane l at
// codes + (64 c + l) * 16):
//   Q4_K 2304: 16 headers (d, dmin, then per lane group g a 24-bit field
//              sc 2g | sc 2g+1 | m 2g | m 2g+1 at bit 24 g) | 2 chunks: GGML qs
//              bytes 32 g .. 32 g + 31 (low nibbles values 0..31, high 32..63)
//   Q6_K 3360: 16 d | 16 x 16 int8 scales | 3 chunks: 8 low-nibble dwords
//              (dword k: values 8k..8k+3 low, 8k+4..8k+7 high nibbles) and 4
//              high-bit dwords (dword m, byte e, bits 2r: value 16m + 4r + e)
//   Q8_0 4352: 16 x 8 d | 4 chunks: the int8 codes of GGML blocks 2g, 2g+1
//   Q2_K 1344: 16 (d, dmin) | 16 x 16 scale bytes | 1 chunk: dword m, byte e,
//              bits 2r: value 16m + 4r + e
constexpr uint32_t tile_bytes(uint32_t type) {
    return type == 11 ? 2304u : type == 13 ? 3360u : type == 7 ? 4352u : type == 9 ? 1344u : 0u;
}

// A weight matrix in device memory. Quantized types: tiles
// [ceil(rows/16)][cols/256][tile_bytes] (rows past `rows` are zero). F32/F16:
// rows verbatim, `row_bytes` apart.
struct DMat {
    const uint8_t* data = nullptr;
    const float* bias = nullptr;  // optional f32 [rows]
    uint32_t type = 0;
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t row_bytes = 0;  // float types only
};

// int8 activation rows: per row, q holds the K codes, d one scale per `blk`
// values and s the sum of every 16 codes. 256-value blocks keep d in f32
// (inputs of the K-quant matrices: GGML's q8_K layout); 32-value blocks store
// d rounded to f16 (inputs of Q8_0 matrices: GGML's q8_0 block).
struct Act8 {
    int8_t* q = nullptr;
    float* d = nullptr;
    int16_t* s = nullptr;
    int32_t K = 0;    // values per row (multiple of 256)
    int32_t blk = kActBlock;
};

// Activation block a quantized matrix of `type` takes: 32 values for Q8_0
// (GGML's q8_0 x q8_0 dot), 256 for the K-quants (GGML's q8_K).
constexpr int32_t act_block(uint32_t type) { return type == 7 ? kActBlock32 : kActBlock; }

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
    int32_t n_end;                 // end-of-generation ids in end_token
    int32_t token[kMaxRows];
    int32_t pos[kMaxRows];
    int32_t seq[kMaxRows];
    int32_t out_row[kMaxRows];     // step row of each logits row
    int32_t draft[kMaxRows];       // token the logits row is compared with (-1: none)
    int32_t end_token[kMaxEndTokens];
    SeqDev seqs[kMaxSeq];
};

// Result block copied back to the host after a step.
struct StepOut {
    int32_t token[kMaxRows];       // argmax of each logits row (first max)
    int32_t accepted[kMaxSeq];     // accepted draft prefix per sequence (stops at an end id)
};

enum GemvMode : int32_t {
    kStore = 0,   // y = W x + bias
    kAdd = 1,     // y += W x (residual)
    kSwiGLU = 2,  // rows interleaved [gate x kGluGroup][up x kGluGroup]: y = silu(gate) * up
    kLogits = 3,  // y = W x + bias (optional store) and the greedy argmax per token
    kQKV = 4,     // fused q|k|v rows: bias, NEOX RoPE of q and k, q to qkv.q, k and v to the f16 cache
};

// Gate/up rows are interleaved in groups of this many rows per matrix (half a tile).
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
// tile holds both halves of every rotated pair.
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
    XIn x;                            // float activations (quantized by the matmul in blocks of `ablk`), or
    Act8 xq;                          // pre-quantized activations (used when xq.q is set)
    int32_t ablk = kActBlock;         // activation block of float inputs (act_block of the weight type)
    float* y = nullptr;               // output [tok][y_stride]
    int32_t y_stride = 0;
    unsigned long long* best = nullptr;  // kLogits: packed (value, -index) per token
    int32_t store_logits = 0;
    QkvOut qkv;
};

// Launchers (all asynchronous on `stream`).
//
// Kernel timing for profiles: while `stop` is set, the launchers of the
// calling thread attach the events to their kernel dispatches
// (hipExtLaunchKernel): `start` takes the begin time of the next dispatch,
// `stop` the end time of the last, so the elapsed time excludes queueing and
// launch gaps. Pass nullptrs to switch it off.
void set_launch_events(hipEvent_t start, hipEvent_t stop);
void launch_embed(const DMat& table, const StepDev* step, float* h, int32_t n_rows, int32_t H,
                  unsigned long long* best, int32_t n_best, hipStream_t stream);
// Matmul of up to kMaxRows token rows (in groups of 8) against one matrix.
void launch_gemv(const GemvArgs& a, hipStream_t stream);
// Quantizes n_rows float rows of K values (K % 256 == 0) into `out` (blocks of out.blk).
void launch_quantize(const float* x, int32_t stride, int32_t n_rows, const Act8& out, hipStream_t stream);
// RMS-normalizes n_rows float rows (row gather[r] when gather is set),
// multiplies them by `gain` and quantizes them into `out` (blocks of out.blk):
// the codes and scales the matmul's normalized-input prologue would stage.
void launch_quantize_norm(const float* x, int32_t stride, const int32_t* gather, const float* gain, float eps,
                          int32_t n_rows, const Act8& out, hipStream_t stream);
// Token rows of one matrix-core matmul launch (steps with more rows than the
// decode matmul's 8-row groups).
constexpr int kWideRows = kMaxRows;
// Whether launch_gemv_wide takes matrices of this type.
bool wide_matmul_supported(uint32_t type);
// Fewest token rows from which launch_gemv_wide outruns the token-quad
// matmul for a format (0: no wide kernel for it).
int32_t wide_min_rows(uint32_t type);
// Matmul of up to kWideRows pre-quantized token rows (a.xq) on matrix cores,
// 16-token tiles per work-group; every row's result equals launch_gemv's for
// that row alone. All modes.
void launch_gemv_wide(const GemvArgs& a, hipStream_t stream);
// Split-K causal GQA flash attention over the f16 caches of the step's
// sequences. Every (row, head, split) writes its (max, sum, unnormalized
// output) to `partial` (split stride `splits`); launch_attention_merge
// combines the splits. `slots` (0: splits) is the number of split slots the
// step can fill, and the grid's: every split of every sequence must fall below
// it (attention_slots).
void launch_attention(const float* q, const StepDev* step, int32_t max_len, int32_t n_seq, int32_t layer,
                      int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits, float* partial,
                      hipStream_t stream, int32_t slots = 0);
// Merges the splits of every (row, head) into out[row][n_head * head_dim]
// and, when xq.q is set, quantizes the rows into xq; reads the first `slots`
// (0: splits) split slots.
void launch_attention_merge(const float* partial, const StepDev* step, int32_t n_rows, int32_t n_head,
                            int32_t head_dim, int32_t splits, float* out, const Act8& xq, hipStream_t stream,
                            int32_t slots = 0);
int32_t attention_splits(int32_t capacity);
// Split slots a step can fill: all `splits` when a sequence of the step may
// bring kQuadGroupRows rows or fewer (the decode rule: about n_keys / splits
// keys per split); a single sequence of more rows (a prefill chunk) splits
// its keys into splits of at least the prefill length, so at most
// ceil(capacity / prefill length) of them.
int32_t attention_slots(int32_t splits, int32_t capacity, int32_t n_rows, int32_t n_seq);
// Query rows (G heads x tokens) one sequence may bring to a step per kv head.
int32_t attention_max_rows(int32_t head_dim);
// Floats of the attention split scratch for `rows` token rows.
size_t attention_partial_floats(int32_t rows, int32_t n_head, int32_t head_dim, int32_t splits);
void launch_finish(unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out,
                   hipStream_t stream);
void launch_dequant_rows(const DMat& m, int32_t row0, int32_t n_rows, float* out, hipStream_t stream);

// Static device scratch of the allocation-free matmul: one array of
// kScratchBytes per GPU, a file-scope __device__ variable that lives until
// the process ends. scratch_setup looks up this GPU's address of it
// (hipGetSymbolAddress) once per device and must run with that device
// current; scratch_address returns it (nullptr before setup). Kernels take
// the address as an argument: the variable's host-side name is no device
// address. Every user of one GPU's scratch holds scratch_lock(device) for
// the duration of its kernels.
constexpr size_t kScratchBytes = size_t{16} << 20;
constexpr int kScratchDevices = 64;
void scratch_setup(int device);
void* scratch_address(int device);
std::mutex& scratch_lock(int device);
// y[t][r] = full[t][device row of r] for r < rows, t < n_tok: the rows of one
// model tensor out of its (possibly fused) device matrix's output rows
// (kind 0 contiguous from offset, 1 RoPE pair order per head, 2 / 3 gate /
// up rows of the interleaved GLU matrix).
void launch_gather_rows(const float* full, int32_t full_stride, float* y, int32_t rows, int32_t n_tok, int32_t offset,
                        int32_t kind, int32_t head_dim, hipStream_t stream);
// Host evaluation of the device tile decoder: value k (< 256) of row (< 16) of one tile.
float dequant_tile_value(uint32_t type, const uint8_t* tile, uint32_t row, uint32_t k);

}  // namespace jfh::gpu
