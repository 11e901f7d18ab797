/*
 * jfo -- CPU oracle for the native Qwen2 stage forward of jetsonfabric.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests, the smoke
 * check and the CPU-baseline leg of the benchmark link it to compare the HIP
 * engine against a plain CPU restatement of the reference algorithm. Nothing
 * in the product (jetsonfabric_amd/) may link, import or call it.
 *
 * What it restates (reference paths relative to the reference checkout):
 *   - GGML block layouts and dequantization for F32, F16, Q8_0, Q2_K, Q4_K,
 *     Q6_K, the tensor types the native engine stores verbatim
 *     (runtime/engines/native/src/tensor_store.cpp:23-40; block geometry
 *     runtime/engines/native/src/engine.c:284-310, docs/jfm-v2-format.md).
 *   - The Qwen2 graph built by ForwardGraph::build
 *     (runtime/engines/native/src/qwen2_architecture.cpp:522-598): embedding
 *     row gather, per layer RMSNorm*gain (373-376), Q/K/V projections with
 *     bias (361-371, 394-396), NEOX RoPE (499-506), F16 KV cache write
 *     (405-424), causal GQA attention with scale hd^-1/2 (438-464, mask
 *     697-708), output projection, residual adds (569-577), SwiGLU FFN
 *     (508-520), output norm + head (+ optional bias) on the selected rows
 *     (584-586, 378-384) and first-index argmax (594).
 *   - Session bookkeeping: positions, capacity checks and rollback
 *     (qwen2_architecture.cpp:800-823, 1040-1054).
 *
 * Matmul numerics. GGML's backends quantize the activation vector to int8
 * blocks before the integer dot with quantized weights. The HIP engine does
 * the same with fixed rules and the oracle restates them, so that GPU and CPU
 * see identical integer sums (JFO_MODE_Q8):
 *   - inputs of K-quant matrices (Q2_K, Q4_K, Q6_K): int8 per 256 values,
 *     d = amax/127 kept in f32, 16-value code sums (the layout of GGML's
 *     q8_K, which its CPU backend pairs with the K-quants);
 *   - inputs of Q8_0 matrices: int8 per 32 values, d = amax/127 stored as
 *     f16 (GGML's q8_0 block, the rule of its q8_0 x q8_0 dot).
 * JFO_MODE_EXACT instead multiplies the exactly dequantized weights with
 * float activations: the mathematically exact product, used to bound the
 * error the activation quantization introduces.
 *
 * Parity status of each function is recorded in oracle/README.md.
 */
#ifndef JFO_H
#define JFO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Stable JFM tensor type ids (runtime/engines/native/include/jetsonfabric/engine.h:13-49). */
enum {
    JFO_F32 = 1,
    JFO_F16 = 2,
    JFO_Q8_0 = 7,
    JFO_Q2_K = 9,
    JFO_Q4_K = 11,
    JFO_Q6_K = 13,
};

/* JFO_MODE_Q8: activations quantized by the block rule of the weight type
 * (32 values for Q8_0, 256 for the K-quants). */
enum { JFO_MODE_EXACT = 0, JFO_MODE_Q8 = 1 };

/* Activation block of a quantized matmul input: 32 for Q8_0 weights, else 256. */
int jfo_act_block(int type);

float jfo_f16_to_f32(uint16_t h);
uint16_t jfo_f32_to_f16(float f);

/* Elements and bytes of one storage block; returns 0 for unsupported types. */
int jfo_type_block(int type, uint32_t * block_elements, uint32_t * block_bytes);

/* Dequantizes n (a multiple of the block size) values of one row. Returns 0 on success. */
int jfo_dequantize_row(int type, const void * src, float * dst, int64_t n);

/*
 * Activation quantization shared with the HIP engine: per block of 256 values
 * amax = max|x|, d = amax / 127, id = d ? 1 / d : 0, q = roundf(x * id).
 * Outputs q[n], d[n/256] and the integer sum of every 16 values, s16[n/16].
 */
void jfo_quantize_act(const float * x, int64_t n, int8_t * q, float * d, int16_t * s16);

/*
 * The same rule over blocks of blk (256 or 32) values, d[n/blk]. For 32-value
 * blocks the stored scale is d rounded to f16 (the codes use the f32 id), as
 * GGML's q8_0 / q8_1 blocks store it.
 */
void jfo_quantize_act_blk(const float * x, int64_t n, int blk, int8_t * q, float * d, int16_t * s16);

/*
 * Quantization of an RMS-normalized row as the HIP engine stages it: the codes
 * of x[i] * gain[i] per 256-value block (d' = amax/127, q = roundf(v / d')),
 * each block scale multiplied by the row's 1 / sqrtf(mean(x^2) + eps), so
 * that d[b] * q[i] approximates (x[i] * rms_scale) * gain[i].
 */
void jfo_quantize_act_normed(const float * x, const float * gain, int64_t n, float eps, int8_t * q, float * d,
                             int16_t * s16);

/* The same over blocks of blk values (256, or 32 for Q8_0 inputs); 32-value
 * block scales are (d' * rms_scale) rounded to f16. */
void jfo_quantize_act_normed_blk(const float * x, const float * gain, int64_t n, float eps, int blk, int8_t * q,
                                 float * d, int16_t * s16);

/* y[t * rows + r] = W[r] . (q, d, s16)[t]: jfo_matmul's JFO_MODE_Q8 on pre-quantized rows
 * (256-value blocks for the K-quants, 32 for Q8_0). */
int jfo_matmul_q8(int type, const void * w, int64_t n, int64_t rows, const int8_t * q, const float * d,
                  const int16_t * s16, int64_t tokens, float * y, int threads);

/* The same with activation blocks of blk values (d: n / blk scales per row);
 * blk must be the weight type's jfo_act_block. */
int jfo_matmul_q8_blk(int type, const void * w, int64_t n, int64_t rows, const int8_t * q, const float * d,
                      const int16_t * s16, int64_t tokens, float * y, int blk, int threads);

/* Dot product of one weight row with a quantized activation (n % 256 == 0):
 * integer dot per sub-block scaled by the sub-block scale, one float combine
 * per 256-value block (K-quants) or per 32-value block (Q8_0). */
double jfo_vec_dot_q8(int type, const void * row, const int8_t * q, const float * d,
                      const int16_t * s16, int64_t n);

/* The same with activation blocks of blk values, which must be the weight
 * type's jfo_act_block (returns 0 otherwise): the K-quants per 256-value
 * block as above; Q8_0 per 32-value block b, d[b] * dw * dot, summed in
 * double (GGML's q8_0 x q8_0 product). */
double jfo_vec_dot_q8_blk(int type, const void * row, const int8_t * q, const float * d, const int16_t * s16,
                          int64_t n, int blk);

/* Dot product of one weight row with float activations, exact dequantization. */
double jfo_vec_dot_f32(int type, const void * row, const float * x, int64_t n);

/*
 * y[t * rows + r] = W[r] . x[t * n ..] for t < tokens, r < rows.
 * mode JFO_MODE_Q8 quantizes each activation row first (types Q8_0/Q2_K/Q4_K/Q6_K);
 * float weight types always use float activations.
 */
int jfo_matmul(int type, const void * w, int64_t n, int64_t rows,
               const float * x, int64_t tokens, float * y, int mode, int threads);

/* Model description: pointers into caller-owned host memory. */
typedef struct jfo_tensor {
    int32_t type;
    int32_t pad;
    int64_t ne0; /* row length (elements) */
    int64_t ne1; /* rows */
    const void * data;
} jfo_tensor;

typedef struct jfo_layer {
    jfo_tensor attn_norm, wq, bq, wk, bk, wv, bv, wo, ffn_norm, w_gate, w_up, w_down;
} jfo_layer;

typedef struct jfo_model {
    int32_t n_layer, n_embd, n_ff, n_head, n_head_kv, n_ctx, n_vocab, pad;
    float rope_base, rms_eps;
    jfo_tensor tok_embd, output_norm, output, output_bias; /* output_bias.data may be NULL */
    const jfo_layer * layers;
} jfo_model;

typedef struct jfo_session jfo_session;

jfo_session * jfo_session_create(const jfo_model * model, int32_t capacity, int32_t mode, int32_t threads);
void jfo_session_destroy(jfo_session * s);
int32_t jfo_session_position(const jfo_session * s);

/*
 * Runs tokens[0..n) at positions pos..pos+n-1 and advances the position.
 * logits_rows = 0: no logits; 1: logits of the last row only; n: logits of
 * every row (verify). argmax_out (may be NULL) gets one id per logits row.
 * Returns 0, or a negative error: -1 argument, -2 capacity, -3 vocabulary.
 */
int32_t jfo_session_forward(jfo_session * s, const int32_t * tokens, int32_t n,
                            int32_t logits_rows, float * logits, int32_t * argmax_out);

/*
 * Stage forward over layers [layer_begin, layer_end) at positions pos..pos+n-1
 * (advances the position; only the range's KV rows are written). The first
 * stage (layer_begin 0) takes token ids and rows_in NULL; a later stage takes
 * tokens NULL and the previous stage's f32 residual rows rows_in [n][n_embd].
 * rows_out (may be NULL) receives (layer_end - layer_begin + 1) blocks of
 * [n][n_embd]: the rows entering each layer of the range, then the rows after
 * its last layer. Logits (as jfo_session_forward) only when layer_end is the
 * model's last layer. Returns 0 or the errors of jfo_session_forward.
 */
int32_t jfo_session_forward_range(jfo_session * s, const int32_t * tokens, const float * rows_in, int32_t n,
                                  int32_t layer_begin, int32_t layer_end, float * rows_out,
                                  int32_t logits_rows, float * logits, int32_t * argmax_out);

/* Rolls back n decoded positions: 0 < n <= position - prefill position. Returns 0 or -1. */
int32_t jfo_session_rollback(jfo_session * s, int32_t n);

/* Fills positions [0, n) of every layer's K/V cache with seeded f16 values and sets
 * the position to n (prefill position n). Used to time decode at a long context. */
int32_t jfo_session_fill_kv(jfo_session * s, int32_t n, uint64_t seed);

/* Copies layer l's cached K and V rows [0, n) as f16, layout [n_head_kv][n][head_dim]. */
int32_t jfo_session_read_kv(const jfo_session * s, int32_t layer, int32_t n, uint16_t * k, uint16_t * v);

/* Writes layer l's cached K and V rows [0, n) (same layout as read). */
int32_t jfo_session_write_kv(jfo_session * s, int32_t layer, int32_t n, const uint16_t * k, const uint16_t * v);

/* RoPE angle table used by oracle and engine: cos/sin of pos * base^(-2i/hd),
 * the angle advanced by repeated float multiplication as GGML's rope does.
 * out has 2 * (hd/2) floats per position: cos at [2i], sin at [2i+1]. */
void jfo_rope_table(float base, int32_t head_dim, int32_t pos_begin, int32_t pos_count, float * out);

/* Greedy argmax (first maximum) of n floats. */
int32_t jfo_argmax(const float * x, int64_t n);

#ifdef __cplusplus
}
#endif

#endif
