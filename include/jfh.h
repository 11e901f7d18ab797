/*
 * jfh.h -- C ABI of the MI355X (gfx950) native Qwen2 stage engine.
 *
 * Plain pointers and sizes only. Every call that can fail returns a
 * jfh_status by value (code + message), like the reference loader's
 * jf_status (runtime/engines/native/include/jetsonfabric/engine.h:51-63).
 * Opaque handles are created/destroyed in pairs; caller-owned input arrays
 * are read during the call; caller-provided output arrays are written.
 *
 * Each entry point names the reference interface it replaces.
 */
#ifndef JFH_H
#define JFH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0..5 equal jf_status_code (engine.h:51-58); 6 = device error. */
typedef enum jfh_status_code {
    JFH_STATUS_OK = 0,
    JFH_STATUS_INVALID_ARGUMENT = 1,
    JFH_STATUS_IO_ERROR = 2,
    JFH_STATUS_FORMAT_ERROR = 3,
    JFH_STATUS_NOT_FOUND = 4,
    JFH_STATUS_OUT_OF_MEMORY = 5,
    JFH_STATUS_DEVICE_ERROR = 6
} jfh_status_code;

typedef struct jfh_status {
    int32_t code;
    char message[256];
} jfh_status;

/* Tensor type ids of the JFM v2 format: the values of jf_tensor_type
 * (engine.h:13-42) for the types this engine runs. */
typedef enum jfh_tensor_type {
    JFH_TENSOR_F32 = 1,
    JFH_TENSOR_F16 = 2,
    JFH_TENSOR_Q8_0 = 7,
    JFH_TENSOR_Q2_K = 9,
    JFH_TENSOR_Q4_K = 11,
    JFH_TENSOR_Q6_K = 13
} jfh_tensor_type;

typedef struct jfh_model jfh_model;     /* host-resident weights + hparams */
typedef struct jfh_engine jfh_engine;   /* device-resident weights, one HIP stream */
typedef struct jfh_session jfh_session; /* one sequence's F16 KV cache + position */

/* Qwen2 hyper-parameters (runtime/engines/native/src/qwen2_metadata.hpp:10-18). */
typedef struct jfh_model_params {
    uint32_t n_layer;
    uint32_t n_embd;
    uint32_t n_ff;
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t n_ctx;
    uint32_t n_vocab;
    uint32_t head_dim;
    float rope_base;
    float rms_eps;
} jfh_model_params;

/* Tensor view (jf_tensor_view, engine.h:85-96). `name` is NUL-terminated and
 * valid, like `data`, until the model is closed. */
typedef struct jfh_tensor_view {
    const char * name;
    uint32_t type;
    uint32_t rank;
    uint64_t shape[4];
    int32_t layer;
    const void * data;
    uint64_t size;
} jfh_tensor_view;

/* Residency statistics (jf_model_stats, engine.h:74-83). */
typedef struct jfh_model_stats {
    uint32_t layer_start;
    uint32_t layer_end;
    uint32_t layer_count;
    uint64_t selected_weight_bytes;
    uint64_t total_weight_bytes;
    uint64_t selected_tensor_count;
    uint64_t total_tensor_count;
} jfh_model_stats;

/* Synthetic model recipe: N(0, stddev) weights keyed by (seed, tensor name). */
typedef struct jfh_synth_spec {
    jfh_model_params params;
    uint32_t type_linear;
    uint32_t type_embd;
    uint32_t type_output;
    uint32_t tied_output; /* output.weight is a byte copy of token_embd.weight */
    uint32_t output_bias;
    uint32_t pad;
    uint64_t seed;
    float stddev;
    int32_t threads; /* 0 = all hardware threads */
} jfh_synth_spec;

typedef struct jfh_engine_options {
    int32_t device;     /* HIP device ordinal */
    int32_t use_graphs; /* capture each step shape in a HIP graph */
} jfh_engine_options;

typedef struct jfh_engine_info {
    uint64_t weight_bytes;
    uint32_t prefill_chunk;
    char device_name[128];
    /* resident layer range [layer_start, layer_end) of the model's n_layer
     * (ModelInfo::resident_layer_start/end, native_inference.hpp:30-40) */
    uint32_t layer_start;
    uint32_t layer_end;
} jfh_engine_info;

/* ---------------------------------------------------------------- formats */

/* jf_tensor_type_layout (engine.h:100-104; engine.c:284-310). */
jfh_status jfh_tensor_type_layout(uint32_t type, uint32_t * block_elements, uint32_t * block_bytes);

/* SHA-256 used for JFM segment integrity (sha256.h:20-23 of the reference loader). */
jfh_status jfh_sha256(const void * data, size_t size, uint8_t digest[32]);

/* ---------------------------------------------------------------- JFM v2 packages */

typedef struct jfh_package jfh_package; /* mmapped JFM v2 package, no model validation */

/* Residency statistics of an open package (jf_model_stats, engine.h:74-83). */
typedef struct jfh_package_stats {
    uint32_t layer_start;
    uint32_t layer_end;
    uint32_t layer_count;
    uint32_t pad;
    uint64_t selected_weight_bytes;
    uint64_t total_weight_bytes;
    uint64_t mapped_bytes;
    uint64_t selected_tensor_count;
    uint64_t total_tensor_count;
} jfh_package_stats;

/* jf_model_open (engine.h:106-111; engine.c:513-757): opens the segments of the
 * half-open layer range (layer_end UINT32_MAX = all), verifying SHA-256s. */
jfh_status jfh_package_open(const char * package_path, uint32_t layer_start, uint32_t layer_end,
                            uint32_t verify_hashes, jfh_package ** out);
/* jf_model_close (engine.h:113). */
void jfh_package_close(jfh_package * package);
/* jf_model_get_stats (engine.h:115). */
jfh_status jfh_package_get_stats(const jfh_package * package, jfh_package_stats * out);
/* jf_model_tensor_count / jf_model_tensor_at / jf_model_find_tensor (engine.h:117-129);
 * tensors are sorted by name. */
size_t jfh_package_tensor_count(const jfh_package * package);
jfh_status jfh_package_tensor_at(const jfh_package * package, size_t index, jfh_tensor_view * out);
jfh_status jfh_package_find_tensor(const jfh_package * package, const char * name, jfh_tensor_view * out);
/* jf_model_get_gguf_metadata / jf_model_get_source_sha256 (engine.h:141-150). */
jfh_status jfh_package_gguf_metadata(const jfh_package * package, const void ** data, size_t * size);
jfh_status jfh_package_source_sha256(const jfh_package * package, uint8_t digest[32]);

/* ---------------------------------------------------------------- host model */

/* jf_model_open (engine.h:107-111) + TensorStore/load_qwen2_hparams
 * (tensor_store.cpp:57-116; qwen2_metadata.cpp:90-125). layer_end may be
 * UINT32_MAX for "all layers". */
jfh_status jfh_model_open(const char * package_path, uint32_t layer_start, uint32_t layer_end,
                          uint32_t verify_hashes, jfh_model ** out);

/* jf_model_compile's input side (runtime/compiler/jf_model_compile.cpp:549-645):
 * a qwen2 GGUF file, memory-mapped, as a host model whose tensors are used in
 * place; jfh_model_write_package then writes its JFM v2 package, recording
 * the file's SHA-256 and size. Tensor types F32, F16, Q8_0, Q2_K, Q4_K, Q6_K;
 * output.weight is required (JFM v2 has no tied output). */
jfh_status jfh_model_open_gguf(const char * gguf_path, jfh_model ** out);

/* Synthetic weights for benchmarks (no reference counterpart: the reference
 * imports real GGUFs, runtime/compiler/jf_model_compile.cpp:549-645). */
jfh_status jfh_model_synthesize(const jfh_synth_spec * spec, jfh_model ** out);

/* In-memory model builder (the reference's tiny fixture writer,
 * runtime/compiler/model_fixture.cpp:92-133, builds models tensor by tensor). */
jfh_status jfh_model_create(const jfh_model_params * params, jfh_model ** out);
jfh_status jfh_model_add_tensor(jfh_model * model, const char * name, uint32_t type, uint32_t rank,
                                const uint64_t * shape, const void * data, uint64_t size);
/* Validates names/shapes (qwen2_architecture.cpp:80-118). */
jfh_status jfh_model_finalize(jfh_model * model);

/* Writes a JFM v2 package (docs/jfm-v2-format.md; segment grouping
 * runtime/compiler/jf_model_compile.cpp:612-624). */
jfh_status jfh_model_write_package(const jfh_model * model, const char * directory);

/* The layer range [layer_start, layer_end) of a finalized model as a model of
 * its own (its tensors copied; the embedding when layer_start is 0, the
 * output norm and head when layer_end is n_layer), the in-memory counterpart
 * of opening a package with a layer range (jf_model_open, engine.h:106-111;
 * engine.c:513-757). An engine created from it is that pipeline stage. */
jfh_status jfh_model_slice(const jfh_model * model, uint32_t layer_start, uint32_t layer_end, jfh_model ** out);

/* jf_model_close (engine.h:113). */
void jfh_model_close(jfh_model * model);

jfh_status jfh_model_get_params(const jfh_model * model, jfh_model_params * out);
/* jf_model_get_stats (engine.h:115). */
jfh_status jfh_model_get_stats(const jfh_model * model, jfh_model_stats * out);
/* jf_model_tensor_count / jf_model_tensor_at / jf_model_find_tensor (engine.h:117-129). */
size_t jfh_model_tensor_count(const jfh_model * model);
jfh_status jfh_model_tensor_at(const jfh_model * model, size_t index, jfh_tensor_view * out);
jfh_status jfh_model_find_tensor(const jfh_model * model, const char * name, jfh_tensor_view * out);
/* Hex SHA-256 of the source GGUF (ModelInfo::source_sha256, native_inference.hpp:34). */
jfh_status jfh_model_source_sha256(const jfh_model * model, char hex[65]);

/* ---------------------------------------------------------------- engine */

/* NativeEngine(package, EngineOptions) (native_inference.hpp:128-129): weights
 * are uploaded once; the model may be closed afterwards. */
jfh_status jfh_engine_create(const jfh_model * model, const jfh_engine_options * options, jfh_engine ** out);
void jfh_engine_destroy(jfh_engine * engine);
jfh_status jfh_engine_get_info(const jfh_engine * engine, jfh_engine_info * out);
/* Hyper-parameters of the engine's model (NativeEngine::model_info,
 * native_inference.hpp:138; the whole model's n_layer also for a stage). */
jfh_status jfh_engine_get_params(const jfh_engine * engine, jfh_model_params * out);
/* End-of-generation ids of the stage's tokenizer (Tokenizer::is_end_token,
 * runtime/tokenization/tokenizer.hpp:16). The on-GPU acceptance of every later
 * verify step (jfh_session_verify, jfh_engine_step_batch out_accepted) stops
 * at a draft position whose greedy id is one of them, as the runner's
 * acceptance loop does (runtime/pipeline_parallel/generation_runner.cpp:
 * 512-517); jfh_generate and jfh_generate_concurrent end a request at one
 * (finish reason "stop"). At most 16 ids, each inside the vocabulary; n = 0
 * clears the set (the default). */
jfh_status jfh_engine_set_end_tokens(jfh_engine * engine, const int32_t * ids, uint32_t n);

/* NativeEngine::create_session (native_inference.hpp:143). */
jfh_status jfh_session_create(jfh_engine * engine, uint32_t capacity, jfh_session ** out);
void jfh_session_destroy(jfh_session * session);
/* NativeSession::capacity/position (native_inference.hpp:108-109). */
uint32_t jfh_session_capacity(const jfh_session * session);
uint32_t jfh_session_position(const jfh_session * session);

/* NativeSession::prefill_greedy / Qwen2Session::prefill_logits
 * (native_inference.hpp:110; qwen2_architecture.cpp:825-879). logits may be
 * NULL; otherwise it receives n_vocab floats for the last row. */
jfh_status jfh_session_prefill(jfh_session * session, const int32_t * tokens, uint32_t n,
                               int32_t * out_token, float * logits);

/* NativeSession::decode_greedy / decode_logits (native_inference.hpp:111;
 * qwen2_architecture.cpp:881-907). */
jfh_status jfh_session_decode(jfh_session * session, int32_t token, int32_t * out_token, float * logits);

/* Draft verification: tokens = [previous, draft...] decoded at consecutive
 * positions in one pass; out_tokens gets the greedy id after every row, and
 * out_accepted the number of leading draft tokens equal to those ids. The
 * session advances by n; the caller rolls back n - 1 - accepted. Replaces the
 * llama.cpp multi-row verify (llama_cpp_stage_adapter.cpp:350-386, 388-475).
 * logits may be NULL, else n * n_vocab floats. */
jfh_status jfh_session_verify(jfh_session * session, const int32_t * tokens, uint32_t n, int32_t * out_tokens,
                              uint32_t * out_accepted, float * logits);

/* Pipeline stages. An engine created from a model opened with a layer range
 * runs only those layers (LayerRange, model_architecture.hpp:15-21): the
 * first stage (layer_start 0) takes token ids, later stages take the
 * previous stage's activations, f32 [n][n_embd] (the residual stream after
 * its last layer); the last stage (layer_end n_layer) writes the greedy id of
 * the last row to out_token, earlier stages write every row's activations to
 * out_activations. Pass NULL for the unused input and output. logits may be
 * NULL; on the last stage it receives n_vocab floats for the last row (as
 * jfh_session_prefill's logits), other stages reject it.
 * NativeSession::prefill_stage_tokens / prefill_stage_activations
 * (native_inference.hpp:112-113; qwen2_architecture.cpp:909-926, 977-1002). */
jfh_status jfh_session_stage_prefill(jfh_session * session, const int32_t * tokens, const float * activations,
                                     uint32_t n, int32_t * out_token, float * out_activations, float * logits);
/* One row: NativeSession::decode_stage_token / decode_stage_activation
 * (native_inference.hpp:114-115; qwen2_architecture.cpp:928-947, 1004-1027).
 * token points to the first stage's input id (NULL on later stages). */
jfh_status jfh_session_stage_decode(jfh_session * session, const int32_t * token, const float * activation,
                                    int32_t * out_token, float * out_activation, float * logits);

/* Activation codecs between pipeline stages (ActivationCodec, created by
 * name from the default factory: runtime/activation/activation_codec.hpp:9-18,
 * activation_codec_factory.cpp:24-46, builtin_activation_codecs.cpp:112-209).
 * "f32" carries the values unchanged, "f16" as little-endian IEEE binary16
 * (round to nearest even; NaNs quieted). encode writes n values' wire bytes
 * (out_size must be n * 2 or n * 4); decode reads size bytes into size / 2 or
 * size / 4 floats. */
jfh_status jfh_activation_encode(const char * codec, const float * values, size_t n, void * out, size_t out_size);
jfh_status jfh_activation_decode(const char * codec, const void * data, size_t size, float * values, size_t n);

/* NativeSession::rollback (native_inference.hpp:116; qwen2_architecture.cpp:818-823). */
jfh_status jfh_session_rollback(jfh_session * session, uint32_t n);

/* Batched decode/verify over several sessions in one pass
 * (Executor::execute_batch, runtime/inference/executor.hpp:20-28;
 * continuous_batching_executor.cpp:60-100). lengths[i] rows for sessions[i],
 * tokens concatenated; out_tokens receives sum(lengths) ids, out_accepted one
 * count per session (may be NULL), logits (may be NULL) sum(lengths) *
 * n_vocab floats, the rows in the order of out_tokens. A step holds at most
 * 256 token rows (JFH_STATUS_INVALID_ARGUMENT beyond); prefills are split into
 * chunks of jfh_engine_info.prefill_chunk rows. */
jfh_status jfh_engine_step_batch(jfh_engine * engine, jfh_session * const * sessions, uint32_t count,
                                 const int32_t * tokens, const uint32_t * lengths, int32_t * out_tokens,
                                 uint32_t * out_accepted, float * logits);

/* Several sessions' rows through one pipeline stage in one pass: the stage
 * form of jfh_engine_step_batch, for draft verification and batched decode in
 * stages (the reference verifies through its llama.cpp stage adapter,
 * llama_cpp_stage_adapter.cpp:350-475, 703-823; its native stage decodes one
 * row per pass, native_stage_executor.cpp:285-306). lengths[i] rows of
 * sessions[i] at its position, every session prefilled; token ids
 * (concatenated) into the first stage, f32 [rows][n_embd] activations into
 * later ones. The last stage writes every row's greedy id to out_tokens and,
 * when logits is set, every row's logits (rows x vocab); the others write
 * every row's output activations to out_activations. */
jfh_status jfh_engine_stage_step_batch(jfh_engine * engine, jfh_session * const * sessions, uint32_t count,
                                       const int32_t * tokens, const float * activations, const uint32_t * lengths,
                                       int32_t * out_tokens, float * out_activations, float * logits);

/* Parity entry points: GPU dequantization of tensor rows (bit-exact with the
 * GGML layouts) and a matmul through the engine's kernels. */
jfh_status jfh_engine_dequantize(jfh_engine * engine, const char * tensor, uint32_t row0, uint32_t n_rows,
                                 float * out);
jfh_status jfh_engine_matmul(jfh_engine * engine, const char * tensor, const float * x, uint32_t n_tok, float * y);

/* Allocation-free variant of jfh_engine_matmul. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). x and y are DEVICE
 * buffers, x f32 [n_tok][cols] and y f32 [n_tok][rows] of the tensor; the
 * result equals jfh_engine_matmul's bit for bit. stream is the caller's HIP
 * stream (hipStream_t; NULL: the null stream): the matmul reads x only after
 * the work already enqueued there, so x may still be in flight on it. The
 * kernels run on the engine's own stream and the call returns after the
 * result is in y; it cannot be recorded into the caller's graph capture. The
 * staging (int8 copies of the rows, the fused device matrix's full output
 * rows) lives in the library's static device scratch, one 16 MiB array per
 * GPU held until the process ends; calls whose staging exceeds it fail with
 * JFH_STATUS_INVALID_ARGUMENT before any work. Calls on one GPU share that
 * array: the library serializes them, so a caller must not expect two of them
 * to overlap. */
jfh_status jfh_engine_matmul_noalloc(jfh_engine * engine, const char * tensor, const float * x, uint32_t n_tok,
                                     float * y, void * stream);

/* Parity entry points for the F16 KV cache (no reference counterpart: the
 * reference's cache lives in GGML tensors, qwen2_architecture.cpp:1056-1092).
 * read_kv copies positions [0, n) of one layer out of a session, layout
 * [kv_head][n][head_dim]; import_kv writes positions [0, n) of every layer,
 * layout [layer][kv_head][n][head_dim], and leaves the session at position n
 * as after a prefill of n tokens (a long context without running it). */
jfh_status jfh_session_read_kv(const jfh_session * session, uint32_t layer, uint32_t n, uint16_t * k, uint16_t * v);
jfh_status jfh_session_import_kv(jfh_session * session, uint32_t n, const uint16_t * k, const uint16_t * v);

/* Device time of `iterations` back-to-back decode steps (ms, HIP events on the
 * engine stream) after `warmup` untimed ones; the session is rolled back after
 * each step, so every step runs at the same position. */
jfh_status jfh_session_time_steps(jfh_session * session, const int32_t * tokens, uint32_t n, uint32_t all_logits,
                                  uint32_t warmup, uint32_t iterations, double * ms_per_step);

/* Per-kernel profile of one step (no reference counterpart: the reference
 * measures with Nsight, docs/benchmarks/evidence/...kernels_cuda_gpu_kern_sum.csv).
 * The step runs `iterations` times without graphs with HIP events attached to
 * every kernel dispatch (hipExtLaunchKernel) on the engine stream; one entry
 * per kernel and role, sorted by device time. */
typedef struct jfh_kernel_stat {
    char label[64];
    double launches; /* per step */
    double total_ms; /* device ms per step */
    double bytes;    /* algorithmic HBM bytes per step */
} jfh_kernel_stat;

jfh_status jfh_session_profile_step(jfh_session * session, const int32_t * tokens, uint32_t n, uint32_t all_logits,
                                    uint32_t iterations, jfh_kernel_stat * out, uint32_t capacity, uint32_t * count);
/* The same profile for one batched step over several sessions (the rows of
 * jfh_engine_step_batch: lengths[i] rows for sessions[i], tokens concatenated),
 * every row producing logits when all_logits is set, else the last row of each
 * session; the sessions are rolled back after every iteration. */
jfh_status jfh_engine_profile_batch(jfh_engine * engine, jfh_session * const * sessions, uint32_t count,
                                    const int32_t * tokens, const uint32_t * lengths, uint32_t all_logits,
                                    uint32_t iterations, jfh_kernel_stat * out, uint32_t capacity,
                                    uint32_t * out_count);

/* ---------------------------------------------------------------- tokenizer */

/* Byte-level BPE tokenizer of a Qwen2 GGUF vocabulary: the reference's
 * LlamaCppTokenizer (runtime/adapters/llama_cpp_tokenizer.hpp:11-31,
 * llama_cpp_tokenizer.cpp:50-137), which serves native packages from their
 * preserved metadata.gguf. `path`: a package directory (its metadata.gguf)
 * or a GGUF file. JFH_STATUS_NOT_FOUND for a package without metadata.gguf,
 * JFH_STATUS_FORMAT_ERROR for metadata without a "gpt2" vocabulary. */
typedef struct jfh_tokenizer jfh_tokenizer;
jfh_status jfh_tokenizer_open(const char * path, jfh_tokenizer ** out);
void jfh_tokenizer_destroy(jfh_tokenizer * tokenizer);
/* Tokenizer::tokenize (runtime/tokenization/tokenizer.hpp:14; llama_cpp_tokenizer.cpp:100-110):
 * special tokens in the text are parsed, BOS/EOS added as the metadata asks;
 * an empty result is JFH_STATUS_INVALID_ARGUMENT. *out_count receives the
 * number of ids; a buffer of fewer than that many is
 * JFH_STATUS_INVALID_ARGUMENT (ask with capacity 0 first). */
jfh_status jfh_tokenizer_tokenize(const jfh_tokenizer * tokenizer, const char * text, size_t length, int32_t * ids,
                                  uint32_t capacity, uint32_t * out_count);
/* Tokenizer::token_piece (tokenizer.hpp:15; llama_cpp_tokenizer.cpp:112-133): the
 * token's bytes (not NUL-terminated) into buf; *out_length receives their
 * count, a smaller buffer is JFH_STATUS_INVALID_ARGUMENT. */
jfh_status jfh_tokenizer_token_piece(const jfh_tokenizer * tokenizer, int32_t token, char * buf, uint32_t capacity,
                                     uint32_t * out_length);
/* Tokenizer::is_end_token (tokenizer.hpp:16; llama_cpp_tokenizer.cpp:135-137). */
jfh_status jfh_tokenizer_is_end_token(const jfh_tokenizer * tokenizer, int32_t token, uint32_t * out);
/* The end-of-generation ids in ascending order (the set is_end_token tests,
 * without -1), e.g. for jfh_engine_set_end_tokens; *out_count receives their
 * number, a smaller buffer is JFH_STATUS_INVALID_ARGUMENT. */
jfh_status jfh_tokenizer_end_tokens(const jfh_tokenizer * tokenizer, int32_t * ids, uint32_t capacity,
                                    uint32_t * out_count);
/* Number of tokens in the vocabulary. */
jfh_status jfh_tokenizer_vocab_size(const jfh_tokenizer * tokenizer, uint32_t * out);

/* ---------------------------------------------------------------- speculation */

/* PromptLookupDraft::propose (runtime/speculative/prompt_lookup_draft.cpp:15-44). */
jfh_status jfh_prompt_lookup_propose(const uint32_t * history, size_t n, uint32_t max_ngram, uint32_t min_ngram,
                                     uint32_t max_tokens, uint32_t * out, uint32_t * out_count);

typedef struct jfh_generation_stats {
    uint32_t completion_tokens;
    uint32_t target_decode_passes;
    uint32_t speculative_draft_tokens;
    uint32_t speculative_accepted_tokens;
    double time_to_first_token_ms;
    double decode_ms;
    uint32_t stopped;  /* 1: ended at an end-of-generation id (finish reason "stop"), 0: at max_tokens */
    uint32_t reserved;
    /* GenerationResult's rates (native_inference.hpp:88-96) */
    double inter_token_latency_ms;        /* decode_ms per token after the first */
    double decode_tokens_per_second;      /* tokens after the first / decode_ms */
    double end_to_end_tokens_per_second;  /* sampled tokens / (time to first token + decode_ms) */
    /* PrefillMetrics (native_inference.hpp:71-78): the prompt's steps */
    uint32_t prefill_plan_reused;         /* every prefill step shape's captured graph existed already */
    uint32_t prefill_attention_matrix_cores; /* attention on MFMA (head dim 64 or 128) */
    double prefill_planning_ms;           /* capturing and instantiating new step graphs */
    double prefill_allocation_ms;         /* the session's KV cache allocation and clearing */
    double prefill_host_input_ms;         /* building and uploading the step descriptors */
    double prefill_compute_ms;            /* device time of the step graphs */
    double prefill_output_read_ms;        /* device time of the result copies */
    /* ExecutionBufferMetrics (native_inference.hpp:80-85) */
    uint64_t kv_cache_bytes;              /* the session's F16 K/V cache */
    uint64_t prefill_scratch_bytes;       /* engine workspace of one prefill chunk's rows */
    uint64_t decode_scratch_bytes;        /* engine workspace of one decode row */
    uint64_t prefill_host_input_bytes;    /* step descriptor bytes uploaded for the prompt */
} jfh_generation_stats;

/* GenerationRunner::run speculative loop (generation_runner.cpp:398-566) over
 * the HIP stage executor: prefill, prompt-lookup drafts of up to draft_max
 * tokens, one verify pass per draft, greedy acceptance, rollback, single-token
 * recovery pass after a rejection. draft_max 0 disables speculation. */
jfh_status jfh_generate(jfh_engine * engine, const int32_t * prompt, uint32_t n_prompt, uint32_t max_tokens,
                        uint32_t draft_max, uint32_t max_ngram, uint32_t min_ngram, int32_t * out_tokens,
                        uint32_t * out_count, jfh_generation_stats * stats);

/* A caller's draft strategy (DraftStrategy::propose,
 * runtime/speculative/draft_strategy.hpp:9-17): given the history (prompt and
 * generated ids, n of them), writes at most max_tokens proposed ids to out
 * and returns how many it wrote (0: no draft this pass). */
typedef uint32_t (*jfh_draft_propose_fn)(void * user, const uint32_t * history, size_t n, uint32_t max_tokens,
                                         uint32_t * out);

/* jfh_generate with drafts from a caller-supplied strategy: the runner of
 * GenerationRunner::run (generation_runner.cpp:469-556) with any
 * DraftStrategy, as the reference's harness installs FixedDraft
 * (runtime/pipeline_parallel/generation_runner_test.cpp:108-119). propose is
 * called on the calling thread before each verify pass (not after a rejected
 * draft: that pass is the single-token recovery pass). */
jfh_status jfh_generate_draft(jfh_engine * engine, const int32_t * prompt, uint32_t n_prompt, uint32_t max_tokens,
                              uint32_t draft_max, jfh_draft_propose_fn propose, void * user, int32_t * out_tokens,
                              uint32_t * out_count, jfh_generation_stats * stats);

/* Continuous-batching generation: n_requests GenerationRunner loops (as
 * jfh_generate, one thread each) over one HIP stage executor wrapped in the
 * ContinuousBatchingExecutor the reference worker installs when
 * --decode-batch-size > 1 (runtime/engine/builtin_inference_engines.cpp:117-123;
 * batching: runtime/pipeline_parallel/continuous_batching_executor.cpp:14-200):
 * concurrent decode steps are coalesced, up to n_requests per step, waiting at
 * most batch_wait_us for a batch to fill, into one multi-sequence forward.
 * prompts holds the requests' prompts back to back (prompt_lengths[i] ids
 * each); out_tokens receives max_tokens slots per request, out_counts and
 * stats (optional) one entry per request. The runners' decode phases start
 * together once every prefill is done; decode_wall_ms (optional) is the time
 * from that start until the last runner has read its last token (its session
 * is closed afterwards, outside that time). n_requests 1..8. */
jfh_status jfh_generate_concurrent(jfh_engine * engine, uint32_t n_requests, const int32_t * prompts,
                                   const uint32_t * prompt_lengths, uint32_t max_tokens, uint32_t draft_max,
                                   uint32_t max_ngram, uint32_t min_ngram, uint32_t batch_wait_us,
                                   int32_t * out_tokens, uint32_t * out_counts, jfh_generation_stats * stats,
                                   double * decode_wall_ms);

#ifdef __cplusplus
}
#endif

#endif
