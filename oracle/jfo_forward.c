/*
 * jfo_forward.c -- CPU restatement of the native Qwen2 stage forward.
 *
 * TEST INFRASTRUCTURE ONLY (the checker); see jfo.h.
 *
 * Follows runtime/engines/native/src/qwen2_architecture.cpp op for op:
 *   embedding get_rows (564-568) -> per layer [rms_norm*gain (373-376),
 *   q/k/v linear + bias (394-396), NEOX rope on q and k (401-402, 499-506),
 *   K/V rows written to the F16 cache at the step's positions (405-424),
 *   causal attention softmax(q.k * hd^-1/2 + mask) v over the cache
 *   (438-464, mask 697-708), output linear (469), residual add (573),
 *   rms_norm*gain, up/gate linear, silu(gate)*up, down linear (508-520),
 *   residual add (576)] -> rows selected for output (584) -> output norm ->
 *   head linear (+ bias if present, 378-384) -> argmax (594).
 * Float rounding points kept from the reference: K/V are stored as binary16;
 * rms_norm scale is 1/sqrtf(mean + eps) applied as (x*scale)*gain; the
 * attention scale is 1/sqrtf(head_dim) in float; silu(x) = x/(1+expf(-x)).
 * Accumulations are in double, which is more precise than the reference.
 */
#include "jfo.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct jfo_session {
    const jfo_model * m;
    int32_t capacity;
    int32_t mode;
    int32_t threads;
    int32_t pos;
    int32_t prefill_pos;
    int32_t head_dim;
    uint16_t * k; /* [layer][kv_head][capacity][head_dim] */
    uint16_t * v;
    float * rope; /* [capacity][head_dim]: cos, sin per pair */
};

void jfo_rope_table(float base, int32_t head_dim, int32_t pos_begin, int32_t pos_count, float * out) {
    /* ggml rope cache: theta starts at the position and is multiplied by
     * theta_scale = base^(-2/n_dims) once per rotated pair. */
    const float theta_scale = powf(base, -2.0f / (float) head_dim);
    for (int32_t p = 0; p < pos_count; ++p) {
        float theta = (float) (pos_begin + p);
        float * row = out + (size_t) p * head_dim;
        for (int32_t i = 0; i < head_dim / 2; ++i) {
            row[2 * i] = cosf(theta);
            row[2 * i + 1] = sinf(theta);
            theta *= theta_scale;
        }
    }
}

int jfo_matmul(int type, const void * w, int64_t n, int64_t rows,
               const float * x, int64_t tokens, float * y, int mode, int threads) {
    uint32_t be = 0, bb = 0;
    if (!jfo_type_block(type, &be, &bb) || n % be != 0) return -1;
    const size_t row_bytes = (size_t) (n / be) * bb;
    const int quantized = mode == JFO_MODE_Q8 && type != JFO_F32 && type != JFO_F16;
    const int blk = jfo_act_block(type);
    int8_t * q = NULL;
    float * d = NULL;
    int16_t * s16 = NULL;
    if (quantized) {
        if (n % 256 != 0) return -1;
        q = malloc((size_t) (tokens * n));
        d = malloc(sizeof(float) * (size_t) (tokens * n / blk));
        s16 = malloc(sizeof(int16_t) * (size_t) (tokens * n / 16));
        if (!q || !d || !s16) {
            free(q); free(d); free(s16);
            return -1;
        }
        for (int64_t t = 0; t < tokens; ++t) {
            jfo_quantize_act_blk(x + t * n, n, blk, q + t * n, d + t * n / blk, s16 + t * n / 16);
        }
    }
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t * row = (const uint8_t *) w + (size_t) r * row_bytes;
        for (int64_t t = 0; t < tokens; ++t) {
            const double v = quantized
                ? jfo_vec_dot_q8_blk(type, row, q + t * n, d + t * n / blk, s16 + t * n / 16, n, blk)
                : jfo_vec_dot_f32(type, row, x + t * n, n);
            y[t * rows + r] = (float) v;
        }
    }
    (void) threads;
    free(q);
    free(d);
    free(s16);
    return 0;
}

int jfo_matmul_q8_blk(int type, const void * w, int64_t n, int64_t rows, const int8_t * q, const float * d,
                      const int16_t * s16, int64_t tokens, float * y, int blk, int threads) {
    uint32_t be = 0, bb = 0;
    if (!jfo_type_block(type, &be, &bb) || n % 256 != 0 || type == JFO_F32 || type == JFO_F16) return -1;
    if (blk != jfo_act_block(type)) return -1;
    const size_t row_bytes = (size_t) (n / be) * bb;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t * row = (const uint8_t *) w + (size_t) r * row_bytes;
        for (int64_t t = 0; t < tokens; ++t) {
            y[t * rows + r] =
                (float) jfo_vec_dot_q8_blk(type, row, q + t * n, d + t * n / blk, s16 + t * n / 16, n, blk);
        }
    }
    (void) threads;
    return 0;
}

int jfo_matmul_q8(int type, const void * w, int64_t n, int64_t rows, const int8_t * q, const float * d,
                  const int16_t * s16, int64_t tokens, float * y, int threads) {
    return jfo_matmul_q8_blk(type, w, n, rows, q, d, s16, tokens, y, jfo_act_block(type), threads);
}

static float rms_scale(const float * x, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double) x[i] * (double) x[i];
    const float mean = (float) (sum / (double) n);
    return 1.0f / sqrtf(mean + eps);
}

void jfo_quantize_act_normed_blk(const float * x, const float * gain, int64_t n, float eps, int blk, int8_t * q,
                                 float * d, int16_t * s16) {
    float * v = calloc((size_t) n, sizeof(float));
    if (!v) return;
    for (int64_t i = 0; i < n; ++i) v[i] = x[i] * gain[i];
    /* the codes of x * gain with the unrounded block scales, then each scale times the row's 1/rms */
    const float scale = rms_scale(x, n, eps);
    if (blk == 32) {
        for (int64_t b = 0; b < n / 32; ++b) {
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const float a = fabsf(v[b * 32 + i]);
                if (a > amax) amax = a;
            }
            const float db = amax / 127.0f;
            const float id = db > 0.0f ? 1.0f / db : 0.0f;
            for (int i = 0; i < 32; ++i) {
                float r = roundf(v[b * 32 + i] * id);
                if (r > 127.0f) r = 127.0f;
                if (r < -127.0f) r = -127.0f;
                q[b * 32 + i] = (int8_t) r;
            }
            d[b] = jfo_f16_to_f32(jfo_f32_to_f16(db * scale));
        }
        for (int64_t g = 0; g < n / 16; ++g) {
            int sum = 0;
            for (int i = 0; i < 16; ++i) sum += q[g * 16 + i];
            s16[g] = (int16_t) sum;
        }
    } else {
        jfo_quantize_act_blk(v, n, 256, q, d, s16);
        for (int64_t b = 0; b < n / 256; ++b) d[b] = d[b] * scale;
    }
    free(v);
}

void jfo_quantize_act_normed(const float * x, const float * gain, int64_t n, float eps, int8_t * q, float * d,
                             int16_t * s16) {
    jfo_quantize_act_normed_blk(x, gain, n, eps, 256, q, d, s16);
}

static void rms_norm(const float * x, const jfo_tensor * gain, int64_t n, float eps, float * out) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double) x[i] * (double) x[i];
    const float mean = (float) (sum / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (gain->type == JFO_F32) {
        const float * gv = (const float *) gain->data;
        for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * scale) * gv[i];
        return;
    }
    float * gv = malloc(sizeof(float) * (size_t) n);
    jfo_dequantize_row(gain->type, gain->data, gv, n);
    for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * scale) * gv[i];
    free(gv);
}

static void add_bias(float * y, const jfo_tensor * b, int64_t tokens, int64_t n) {
    if (b->data == NULL) return;
    float * tmp = malloc(sizeof(float) * (size_t) n);
    jfo_dequantize_row(b->type, b->data, tmp, n);
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t i = 0; i < n; ++i) y[t * n + i] += tmp[i];
    }
    free(tmp);
}

/*
 * Input rows of one or more matmuls. In JFO_MODE_Q8 they are quantized the
 * way the HIP engine stages them, once per activation block size a consumer
 * needs (jfo_act_block: 32 values for Q8_0 weights, 256 for the K-quants):
 * plain rows as jfo_quantize_act_blk; rows behind an RMSNorm as
 * jfo_quantize_act_normed_blk (codes of x*gain, block scales times the row's
 * 1/rms). Float weights and JFO_MODE_EXACT use the float rows
 * ((x*rms_scale)*gain for normed inputs, as the reference graph).
 */
typedef struct act_q8 {
    int8_t * q;
    float * d;
    int16_t * s16;
} act_q8;

typedef struct act_rows {
    const float * x;    /* float rows (normed when a gain was given) */
    const float * raw;  /* the rows before the norm */
    float * gain;       /* dequantized gain, NULL for plain rows */
    int quantize;       /* JFO_MODE_Q8 session */
    act_q8 blk256, blk32;
    int64_t n, tokens;
} act_rows;

static void act_prepare(const jfo_session * s, act_rows * a, const float * x, const jfo_tensor * gain, int64_t n,
                        int64_t tokens, float * xn) {
    memset(a, 0, sizeof(*a));
    a->n = n;
    a->tokens = tokens;
    a->raw = x;
    a->quantize = s->mode == JFO_MODE_Q8 && n % 256 == 0;
    if (gain) {
        for (int64_t t = 0; t < tokens; ++t) rms_norm(x + t * n, gain, n, s->m->rms_eps, xn + t * n);
        a->x = xn;
        a->gain = malloc(sizeof(float) * (size_t) n);
        jfo_dequantize_row(gain->type, gain->data, a->gain, n);
    } else {
        a->x = x;
    }
}

/* The rows quantized in blocks of blk values (computed on first use). */
static const act_q8 * act_quantized(const jfo_session * s, act_rows * a, int blk) {
    act_q8 * v = blk == 32 ? &a->blk32 : &a->blk256;
    if (v->q) return v;
    const int64_t n = a->n, tokens = a->tokens;
    v->q = malloc((size_t) (tokens * n));
    v->d = malloc(sizeof(float) * (size_t) (tokens * n / blk));
    v->s16 = malloc(sizeof(int16_t) * (size_t) (tokens * n / 16));
    for (int64_t t = 0; t < tokens; ++t) {
        if (a->gain) {
            jfo_quantize_act_normed_blk(a->raw + t * n, a->gain, n, s->m->rms_eps, blk, v->q + t * n,
                                        v->d + t * n / blk, v->s16 + t * n / 16);
        } else {
            jfo_quantize_act_blk(a->raw + t * n, n, blk, v->q + t * n, v->d + t * n / blk, v->s16 + t * n / 16);
        }
    }
    return v;
}

static void act_release(act_rows * a) {
    act_q8 * v[2] = {&a->blk256, &a->blk32};
    for (int i = 0; i < 2; ++i) {
        free(v[i]->q);
        free(v[i]->d);
        free(v[i]->s16);
        v[i]->q = NULL;
        v[i]->d = NULL;
        v[i]->s16 = NULL;
    }
    free(a->gain);
    a->gain = NULL;
}

static int linear(const jfo_session * s, const jfo_tensor * w, act_rows * a, float * y) {
    const int float_weights = w->type == JFO_F32 || w->type == JFO_F16;
    if (a->quantize && !float_weights) {
        const int blk = jfo_act_block(w->type);
        const act_q8 * v = act_quantized(s, a, blk);
        return jfo_matmul_q8_blk(w->type, w->data, w->ne0, w->ne1, v->q, v->d, v->s16, a->tokens, y, blk,
                                 s->threads);
    }
    return jfo_matmul(w->type, w->data, w->ne0, w->ne1, a->x, a->tokens, y, JFO_MODE_EXACT, s->threads);
}

static void rope_rows(const jfo_session * s, float * x, int64_t tokens, int32_t heads, int32_t pos0) {
    const int32_t hd = s->head_dim, half = hd / 2;
    for (int64_t t = 0; t < tokens; ++t) {
        const float * cs = s->rope + (size_t) (pos0 + t) * hd;
        for (int32_t h = 0; h < heads; ++h) {
            float * v = x + (t * heads + h) * hd;
            for (int32_t i = 0; i < half; ++i) {
                const float c = cs[2 * i], sn = cs[2 * i + 1];
                const float x0 = v[i], x1 = v[i + half];
                v[i] = x0 * c - x1 * sn;
                v[i + half] = x0 * sn + x1 * c;
            }
        }
    }
}

jfo_session * jfo_session_create(const jfo_model * model, int32_t capacity, int32_t mode, int32_t threads) {
    if (model == NULL || capacity <= 0 || capacity > model->n_ctx || model->n_head <= 0 ||
        model->n_head_kv <= 0 || model->n_embd % model->n_head != 0 ||
        model->n_head % model->n_head_kv != 0) {
        return NULL;
    }
    jfo_session * s = calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->m = model;
    s->capacity = capacity;
    s->mode = mode;
    s->threads = threads;
    s->head_dim = model->n_embd / model->n_head;
    const size_t per_layer = (size_t) model->n_head_kv * capacity * s->head_dim;
    s->k = calloc(per_layer * model->n_layer, sizeof(uint16_t));
    s->v = calloc(per_layer * model->n_layer, sizeof(uint16_t));
    s->rope = malloc(sizeof(float) * (size_t) capacity * s->head_dim);
    if (!s->k || !s->v || !s->rope) {
        jfo_session_destroy(s);
        return NULL;
    }
    jfo_rope_table(model->rope_base, s->head_dim, 0, capacity, s->rope);
    return s;
}

void jfo_session_destroy(jfo_session * s) {
    if (!s) return;
    free(s->k);
    free(s->v);
    free(s->rope);
    free(s);
}

int32_t jfo_session_position(const jfo_session * s) { return s->pos; }

int32_t jfo_session_rollback(jfo_session * s, int32_t n) {
    /* qwen2_architecture.cpp:818-823: KV rows are left in place and overwritten later. */
    if (n <= 0 || n > s->pos - s->prefill_pos) return -1;
    s->pos -= n;
    return 0;
}

static uint16_t * cache_row(const jfo_session * s, uint16_t * base, int32_t layer, int32_t kvh, int32_t p) {
    const jfo_model * m = s->m;
    return base + (((size_t) layer * m->n_head_kv + kvh) * s->capacity + p) * s->head_dim;
}

static void attention(const jfo_session * s, int32_t layer, const float * q, int64_t tokens,
                      int32_t pos0, float * out) {
    const jfo_model * m = s->m;
    const int32_t hd = s->head_dim, group = m->n_head / m->n_head_kv;
    const float scale = 1.0f / sqrtf((float) hd);
#ifdef _OPENMP
#pragma omp parallel for collapse(2) num_threads(s->threads > 0 ? s->threads : 1) schedule(static)
#endif
    for (int64_t t = 0; t < tokens; ++t) {
        for (int32_t h = 0; h < m->n_head; ++h) {
            const int32_t kvh = h / group;
            const int32_t keys = pos0 + (int32_t) t + 1; /* causal: keys <= query position */
            const float * qv = q + (t * m->n_head + h) * hd;
            double * score = malloc(sizeof(double) * (size_t) keys);
            double mx = -INFINITY;
            for (int32_t j = 0; j < keys; ++j) {
                const uint16_t * kr = cache_row(s, s->k, layer, kvh, j);
                double dot = 0.0;
                for (int32_t d = 0; d < hd; ++d) dot += (double) qv[d] * jfo_f16_to_f32(kr[d]);
                score[j] = dot * scale;
                if (score[j] > mx) mx = score[j];
            }
            double denom = 0.0;
            for (int32_t j = 0; j < keys; ++j) {
                score[j] = exp(score[j] - mx);
                denom += score[j];
            }
            float * o = out + (t * m->n_head + h) * hd;
            for (int32_t d = 0; d < hd; ++d) {
                double acc = 0.0;
                for (int32_t j = 0; j < keys; ++j) {
                    acc += score[j] * jfo_f16_to_f32(cache_row(s, s->v, layer, kvh, j)[d]);
                }
                o[d] = (float) (acc / denom);
            }
            free(score);
        }
    }
}

int32_t jfo_session_forward(jfo_session * s, const int32_t * tokens, int32_t n,
                            int32_t logits_rows, float * logits, int32_t * argmax_out) {
    if (tokens == NULL) return -1;
    return jfo_session_forward_range(s, tokens, NULL, n, 0, s->m->n_layer, NULL, logits_rows, logits, argmax_out);
}

/*
 * One pipeline stage's forward over layers [layer_begin, layer_end):
 * Qwen2Session::prefill_stage_* / decode_stage_* (qwen2_architecture.cpp:
 * 909-947, 977-1027) build the same per-layer graph as the full model over
 * the stage's LayerRange (model_architecture.hpp:15-21); the first stage
 * embeds token ids, a later one starts from the previous stage's residual
 * rows, and only the last one applies the output norm and head.
 */
int32_t jfo_session_forward_range(jfo_session * s, const int32_t * tokens, const float * rows_in, int32_t n,
                                  int32_t layer_begin, int32_t layer_end, float * rows_out,
                                  int32_t logits_rows, float * logits, int32_t * argmax_out) {
    const jfo_model * m = s->m;
    if (n <= 0 || (logits_rows != 0 && logits_rows != 1 && logits_rows != n)) return -1;
    if (layer_begin < 0 || layer_begin >= layer_end || layer_end > m->n_layer) return -1;
    if ((layer_begin == 0) != (tokens != NULL) || (tokens == NULL) == (rows_in == NULL)) return -1;
    if (logits_rows > 0 && layer_end != m->n_layer) return -1;
    if ((int64_t) s->pos + n > s->capacity) return -2;
    for (int32_t t = 0; tokens && t < n; ++t) {
        if (tokens[t] < 0 || tokens[t] >= m->n_vocab) return -3;
    }
    const int64_t H = m->n_embd, F = m->n_ff, hd = s->head_dim;
    const int64_t kv = (int64_t) m->n_head_kv * hd;
    const int32_t pos0 = s->pos;
    float * h = malloc(sizeof(float) * (size_t) (n * H));
    float * xn = malloc(sizeof(float) * (size_t) (n * H));
    float * q = malloc(sizeof(float) * (size_t) (n * H));
    float * k = malloc(sizeof(float) * (size_t) (n * kv));
    float * v = malloc(sizeof(float) * (size_t) (n * kv));
    float * att = malloc(sizeof(float) * (size_t) (n * H));
    float * o = malloc(sizeof(float) * (size_t) (n * H));
    float * g = malloc(sizeof(float) * (size_t) (n * F));
    float * u = malloc(sizeof(float) * (size_t) (n * F));
    if (!h || !xn || !q || !k || !v || !att || !o || !g || !u) {
        free(h); free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
        return -1;
    }
    /* embedding rows (first stage) or the previous stage's residual rows */
    if (rows_in) {
        memcpy(h, rows_in, sizeof(float) * (size_t) (n * H));
    } else {
        uint32_t be = 0, bb = 0;
        jfo_type_block(m->tok_embd.type, &be, &bb);
        const size_t row_bytes = (size_t) (H / be) * bb;
        for (int32_t t = 0; t < n; ++t) {
            jfo_dequantize_row(m->tok_embd.type,
                               (const uint8_t *) m->tok_embd.data + (size_t) tokens[t] * row_bytes,
                               h + t * H, H);
        }
    }
    for (int32_t l = layer_begin; l < layer_end; ++l) {
        if (rows_out) memcpy(rows_out + (size_t) (l - layer_begin) * n * H, h, sizeof(float) * (size_t) (n * H));
        const jfo_layer * L = &m->layers[l];
        act_rows in;
        act_prepare(s, &in, h, &L->attn_norm, H, n, xn);
        linear(s, &L->wq, &in, q);
        add_bias(q, &L->bq, n, H);
        linear(s, &L->wk, &in, k);
        add_bias(k, &L->bk, n, kv);
        linear(s, &L->wv, &in, v);
        add_bias(v, &L->bv, n, kv);
        act_release(&in);
        rope_rows(s, q, n, m->n_head, pos0);
        rope_rows(s, k, n, m->n_head_kv, pos0);
        for (int32_t t = 0; t < n; ++t) {
            for (int32_t kh = 0; kh < m->n_head_kv; ++kh) {
                uint16_t * kr = cache_row(s, s->k, l, kh, pos0 + t);
                uint16_t * vr = cache_row(s, s->v, l, kh, pos0 + t);
                for (int64_t d = 0; d < hd; ++d) {
                    kr[d] = jfo_f32_to_f16(k[t * kv + kh * hd + d]);
                    vr[d] = jfo_f32_to_f16(v[t * kv + kh * hd + d]);
                }
            }
        }
        attention(s, l, q, n, pos0, att);
        act_prepare(s, &in, att, NULL, H, n, NULL);
        linear(s, &L->wo, &in, o);
        act_release(&in);
        for (int64_t i = 0; i < n * H; ++i) h[i] += o[i];
        act_prepare(s, &in, h, &L->ffn_norm, H, n, xn);
        linear(s, &L->w_up, &in, u);
        linear(s, &L->w_gate, &in, g);
        act_release(&in);
        for (int64_t i = 0; i < n * F; ++i) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
        act_prepare(s, &in, g, NULL, F, n, NULL);
        linear(s, &L->w_down, &in, o);
        act_release(&in);
        for (int64_t i = 0; i < n * H; ++i) h[i] += o[i];
    }
    if (rows_out) {
        memcpy(rows_out + (size_t) (layer_end - layer_begin) * n * H, h, sizeof(float) * (size_t) (n * H));
    }
    if (logits_rows > 0) {
        const int32_t first = n - logits_rows;
        const int64_t V = m->n_vocab;
        float * lg = logits ? logits : malloc(sizeof(float) * (size_t) (logits_rows * V));
        act_rows in;
        act_prepare(s, &in, h + (size_t) first * H, &m->output_norm, H, logits_rows, xn);
        linear(s, &m->output, &in, lg);
        act_release(&in);
        add_bias(lg, &m->output_bias, logits_rows, V);
        if (argmax_out) {
            for (int32_t r = 0; r < logits_rows; ++r) argmax_out[r] = jfo_argmax(lg + r * V, V);
        }
        if (!logits) free(lg);
    }
    if (s->pos == 0) s->prefill_pos = n;
    s->pos += n;
    free(h); free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
    return 0;
}

int32_t jfo_session_fill_kv(jfo_session * s, int32_t n, uint64_t seed) {
    if (n <= 0 || n > s->capacity) return -1;
    const jfo_model * m = s->m;
    uint64_t state = seed ? seed : 0x9E3779B97F4A7C15ull;
    for (int32_t l = 0; l < m->n_layer; ++l) {
        for (int32_t kh = 0; kh < m->n_head_kv; ++kh) {
            for (int32_t p = 0; p < n; ++p) {
                uint16_t * kr = cache_row(s, s->k, l, kh, p);
                uint16_t * vr = cache_row(s, s->v, l, kh, p);
                for (int32_t d = 0; d < s->head_dim; ++d) {
                    state ^= state << 13; state ^= state >> 7; state ^= state << 17;
                    kr[d] = jfo_f32_to_f16((float) ((int32_t) (state & 0xFFFF) - 32768) / 32768.0f);
                    vr[d] = jfo_f32_to_f16((float) ((int32_t) ((state >> 16) & 0xFFFF) - 32768) / 32768.0f);
                }
            }
        }
    }
    s->pos = n;
    s->prefill_pos = n;
    return 0;
}

int32_t jfo_session_read_kv(const jfo_session * s, int32_t layer, int32_t n, uint16_t * k, uint16_t * v) {
    const jfo_model * m = s->m;
    if (layer < 0 || layer >= m->n_layer || n < 0 || n > s->capacity) return -1;
    for (int32_t kh = 0; kh < m->n_head_kv; ++kh) {
        memcpy(k + (size_t) kh * n * s->head_dim, cache_row(s, s->k, layer, kh, 0),
               sizeof(uint16_t) * (size_t) n * s->head_dim);
        memcpy(v + (size_t) kh * n * s->head_dim, cache_row(s, s->v, layer, kh, 0),
               sizeof(uint16_t) * (size_t) n * s->head_dim);
    }
    return 0;
}

int32_t jfo_session_write_kv(jfo_session * s, int32_t layer, int32_t n, const uint16_t * k, const uint16_t * v) {
    const jfo_model * m = s->m;
    if (layer < 0 || layer >= m->n_layer || n < 0 || n > s->capacity) return -1;
    for (int32_t kh = 0; kh < m->n_head_kv; ++kh) {
        memcpy(cache_row(s, s->k, layer, kh, 0), k + (size_t) kh * n * s->head_dim,
               sizeof(uint16_t) * (size_t) n * s->head_dim);
        memcpy(cache_row(s, s->v, layer, kh, 0), v + (size_t) kh * n * s->head_dim,
               sizeof(uint16_t) * (size_t) n * s->head_dim);
    }
    return 0;
}
