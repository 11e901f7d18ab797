/*
 * jfo_quant.c -- block formats, dequantization and quantized dot products.
 *
 * TEST INFRASTRUCTURE ONLY (the checker); see jfo.h.
 *
 * Block layouts are GGML's public ones, stored verbatim by the reference
 * (runtime/engines/native/src/tensor_store.cpp:185-196 copies bytes as-is;
 * geometry table runtime/engines/native/src/engine.c:292-303). The GGML
 * sources are not in the reference checkout (llama.cpp pinned at
 * bf2c86ddc0685f580595954056c2e77ebabfab4f, Makefile:28-30), so each
 * dequantizer below restates the published layout; tests pin them with
 * closed-form blocks and exactness invariants.
 */
#include "jfo.h"

#include <math.h>
#include <string.h>

/* IEEE binary16 -> binary32, exact. */
float jfo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            /* subnormal: renormalize */
            int e = -1;
            do {
                ++e;
                mantissa <<= 1;
            } while ((mantissa & 0x400u) == 0);
            mantissa &= 0x3FFu;
            bits = sign | ((uint32_t) (127 - 15 - e) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1Fu) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + (127 - 15)) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* IEEE binary32 -> binary16, round to nearest even (the hardware conversion). */
uint16_t jfo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof(x));
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t abs = x & 0x7FFFFFFFu;
    if (abs >= 0x7F800000u) { /* inf or nan */
        return (uint16_t) (sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));
    }
    if (abs >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t) (sign | 0x7C00u);
    }
    if (abs < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        if (abs < 0x33000000u) return sign; /* < 2^-25 rounds to zero */
        const uint32_t e = abs >> 23;
        const uint32_t m = (abs & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e; /* 14 + (113 - e) - 1 + 1 */
        uint32_t half = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t mid = 1u << (shift - 1u);
        if (rem > mid || (rem == mid && (half & 1u))) ++half;
        return (uint16_t) (sign | half);
    }
    uint32_t half = ((abs >> 13) - (112u << 10));
    const uint32_t rem = abs & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;
    return (uint16_t) (sign | half);
}

int jfo_type_block(int type, uint32_t * block_elements, uint32_t * block_bytes) {
    uint32_t e = 0, b = 0;
    switch (type) {
    case JFO_F32: e = 1; b = 4; break;
    case JFO_F16: e = 1; b = 2; break;
    case JFO_Q8_0: e = 32; b = 34; break;
    case JFO_Q2_K: e = 256; b = 84; break;
    case JFO_Q4_K: e = 256; b = 144; break;
    case JFO_Q6_K: e = 256; b = 210; break;
    default: return 0;
    }
    if (block_elements) *block_elements = e;
    if (block_bytes) *block_bytes = b;
    return 1;
}

static float f16_at(const uint8_t * p) {
    return jfo_f16_to_f32((uint16_t) (p[0] | (p[1] << 8)));
}

/*
 * Q4_K: 6-bit scale and min of sub-block j (0..7) from the 12 packed bytes.
 * j < 4: low 6 bits of bytes j and j+4; j >= 4: a nibble of byte j+4 plus the
 * top two bits of bytes j-4 (scale) and j (min).
 */
static void q4k_scale_min(const uint8_t * s, int j, int * sc, int * m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K element i (0..255) of a block: nibble and sub-block. */
static int q4k_nibble(const uint8_t * qs, int i, int * sub) {
    const int pair = i / 64, within = i % 64;
    const uint8_t byte = qs[pair * 32 + (within % 32)];
    *sub = pair * 2 + within / 32;
    return within < 32 ? (byte & 0xF) : (byte >> 4);
}

/* Q2_K element i: 2-bit value and its 16-value group (scale byte index). */
static int q2k_value(const uint8_t * qs, int i, int * group) {
    const int half = i / 128, within = i % 128;
    const int shift_index = within / 32, part = (within % 32) / 16, l = within % 16;
    *group = half * 8 + shift_index * 2 + part;
    return (qs[half * 32 + part * 16 + l] >> (2 * shift_index)) & 3;
}

/* Q6_K element i: 6-bit unsigned value (0..63) and its 16-value group. */
static int q6k_value(const uint8_t * ql, const uint8_t * qh, int i, int * group) {
    const int half = i / 128, within = i % 128;
    const int quarter = within / 32, l = within % 32;
    const uint8_t * lo = ql + half * 64;
    const uint8_t * hi = qh + half * 32;
    int low;
    switch (quarter) {
    case 0: low = lo[l] & 0xF; break;
    case 1: low = lo[l + 32] & 0xF; break;
    case 2: low = lo[l] >> 4; break;
    default: low = lo[l + 32] >> 4; break;
    }
    const int high = (hi[l] >> (2 * quarter)) & 3;
    *group = half * 8 + l / 16 + 2 * quarter;
    return low | (high << 4);
}

int jfo_dequantize_row(int type, const void * src, float * dst, int64_t n) {
    const uint8_t * p = (const uint8_t *) src;
    uint32_t be = 0, bb = 0;
    if (!jfo_type_block(type, &be, &bb) || n % be != 0) return -1;
    const int64_t blocks = n / be;
    switch (type) {
    case JFO_F32:
        memcpy(dst, src, (size_t) n * sizeof(float));
        return 0;
    case JFO_F16:
        for (int64_t i = 0; i < n; ++i) dst[i] = f16_at(p + 2 * i);
        return 0;
    case JFO_Q8_0:
        for (int64_t b = 0; b < blocks; ++b, p += 34) {
            const float d = f16_at(p);
            for (int i = 0; i < 32; ++i) dst[b * 32 + i] = (float) (int8_t) p[2 + i] * d;
        }
        return 0;
    case JFO_Q4_K:
        for (int64_t b = 0; b < blocks; ++b, p += 144) {
            const float d = f16_at(p), dmin = f16_at(p + 2);
            for (int i = 0; i < 256; ++i) {
                int sub, sc, m;
                const int q = q4k_nibble(p + 16, i, &sub);
                q4k_scale_min(p + 4, sub, &sc, &m);
                const float d1 = d * (float) sc, m1 = dmin * (float) m;
                dst[b * 256 + i] = d1 * (float) q - m1;
            }
        }
        return 0;
    case JFO_Q2_K:
        for (int64_t b = 0; b < blocks; ++b, p += 84) {
            const float d = f16_at(p + 80), dmin = f16_at(p + 82);
            for (int i = 0; i < 256; ++i) {
                int group;
                const int q = q2k_value(p + 16, i, &group);
                const uint8_t s = p[group];
                const float dl = d * (float) (s & 0xF), ml = dmin * (float) (s >> 4);
                dst[b * 256 + i] = dl * (float) q - ml;
            }
        }
        return 0;
    case JFO_Q6_K:
        for (int64_t b = 0; b < blocks; ++b, p += 210) {
            const float d = f16_at(p + 208);
            const int8_t * scales = (const int8_t *) (p + 192);
            for (int i = 0; i < 256; ++i) {
                int group;
                const int q = q6k_value(p, p + 128, i, &group) - 32;
                /* evaluated left to right: (d * scale) * q */
                dst[b * 256 + i] = d * (float) scales[group] * (float) q;
            }
        }
        return 0;
    default:
        return -1;
    }
}

int jfo_act_block(int type) { return type == JFO_Q8_0 ? 32 : 256; }

void jfo_quantize_act_blk(const float * x, int64_t n, int blk, int8_t * q, float * d, int16_t * s16) {
    for (int64_t b = 0; b < n / blk; ++b) {
        const float * xb = x + b * blk;
        float amax = 0.0f;
        for (int i = 0; i < blk; ++i) {
            const float a = fabsf(xb[i]);
            if (a > amax) amax = a;
        }
        const float db = amax / 127.0f;
        const float id = db > 0.0f ? 1.0f / db : 0.0f;
        for (int i = 0; i < blk; ++i) {
            float r = roundf(xb[i] * id);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[b * blk + i] = (int8_t) r;
        }
        /* 32-value blocks store their scale as f16 (GGML's q8_0 / q8_1 block) */
        d[b] = blk == 32 ? jfo_f16_to_f32(jfo_f32_to_f16(db)) : db;
    }
    for (int64_t g = 0; g < n / 16; ++g) {
        int sum = 0;
        for (int i = 0; i < 16; ++i) sum += q[g * 16 + i];
        s16[g] = (int16_t) sum;
    }
}

void jfo_quantize_act(const float * x, int64_t n, int8_t * q, float * d, int16_t * s16) {
    jfo_quantize_act_blk(x, n, 256, q, d, s16);
}

/*
 * Unpacks the raw unsigned quant values of one K-quant block into v[256]
 * (Q4_K: 0..15, Q2_K: 0..3, Q6_K: 0..63). Element i of Q2_K and Q6_K belongs
 * to 16-value group i / 16; element i of Q4_K to 32-value sub-block i / 32.
 */
static void unpack_kquant(int type, const uint8_t * p, uint8_t * v) {
    int unused;
    for (int i = 0; i < 256; ++i) {
        switch (type) {
        case JFO_Q4_K: v[i] = (uint8_t) q4k_nibble(p + 16, i, &unused); break;
        case JFO_Q2_K: v[i] = (uint8_t) q2k_value(p + 16, i, &unused); break;
        default: v[i] = (uint8_t) q6k_value(p, p + 128, i, &unused); break;
        }
    }
}

/* Dot of one Q8_0 row with activation blocks of 32 values (jfo.h). */
static double vec_dot_q8_32(int type, const uint8_t * p, const int8_t * q, const float * d, int64_t n) {
    double sum = 0.0;
    if (type != JFO_Q8_0) return 0.0;
    for (int64_t b = 0; b < n / 32; ++b, p += 34) {
        int dot = 0;
        for (int i = 0; i < 32; ++i) dot += (int) (int8_t) p[2 + i] * q[b * 32 + i];
        sum += (double) d[b] * (double) f16_at(p) * (double) dot;
    }
    return sum;
}

double jfo_vec_dot_q8_blk(int type, const void * row, const int8_t * q, const float * d, const int16_t * s16,
                          int64_t n, int blk) {
    const uint8_t * p = (const uint8_t *) row;
    if (blk != jfo_act_block(type)) return 0.0;
    if (blk == 32) return vec_dot_q8_32(type, p, q, d, n);
    uint8_t v[256];
    double sum = 0.0;
    switch (type) {
    case JFO_Q4_K:
        for (int64_t b = 0; b < n / 256; ++b, p += 144) {
            const double dw = f16_at(p), dmin = f16_at(p + 2);
            unpack_kquant(type, p, v);
            int64_t isum = 0, msum = 0;
            for (int sub = 0; sub < 8; ++sub) {
                int sc, m, dot = 0;
                q4k_scale_min(p + 4, sub, &sc, &m);
                for (int l = 0; l < 32; ++l) dot += v[sub * 32 + l] * q[b * 256 + sub * 32 + l];
                isum += (int64_t) sc * dot;
                msum += (int64_t) m * (s16[b * 16 + 2 * sub] + s16[b * 16 + 2 * sub + 1]);
            }
            sum += (double) d[b] * (dw * (double) isum - dmin * (double) msum);
        }
        return sum;
    case JFO_Q2_K:
        for (int64_t b = 0; b < n / 256; ++b, p += 84) {
            const double dw = f16_at(p + 80), dmin = f16_at(p + 82);
            unpack_kquant(type, p, v);
            int64_t isum = 0, msum = 0;
            for (int g = 0; g < 16; ++g) {
                int dot = 0;
                for (int l = 0; l < 16; ++l) dot += v[g * 16 + l] * q[b * 256 + g * 16 + l];
                isum += (int64_t) (p[g] & 0xF) * dot;
                msum += (int64_t) (p[g] >> 4) * s16[b * 16 + g];
            }
            sum += (double) d[b] * (dw * (double) isum - dmin * (double) msum);
        }
        return sum;
    case JFO_Q6_K:
        for (int64_t b = 0; b < n / 256; ++b, p += 210) {
            const double dw = f16_at(p + 208);
            const int8_t * scales = (const int8_t *) (p + 192);
            unpack_kquant(type, p, v);
            int64_t isum = 0;
            for (int g = 0; g < 16; ++g) {
                int dot = 0;
                for (int l = 0; l < 16; ++l) dot += v[g * 16 + l] * q[b * 256 + g * 16 + l];
                isum += (int64_t) scales[g] * (dot - 32 * s16[b * 16 + g]);
            }
            sum += (double) d[b] * dw * (double) isum;
        }
        return sum;
    default:
        return 0.0;
    }
}


double jfo_vec_dot_q8(int type, const void * row, const int8_t * q, const float * d, const int16_t * s16, int64_t n) {
    return jfo_vec_dot_q8_blk(type, row, q, d, s16, n, jfo_act_block(type));
}

double jfo_vec_dot_f32(int type, const void * row, const float * x, int64_t n) {
    float tmp[256];
    uint32_t be = 0, bb = 0;
    if (!jfo_type_block(type, &be, &bb)) return 0.0;
    const uint8_t * p = (const uint8_t *) row;
    double sum = 0.0;
    if (type == JFO_F32) {
        const float * w = (const float *) row;
        for (int64_t i = 0; i < n; ++i) sum += (double) w[i] * x[i];
        return sum;
    }
    if (type == JFO_F16) {
        for (int64_t i = 0; i < n; ++i) sum += (double) f16_at(p + 2 * i) * x[i];
        return sum;
    }
    for (int64_t b = 0; b < n / be; ++b, p += bb) {
        jfo_dequantize_row(type, p, tmp, be);
        for (uint32_t i = 0; i < be; ++i) sum += (double) tmp[i] * x[b * be + i];
    }
    return sum;
}

int32_t jfo_argmax(const float * x, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i) {
        if (x[i] > x[best]) best = i;
    }
    return (int32_t) best;
}
