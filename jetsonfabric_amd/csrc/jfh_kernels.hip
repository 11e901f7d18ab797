// gfx950 kernels for the Qwen2 stage forward (decode, draft verify, prefill).
//
// Graph being implemented: runtime/engines/native/src/qwen2_architecture.cpp:522-598.
// Weights stay in their GGML block encodings (tensor_store.cpp:185-196); the
// matmuls quantize the activation row to int8 in 256-value blocks and use
// v_dot4 integer dot products against the unpacked quants, the same scheme
// GGML's CPU backend uses for K-quants (activation q8 blocks + integer dot).
#include "jfh_kernels.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace jfh::gpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kLdsActBytes = 32768;  // int8 activation bytes staged per K chunk

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16 & 0xFFFFu)));
}

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int dot16(const uint32_t* w, const uint4& x, int acc) {
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[0]), static_cast<int>(x.x), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[1]), static_cast<int>(x.y), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[2]), static_cast<int>(x.z), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(w[3]), static_cast<int>(x.w), acc, false);
    return acc;
}

__device__ __forceinline__ uint32_t u4_word(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ uint32_t u4_byte(const uint4& v, int i) {
    return (u4_word(v, i >> 2) >> (8 * (i & 3))) & 0xFFu;
}

// Q4_K 6-bit scale/min of sub-block j from the header's scale bytes (hdr.y..w).
__device__ __forceinline__ void q4k_scale_min(const uint4& h, int j, int& sc, int& m) {
    if (j < 4) {
        sc = (h.y >> (8 * j)) & 63;
        m = (h.z >> (8 * j)) & 63;
    } else {
        const int k = j - 4;
        sc = ((h.w >> (8 * k)) & 0xF) | (((h.y >> (8 * k + 6)) & 3) << 4);
        m = ((h.w >> (8 * k + 4)) & 0xF) | (((h.z >> (8 * k + 6)) & 3) << 4);
    }
}

// ------------------------------------------------------------------ element dequantization
// Exact GGML dequantization of one element from the device layout; the
// arithmetic order matches the reference formulas (see oracle/jfo_quant.c).
__device__ float dequant_elem(const DMat& m, uint32_t row, uint32_t c) {
    const uint8_t* base = m.main + static_cast<size_t>(row) * m.main_row_bytes;
    switch (m.type) {
    case 1: return reinterpret_cast<const float*>(base)[c];
    case 2: return h2f(reinterpret_cast<const uint16_t*>(base)[c]);
    case 7: {
        const uint32_t b = c / 32;
        const float d = h2f(reinterpret_cast<const uint16_t*>(m.aux + static_cast<size_t>(row) * m.aux_row_bytes)[b]);
        return static_cast<float>(static_cast<int8_t>(base[b * 32 + c % 32])) * d;
    }
    case 11: {
        const uint8_t* blk = base + static_cast<size_t>(c / 256) * 144;
        const uint32_t i = c % 256;
        const float d = h2f(blk[0] | (blk[1] << 8)), dmin = h2f(blk[2] | (blk[3] << 8));
        uint4 h;
        h.x = 0;
        h.y = blk[4] | (blk[5] << 8) | (blk[6] << 16) | (uint32_t(blk[7]) << 24);
        h.z = blk[8] | (blk[9] << 8) | (blk[10] << 16) | (uint32_t(blk[11]) << 24);
        h.w = blk[12] | (blk[13] << 8) | (blk[14] << 16) | (uint32_t(blk[15]) << 24);
        const uint32_t byte = blk[16 + (i / 64) * 32 + (i % 32)];
        const int q = (i % 64) < 32 ? (byte & 0xF) : (byte >> 4);
        int sc, mn;
        q4k_scale_min(h, static_cast<int>((i / 64) * 2 + (i % 64) / 32), sc, mn);
        const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(mn);
        return d1 * static_cast<float>(q) - m1;
    }
    case 13: {
        const uint32_t b = c / 256, i = c % 256;
        const uint8_t* blk = base + static_cast<size_t>(b) * 208;
        const float d = h2f(reinterpret_cast<const uint16_t*>(m.aux + static_cast<size_t>(row) * m.aux_row_bytes)[b]);
        const uint32_t half = i / 128, w = i % 128, quarter = w / 32, l = w % 32;
        const uint32_t lo = blk[64 * half + l + (quarter & 1) * 32];
        const uint32_t nib = quarter < 2 ? (lo & 0xF) : (lo >> 4);
        const uint32_t hi = (blk[128 + 32 * half + l] >> (2 * quarter)) & 3;
        const int q = static_cast<int>(nib | (hi << 4)) - 32;
        const float sc = static_cast<float>(static_cast<int8_t>(blk[192 + i / 16]));
        const float ds = d * sc;
        return ds * static_cast<float>(q);
    }
    case 9: {
        const uint32_t b = c / 256, i = c % 256;
        const uint8_t* blk = base + static_cast<size_t>(b) * 80;
        const uint32_t dd = reinterpret_cast<const uint32_t*>(m.aux + static_cast<size_t>(row) * m.aux_row_bytes)[b];
        const float d = h2f(dd), dmin = h2f(dd >> 16);
        const uint32_t half = i / 128, w = i % 128, shift = w / 32, part = (w % 32) / 16, l = w % 16;
        const int q = (blk[16 + 32 * half + 16 * part + l] >> (2 * shift)) & 3;
        const uint32_t sb = blk[i / 16];
        const float dl = d * static_cast<float>(sb & 0xF), ml = dmin * static_cast<float>(sb >> 4);
        return dl * static_cast<float>(q) - ml;
    }
    default:
        return 0.0F;
    }
}

__global__ __launch_bounds__(kThreads) void k_dequant_rows(DMat m, int32_t row0, float* out) {
    const uint32_t r = blockIdx.y;
    const uint32_t c = blockIdx.x * kThreads + threadIdx.x;
    if (c < m.cols) out[static_cast<size_t>(r) * m.cols + c] = dequant_elem(m, row0 + r, c);
}

// ------------------------------------------------------------------ embedding
__global__ __launch_bounds__(kThreads) void k_embed(DMat table, const StepDev* step, float* h, int32_t H,
                                                    unsigned long long* best, int32_t n_best) {
    const int r = blockIdx.y;
    if (blockIdx.x == 0 && r == 0) {
        for (int i = threadIdx.x; i < n_best; i += kThreads) best[i] = 0ull;
    }
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (r < step->n_rows && c < H) {
        h[static_cast<size_t>(r) * H + c] = dequant_elem(table, static_cast<uint32_t>(step->token[r]), c);
    }
}

// ------------------------------------------------------------------ activation quantization
// Quantizes 256 values held 4 per lane by one wave: d = amax/127,
// q = roundf(x * (1/d)), plus the sum of every 16 quantized values.
#pragma clang fp contract(off)
__device__ __forceinline__ void quant_block_wave(const float v[4], int lane, int8_t* q, float* d, int16_t* s) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = wave_max(amax);
    const float db = amax / 127.0F;
    const float id = db > 0.0F ? 1.0F / db : 0.0F;
    int qi[4];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float r = roundf(v[i] * id);
        r = fminf(127.0F, fmaxf(-127.0F, r));
        qi[i] = static_cast<int>(r);
        sum += qi[i];
    }
    const uint32_t packed = (qi[0] & 0xFF) | ((qi[1] & 0xFF) << 8) | ((qi[2] & 0xFF) << 16) | ((qi[3] & 0xFF) << 24);
    reinterpret_cast<uint32_t*>(q)[lane] = packed;
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if ((lane & 3) == 0) s[lane >> 2] = static_cast<int16_t>(sum);
    if (lane == 0) *d = db;
}

// RMSNorm * gain of each selected row (qwen2_architecture.cpp:373-376), then
// the int8 quantization consumed by the next matmul.
// One wave per (256-value block, row): every wave reduces the whole row's sum
// of squares itself (the row is a few KB, served from L2), then scales and
// quantizes only its own block, so a row is spread over H/256 work-groups.
__global__ __launch_bounds__(kWave) void k_norm_quant(const float* h, int32_t hs, const float* gain, float eps,
                                                      int32_t H, const StepDev* step, int32_t select_out,
                                                      int32_t quant, Act x) {
    const int r = blockIdx.y, b = blockIdx.x, lane = threadIdx.x;
    const int src = select_out ? step->out_row[r] : r;
    const float* hr = h + static_cast<size_t>(src) * hs;
    float ss = 0.0F;
    for (int i = 4 * lane; i < H; i += 4 * kWave) {
        const float4 v = *reinterpret_cast<const float4*>(hr + i);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = wave_sum(ss);
    const float mean = ss / static_cast<float>(H);
    const float scale = 1.0F / sqrtf(mean + eps);
    float v[4] = {0.0F, 0.0F, 0.0F, 0.0F};
    float* xf = x.f + static_cast<size_t>(r) * x.stride;
    const int e0 = b * kActBlock + 4 * lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (e0 + i < H) {
            v[i] = (hr[e0 + i] * scale) * gain[e0 + i];
            xf[e0 + i] = v[i];
        }
    }
    if (!quant) return;
    quant_block_wave(v, lane, x.q + static_cast<size_t>(r) * x.stride + b * kActBlock,
                     x.d + static_cast<size_t>(r) * (x.stride / kActBlock) + b,
                     x.s + static_cast<size_t>(r) * (x.stride / 16) + b * 16);
}

// Quantizes float rows (SwiGLU and attention outputs), one wave per
// (256-value block, row), keeping the float copy when the source differs.
__global__ __launch_bounds__(kWave) void k_quant(const float* src, int32_t ss, int32_t K, int32_t quant, Act x) {
    const int r = blockIdx.y, b = blockIdx.x, lane = threadIdx.x;
    const float* row = src + static_cast<size_t>(r) * ss;
    const int e0 = b * kActBlock + 4 * lane;
    float v[4] = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (e0 + i < K) {
            v[i] = row[e0 + i];
            if (x.f != src) x.f[static_cast<size_t>(r) * x.stride + e0 + i] = v[i];
        }
    }
    if (!quant) return;
    quant_block_wave(v, lane, x.q + static_cast<size_t>(r) * x.stride + b * kActBlock,
                     x.d + static_cast<size_t>(r) * (x.stride / kActBlock) + b,
                     x.s + static_cast<size_t>(r) * (x.stride / 16) + b * 16);
}
#pragma clang fp contract(on)

// ------------------------------------------------------------------ quantized matmul
// Staged activation chunk in LDS: q [NT][chunk], d [NT][chunk/256], s [NT][chunk/16].
struct Staged {
    const int8_t* q;
    const float* d;
    const int16_t* s;
    int32_t chunk;
};

struct RowRef {
    const uint8_t* main;
    const uint8_t* aux;
    bool valid;
};

// --- Q4_K: lane part p (0..3) owns qs bytes [32p, 32p+32) = sub-blocks 2p (low nibbles) and 2p+1 (high).
struct Q4KRegs {
    uint4 hdr, q0, q1;
};

__device__ __forceinline__ Q4KRegs q4k_load(const RowRef& r, int gb, int part) {
    const uint8_t* blk = r.main + static_cast<size_t>(gb) * 144;
    Q4KRegs v;
    v.hdr = *reinterpret_cast<const uint4*>(blk);
    v.q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * part);
    v.q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * part);
    return v;
}

template <int NT>
__device__ __forceinline__ void q4k_compute(const Q4KRegs& v, int part, const Staged& x, int lb, float* acc) {
    const float d = h2f(v.hdr.x), dmin = h2f(v.hdr.x >> 16);
    int sc0, m0, sc1, m1;
    q4k_scale_min(v.hdr, 2 * part, sc0, m0);
    q4k_scale_min(v.hdr, 2 * part + 1, sc1, m1);
    constexpr uint32_t M = 0x0F0F0F0Fu;
    const uint32_t lo0[4] = {v.q0.x & M, v.q0.y & M, v.q0.z & M, v.q0.w & M};
    const uint32_t lo1[4] = {v.q1.x & M, v.q1.y & M, v.q1.z & M, v.q1.w & M};
    const uint32_t hi0[4] = {(v.q0.x >> 4) & M, (v.q0.y >> 4) & M, (v.q0.z >> 4) & M, (v.q0.w >> 4) & M};
    const uint32_t hi1[4] = {(v.q1.x >> 4) & M, (v.q1.y >> 4) & M, (v.q1.z >> 4) & M, (v.q1.w >> 4) & M};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int8_t* xb = x.q + t * x.chunk + lb * 256 + 64 * part;
        const uint4 x0 = *reinterpret_cast<const uint4*>(xb);
        const uint4 x1 = *reinterpret_cast<const uint4*>(xb + 16);
        const uint4 x2 = *reinterpret_cast<const uint4*>(xb + 32);
        const uint4 x3 = *reinterpret_cast<const uint4*>(xb + 48);
        const int i0 = dot16(lo1, x1, dot16(lo0, x0, 0));
        const int i1 = dot16(hi1, x3, dot16(hi0, x2, 0));
        const int16_t* s = x.s + t * (x.chunk / 16) + lb * 16 + 4 * part;
        const int s0 = s[0] + s[1], s1 = s[2] + s[3];
        const int isum = sc0 * i0 + sc1 * i1;
        const int msum = m0 * s0 + m1 * s1;
        acc[t] += x.d[t * (x.chunk / 256) + lb] * (d * static_cast<float>(isum) - dmin * static_cast<float>(msum));
    }
}

// --- Q6_K (main 208 B: ql 128 | qh 64 | scales 16; aux: d). Lane part: half = p>>1, s = p&1,
// l in [16s, 16s+16): four quarters of 16 values each, groups 8*half + 2q + s.
struct Q6KRegs {
    uint4 l0, l1, h, sc;
    uint32_t d;
};

__device__ __forceinline__ Q6KRegs q6k_load(const RowRef& r, int gb, int part) {
    const uint8_t* blk = r.main + static_cast<size_t>(gb) * 208;
    const int half = part >> 1, s = part & 1;
    Q6KRegs v;
    v.l0 = *reinterpret_cast<const uint4*>(blk + 64 * half + 16 * s);
    v.l1 = *reinterpret_cast<const uint4*>(blk + 64 * half + 32 + 16 * s);
    v.h = *reinterpret_cast<const uint4*>(blk + 128 + 32 * half + 16 * s);
    v.sc = *reinterpret_cast<const uint4*>(blk + 192);
    v.d = reinterpret_cast<const uint16_t*>(r.aux)[gb];
    return v;
}

template <int NT>
__device__ __forceinline__ void q6k_compute(const Q6KRegs& v, int part, const Staged& x, int lb, float* acc) {
    const int half = part >> 1, s = part & 1;
    const float d = h2f(v.d);
    uint32_t q[4][4];
    const uint32_t l0[4] = {v.l0.x, v.l0.y, v.l0.z, v.l0.w};
    const uint32_t l1[4] = {v.l1.x, v.l1.y, v.l1.z, v.l1.w};
    const uint32_t hh[4] = {v.h.x, v.h.y, v.h.z, v.h.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[0][i] = (l0[i] & 0x0F0F0F0Fu) | ((hh[i] & 0x03030303u) << 4);
        q[1][i] = (l1[i] & 0x0F0F0F0Fu) | ((hh[i] << 2) & 0x30303030u);
        q[2][i] = ((l0[i] >> 4) & 0x0F0F0F0Fu) | (hh[i] & 0x30303030u);
        q[3][i] = ((l1[i] >> 4) & 0x0F0F0F0Fu) | ((hh[i] >> 2) & 0x30303030u);
    }
    int sc[4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) sc[qq] = static_cast<int8_t>(u4_byte(v.sc, 8 * half + 2 * qq + s));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int8_t* xb = x.q + t * x.chunk + lb * 256 + 128 * half + 16 * s;
        const int16_t* sb = x.s + t * (x.chunk / 16) + lb * 16 + 8 * half + s;
        int isum = 0;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xb + 32 * qq);
            const int iq = dot16(q[qq], xv, 0);
            isum += sc[qq] * (iq - 32 * static_cast<int>(sb[2 * qq]));
        }
        acc[t] += x.d[t * (x.chunk / 256) + lb] * (d * static_cast<float>(isum));
    }
}

// --- Q2_K (main 80 B: scales 16 | qs 64; aux: d, dmin). Lane part: half = p>>1, prt = p&1;
// one 16-byte qs slice holds four 2-bit planes (shift k) of 16 values, group 8*half + 2k + prt.
struct Q2KRegs {
    uint4 qb, sc;
    uint32_t dd;
};

__device__ __forceinline__ Q2KRegs q2k_load(const RowRef& r, int gb, int part) {
    const uint8_t* blk = r.main + static_cast<size_t>(gb) * 80;
    const int half = part >> 1, prt = part & 1;
    Q2KRegs v;
    v.qb = *reinterpret_cast<const uint4*>(blk + 16 + 32 * half + 16 * prt);
    v.sc = *reinterpret_cast<const uint4*>(blk);
    v.dd = reinterpret_cast<const uint32_t*>(r.aux)[gb];
    return v;
}

template <int NT>
__device__ __forceinline__ void q2k_compute(const Q2KRegs& v, int part, const Staged& x, int lb, float* acc) {
    const int half = part >> 1, prt = part & 1;
    const float d = h2f(v.dd), dmin = h2f(v.dd >> 16);
    const uint32_t qw[4] = {v.qb.x, v.qb.y, v.qb.z, v.qb.w};
    uint32_t vals[4][4];
    int scl[4], mn[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) vals[k][i] = (qw[i] >> (2 * k)) & 0x03030303u;
        const uint32_t b = u4_byte(v.sc, 8 * half + 2 * k + prt);
        scl[k] = static_cast<int>(b & 0xF);
        mn[k] = static_cast<int>(b >> 4);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int8_t* xb = x.q + t * x.chunk + lb * 256 + 128 * half + 16 * prt;
        const int16_t* sb = x.s + t * (x.chunk / 16) + lb * 16 + 8 * half + prt;
        int isum = 0, msum = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xb + 32 * k);
            isum += scl[k] * dot16(vals[k], xv, 0);
            msum += mn[k] * static_cast<int>(sb[2 * k]);
        }
        acc[t] += x.d[t * (x.chunk / 256) + lb] * (d * static_cast<float>(isum) - dmin * static_cast<float>(msum));
    }
}

// --- Q8_0 (main 32 B qs per 32 values; aux: d). Lane part p owns Q8_0 blocks 8*gb + 2p, +1.
struct Q80Regs {
    uint4 w0, w1, w2, w3;
    uint32_t dd;
};

__device__ __forceinline__ Q80Regs q80_load(const RowRef& r, int gb, int part) {
    const int b = gb * 8 + 2 * part;
    const uint8_t* p = r.main + static_cast<size_t>(b) * 32;
    Q80Regs v;
    v.w0 = *reinterpret_cast<const uint4*>(p);
    v.w1 = *reinterpret_cast<const uint4*>(p + 16);
    v.w2 = *reinterpret_cast<const uint4*>(p + 32);
    v.w3 = *reinterpret_cast<const uint4*>(p + 48);
    v.dd = *reinterpret_cast<const uint32_t*>(r.aux + static_cast<size_t>(b) * 2);
    return v;
}

template <int NT>
__device__ __forceinline__ void q80_compute(const Q80Regs& v, int part, const Staged& x, int lb, float* acc) {
    const float d0 = h2f(v.dd), d1 = h2f(v.dd >> 16);
    const uint32_t w0[4] = {v.w0.x, v.w0.y, v.w0.z, v.w0.w};
    const uint32_t w1[4] = {v.w1.x, v.w1.y, v.w1.z, v.w1.w};
    const uint32_t w2[4] = {v.w2.x, v.w2.y, v.w2.z, v.w2.w};
    const uint32_t w3[4] = {v.w3.x, v.w3.y, v.w3.z, v.w3.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int8_t* xb = x.q + t * x.chunk + lb * 256 + 64 * part;
        const int i0 = dot16(w1, *reinterpret_cast<const uint4*>(xb + 16), dot16(w0, *reinterpret_cast<const uint4*>(xb), 0));
        const int i1 = dot16(w3, *reinterpret_cast<const uint4*>(xb + 48), dot16(w2, *reinterpret_cast<const uint4*>(xb + 32), 0));
        acc[t] += x.d[t * (x.chunk / 256) + lb] * (d0 * static_cast<float>(i0) + d1 * static_cast<float>(i1));
    }
}

template <uint32_t TYPE, int NT>
__device__ __forceinline__ void block_dot(const RowRef& r, int gb, int part, const Staged& x, int lb, float* acc) {
    if constexpr (TYPE == 11) {
        q4k_compute<NT>(q4k_load(r, gb, part), part, x, lb, acc);
    } else if constexpr (TYPE == 13) {
        q6k_compute<NT>(q6k_load(r, gb, part), part, x, lb, acc);
    } else if constexpr (TYPE == 9) {
        q2k_compute<NT>(q2k_load(r, gb, part), part, x, lb, acc);
    } else {
        q80_compute<NT>(q80_load(r, gb, part), part, x, lb, acc);
    }
}

// Which matrix and local row a concatenated row index belongs to.
__device__ __forceinline__ int locate(const GemvArgs& a, int r, int& local) {
    local = r;
    for (int i = 0; i < a.n_mat; ++i) {
        if (local < static_cast<int>(a.mat[i].rows)) return i;
        local -= static_cast<int>(a.mat[i].rows);
    }
    return -1;
}

__device__ __forceinline__ unsigned long long pack_best(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - idx);
}

// Shared epilogue: values of the wave's two weight rows for every token.
template <int NT>
__device__ void gemv_epilogue(const GemvArgs& a, const int mi[2], const int lr[2], const int gr[2], float acc[2][NT],
                              int wave, int lane) {
    __shared__ float best_v[kThreads / kWave][NT];
    __shared__ uint32_t best_i[kThreads / kWave][NT];
    if (a.mode == kLogits) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float bv = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (mi[k] < 0) continue;
                float v = acc[k][t];
                if (a.mat[mi[k]].bias) v += a.mat[mi[k]].bias[lr[k]];
                if (a.store_logits && lane == 0 && t < a.n_tok) a.y[static_cast<size_t>(t) * a.y_stride + gr[k]] = v;
                if (v > bv || (v == bv && static_cast<uint32_t>(gr[k]) < bi)) { bv = v; bi = static_cast<uint32_t>(gr[k]); }
            }
            if (lane == 0) { best_v[wave][t] = bv; best_i[wave][t] = bi; }
        }
        __syncthreads();
        if (threadIdx.x < static_cast<unsigned>(a.n_tok) && threadIdx.x < NT) {
            const int t = threadIdx.x;
            float bv = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
            for (int w = 0; w < kThreads / kWave; ++w) {
                if (best_i[w][t] == 0xFFFFFFFFu) continue;
                if (best_v[w][t] > bv || (best_v[w][t] == bv && best_i[w][t] < bi)) { bv = best_v[w][t]; bi = best_i[w][t]; }
            }
            if (bi != 0xFFFFFFFFu) atomicMax(a.best + t, pack_best(bv, bi));
        }
        return;
    }
    if (lane != 0) return;
    if (a.mode == kSwiGLU) {
        if (mi[0] < 0) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t >= a.n_tok) break;
            const float g = acc[0][t], u = acc[1][t];
            a.y[static_cast<size_t>(t) * a.y_stride + lr[0]] = g / (1.0F + expf(-g)) * u;
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (mi[k] < 0) continue;
        const float b = a.mat[mi[k]].bias ? a.mat[mi[k]].bias[lr[k]] : 0.0F;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t >= a.n_tok) break;
            float* out = a.y + static_cast<size_t>(t) * a.y_stride + gr[k];
            if (a.mode == kAdd) *out += acc[k][t];
            else *out = acc[k][t] + b;
        }
    }
}

__device__ __forceinline__ void wave_rows(const GemvArgs& a, int wave_global, int mi[2], int lr[2], int gr[2]) {
    if (a.mode == kSwiGLU) {
        const int r = wave_global;
        const bool ok = r < static_cast<int>(a.mat[0].rows);
        mi[0] = ok ? 0 : -1;
        mi[1] = ok ? 1 : -1;
        lr[0] = lr[1] = r;
        gr[0] = gr[1] = r;
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            gr[k] = 2 * wave_global + k;
            mi[k] = locate(a, gr[k], lr[k]);
        }
    }
}

template <uint32_t TYPE, int NT>
__global__ __launch_bounds__(kThreads) void k_gemv_q(GemvArgs a, int32_t chunk) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* sq = reinterpret_cast<int8_t*>(lds_raw);
    float* sd = reinterpret_cast<float*>(lds_raw + NT * chunk);
    int16_t* ss = reinterpret_cast<int16_t*>(sd + NT * (chunk / 256));
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int part = lane & 3, slot = lane >> 2;
    int mi[2], lr[2], gr[2];
    wave_rows(a, blockIdx.x * (kThreads / kWave) + wave, mi, lr, gr);
    RowRef rows[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        rows[k].valid = mi[k] >= 0;
        const DMat& m = a.mat[rows[k].valid ? mi[k] : 0];
        rows[k].main = m.main + static_cast<size_t>(rows[k].valid ? lr[k] : 0) * m.main_row_bytes;
        rows[k].aux = m.aux ? m.aux + static_cast<size_t>(rows[k].valid ? lr[k] : 0) * m.aux_row_bytes : nullptr;
    }
    float acc[2][NT];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = 0.0F;

    const int K = static_cast<int>(a.mat[0].cols);
    const Staged st{sq, sd, ss, chunk};
    for (int c0 = 0; c0 < K; c0 += chunk) {
        const int ce = min(chunk, K - c0);
        __syncthreads();
        for (int t = 0; t < NT; ++t) {
            const int8_t* gq = a.x.q + static_cast<size_t>(t) * a.x.stride + c0;
            for (int i = threadIdx.x * 16; i < ce; i += kThreads * 16) {
                *reinterpret_cast<uint4*>(sq + t * chunk + i) = *reinterpret_cast<const uint4*>(gq + i);
            }
            for (int i = threadIdx.x; i < ce / 256; i += kThreads) {
                sd[t * (chunk / 256) + i] = a.x.d[static_cast<size_t>(t) * (a.x.stride / 256) + c0 / 256 + i];
            }
            for (int i = threadIdx.x; i < ce / 16; i += kThreads) {
                ss[t * (chunk / 16) + i] = a.x.s[static_cast<size_t>(t) * (a.x.stride / 16) + c0 / 16 + i];
            }
        }
        __syncthreads();
        const int nb = ce / 256;
        for (int lb = slot; lb < nb; lb += kWave / 4) {
            const int gb = c0 / 256 + lb;
            if (rows[0].valid) block_dot<TYPE, NT>(rows[0], gb, part, st, lb, acc[0]);
            if (rows[1].valid) block_dot<TYPE, NT>(rows[1], gb, part, st, lb, acc[1]);
        }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = wave_sum(acc[k][t]);
    gemv_epilogue<NT>(a, mi, lr, gr, acc, wave, lane);
}

// Float weights (F32/F16): float activations, lanes stride over the row.
template <int NT>
__global__ __launch_bounds__(kThreads) void k_gemv_f(GemvArgs a) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    int mi[2], lr[2], gr[2];
    wave_rows(a, blockIdx.x * (kThreads / kWave) + wave, mi, lr, gr);
    float acc[2][NT];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = 0.0F;
    const int K = static_cast<int>(a.mat[0].cols);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (mi[k] < 0) continue;
        const DMat& m = a.mat[mi[k]];
        for (int c = lane; c < K; c += kWave) {
            const float w = dequant_elem(m, static_cast<uint32_t>(lr[k]), static_cast<uint32_t>(c));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t < a.n_tok) acc[k][t] += w * a.x.f[static_cast<size_t>(t) * a.x.stride + c];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[k][t] = wave_sum(acc[k][t]);
    gemv_epilogue<NT>(a, mi, lr, gr, acc, wave, lane);
}

// ------------------------------------------------------------------ RoPE + KV write
#pragma clang fp contract(off)
// NEOX rotation of q and k heads (qwen2_architecture.cpp:499-506) with the
// shared cos/sin table; k and v rows are stored as f16 at the row's position.
__global__ __launch_bounds__(kThreads) void k_rope_kv(const float* qkv, int32_t n_head, int32_t n_head_kv,
                                                      int32_t hd, const float* rope, const StepDev* step,
                                                      int32_t layer, float* qout) {
    const int r = blockIdx.x;
    if (r >= step->n_rows) return;
    const int H = n_head * hd, kv = n_head_kv * hd, half = hd / 2;
    const int pos = step->pos[r];
    const SeqDev& sd = step->seqs[step->seq[r]];
    const float* src = qkv + static_cast<size_t>(r) * (H + 2 * kv);
    const float* cs = rope + static_cast<size_t>(pos) * hd;
    for (int idx = threadIdx.x; idx < (n_head + n_head_kv) * half; idx += kThreads) {
        const int head = idx / half, i = idx % half;
        const float c = cs[2 * i], s = cs[2 * i + 1];
        if (head < n_head) {
            const float x0 = src[head * hd + i], x1 = src[head * hd + i + half];
            float* o = qout + static_cast<size_t>(r) * H + head * hd;
            o[i] = x0 * c - x1 * s;
            o[i + half] = x0 * s + x1 * c;
        } else {
            const int kh = head - n_head;
            const float x0 = src[H + kh * hd + i], x1 = src[H + kh * hd + i + half];
            uint16_t* kr = sd.k + ((static_cast<size_t>(layer) * n_head_kv + kh) * sd.capacity + pos) * hd;
            kr[i] = f2h(x0 * c - x1 * s);
            kr[i + half] = f2h(x0 * s + x1 * c);
        }
    }
    for (int idx = threadIdx.x; idx < kv; idx += kThreads) {
        const int kh = idx / hd, dd = idx % hd;
        uint16_t* vr = sd.v + ((static_cast<size_t>(layer) * n_head_kv + kh) * sd.capacity + pos) * hd;
        vr[dd] = f2h(src[H + kv + idx]);
    }
}
#pragma clang fp contract(on)

// ------------------------------------------------------------------ attention
// Split-K causal GQA flash attention (qwen2_architecture.cpp:438-464, mask
// 697-708) over the f16 cache. Work-group = (key split, kv head, sequence);
// its 4 waves own disjoint slices of the query rows (G heads x T rows) that
// share the kv head. Inside a wave each lane owns one key of a 64-key tile:
// the lane loads its K row once and scores it against the wave's queries
// (query values are wave-uniform, read through the scalar cache), the online
// softmax keeps (max, sum, output) in registers, and for P.V the lanes switch
// to owning two head dims each. The last work-group of a (sequence, kv head)
// to finish merges the splits' partials (atomic counter, reset afterwards).
constexpr int kAttnWaves = 4;

template <int QPW>
__global__ __launch_bounds__(kAttnWaves * kWave) void k_attention(
    const float* __restrict__ q, const StepDev* __restrict__ step, int32_t layer, int32_t n_head, int32_t n_head_kv,
    int32_t hd, int32_t splits_max, float* __restrict__ partial, int32_t* __restrict__ counters,
    float* __restrict__ out, int32_t out_stride) {
    __shared__ float P[kAttnWaves][QPW][kWave];
    __shared__ int32_t last;
    const int seq = blockIdx.z;
    if (seq >= step->n_seq) return;
    const int32_t pos0 = step->seqs[seq].pos0, len = step->seqs[seq].len, row0 = step->seqs[seq].row0;
    const int32_t capacity = step->seqs[seq].capacity;
    const int n_keys = pos0 + len;
    int L = (n_keys + splits_max - 1) / splits_max;
    L = (L + kWave - 1) / kWave * kWave;
    const int n_splits = (n_keys + L - 1) / L;
    const int split = blockIdx.x;
    if (split >= n_splits) return;
    const int k0 = split * L, k1 = min(n_keys, k0 + L);
    const int kvh = blockIdx.y;
    const int G = n_head / n_head_kv, NQ = G * len, H = n_head * hd;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int q_begin = wave * QPW;
    const int nq = max(0, min(QPW, NQ - q_begin));
    const float scale = 1.0F / sqrtf(static_cast<float>(hd));
    const size_t head_base = (static_cast<size_t>(layer) * n_head_kv + kvh) * capacity;
    const uint16_t* kc = step->seqs[seq].k + head_base * hd;
    const uint16_t* vc = step->seqs[seq].v + head_base * hd;

    const float* qrow[QPW];
    int limit[QPW];  // last visible key of each query row (causal)
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
        const int qi = min(q_begin + i, NQ - 1);
        const int t = qi / G, head = kvh * G + qi % G;
        qrow[i] = q + static_cast<size_t>(row0 + t) * H + head * hd;
        limit[i] = pos0 + t;
    }
    float m[QPW], l[QPW], o0[QPW], o1[QPW];
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0F;
        o0[i] = 0.0F;
        o1[i] = 0.0F;
    }
    const bool vec8 = (hd & 7) == 0;
    for (int t0 = k0; t0 < k1; t0 += kWave) {
        const int key = t0 + lane;
        const uint16_t* krow = kc + static_cast<size_t>(min(key, capacity - 1)) * hd;
        float sc[QPW];
#pragma unroll
        for (int i = 0; i < QPW; ++i) sc[i] = 0.0F;
        if (vec8) {
            for (int d = 0; d < hd; d += 8) {
                const uint4 kv = *reinterpret_cast<const uint4*>(krow + d);
                const float kf[8] = {h2f(kv.x), h2f(kv.x >> 16), h2f(kv.y), h2f(kv.y >> 16),
                                     h2f(kv.z), h2f(kv.z >> 16), h2f(kv.w), h2f(kv.w >> 16)};
#pragma unroll
                for (int i = 0; i < QPW; ++i) {
                    if (i < nq) {
                        const float* qd = qrow[i] + d;
                        float acc = sc[i];
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc += kf[e] * qd[e];
                        sc[i] = acc;
                    }
                }
            }
        } else {
            for (int d = 0; d < hd; ++d) {
                const float kf = h2f(krow[d]);
#pragma unroll
                for (int i = 0; i < QPW; ++i) {
                    if (i < nq) sc[i] += kf * qrow[i][d];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            if (i < nq) {
                const bool vis = key < k1 && key <= limit[i];
                const float s = vis ? sc[i] * scale : -INFINITY;
                const float m_new = fmaxf(m[i], wave_max(s));
                float p = 0.0F, alpha = 1.0F;
                if (m_new != -INFINITY) {
                    alpha = m[i] == -INFINITY ? 0.0F : expf(m[i] - m_new);
                    p = vis ? expf(s - m_new) : 0.0F;
                }
                l[i] = l[i] * alpha + p;
                o0[i] *= alpha;
                o1[i] *= alpha;
                m[i] = m_new;
                P[wave][i][lane] = p;
            }
        }
        __syncthreads();
        const int nk = min(kWave, k1 - t0);
        if (2 * lane < hd) {
            for (int j = 0; j < nk; ++j) {
                const uint32_t vv = *reinterpret_cast<const uint32_t*>(vc + static_cast<size_t>(t0 + j) * hd + 2 * lane);
                const float v0 = h2f(vv), v1 = h2f(vv >> 16);
#pragma unroll
                for (int i = 0; i < QPW; ++i) {
                    if (i < nq) {
                        const float pj = P[wave][i][j];
                        o0[i] += pj * v0;
                        o1[i] += pj * v1;
                    }
                }
            }
        }
        __syncthreads();
    }
    // split partial: (max, sum, unnormalized output) per query row
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
        if (i < nq) {
            const float lsum = wave_sum(l[i]);
            const int qi = q_begin + i;
            const int t = qi / G, head = kvh * G + qi % G;
            float* dst = partial + ((static_cast<size_t>(row0 + t) * n_head + head) * splits_max + split) * (hd + 2);
            if (lane == 0) {
                dst[0] = m[i];
                dst[1] = lsum;
            }
            if (2 * lane < hd) {
                dst[2 + 2 * lane] = o0[i];
                dst[3 + 2 * lane] = o1[i];
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(counters + seq * n_head_kv + kvh, 1) == n_splits - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    // merge the splits: lanes over splits for the statistics, lanes over dims for the output
    for (int qi = wave; qi < NQ; qi += kAttnWaves) {
        const int t = qi / G, head = kvh * G + qi % G;
        const float* base = partial + (static_cast<size_t>(row0 + t) * n_head + head) * splits_max * (hd + 2);
        const float ms = lane < n_splits ? base[lane * (hd + 2)] : -INFINITY;
        const float ls = lane < n_splits ? base[lane * (hd + 2) + 1] : 0.0F;
        const float M = wave_max(ms);
        const float w = ms == -INFINITY ? 0.0F : expf(ms - M);
        const float total = wave_sum(ls * w);
        float a0 = 0.0F, a1 = 0.0F;
        for (int sp = 0; sp < n_splits; ++sp) {
            const float ws = __shfl(w, sp);
            if (2 * lane < hd) {
                a0 += ws * base[sp * (hd + 2) + 2 + 2 * lane];
                a1 += ws * base[sp * (hd + 2) + 3 + 2 * lane];
            }
        }
        if (2 * lane < hd) {
            float* o = out + static_cast<size_t>(row0 + t) * out_stride + head * hd;
            o[2 * lane] = a0 / total;
            o[2 * lane + 1] = a1 / total;
        }
    }
    if (threadIdx.x == 0) counters[seq * n_head_kv + kvh] = 0;
}

// ------------------------------------------------------------------ argmax + acceptance
// Greedy ids of the logits rows (first maximum, qwen2_architecture.cpp:594) and,
// per sequence, the accepted draft prefix: rows are compared in order with the
// next input token until the first mismatch (generation_runner.cpp:512-517).
__global__ void k_finish(const unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out) {
    __shared__ int32_t tok[kMaxRows];
    for (int i = threadIdx.x; i < n_out; i += blockDim.x) {
        const uint32_t low = static_cast<uint32_t>(best[i] & 0xFFFFFFFFull);
        tok[i] = best[i] == 0ull ? -1 : static_cast<int32_t>(0xFFFFFFFFu - low);
        out->token[i] = tok[i];
    }
    __syncthreads();
    for (int s = threadIdx.x; s < step->n_seq; s += blockDim.x) {
        int accepted = 0;
        bool open = true;
        for (int i = 0; i < n_out; ++i) {
            const int r = step->out_row[i];
            if (step->seq[r] != s || !open) continue;
            if (step->draft[i] >= 0 && tok[i] == step->draft[i]) ++accepted;
            else open = false;
        }
        out->accepted[s] = accepted;
    }
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <uint32_t TYPE, int NT>
void gemv_q(const GemvArgs& a, int blocks, hipStream_t stream) {
    const int K = static_cast<int>(a.mat[0].cols);
    const int chunk = gemv_chunk_values(NT, K);
    const size_t lds = static_cast<size_t>(NT) * chunk + static_cast<size_t>(NT) * (chunk / 256) * 4 +
                       static_cast<size_t>(NT) * (chunk / 16) * 2;
    hipLaunchKernelGGL((k_gemv_q<TYPE, NT>), dim3(blocks), dim3(kThreads), lds, stream, a, chunk);
    check(hipGetLastError(), "gemv launch");
}

template <uint32_t TYPE>
void gemv_q_nt(const GemvArgs& a, int blocks, hipStream_t stream) {
    switch (a.n_tok) {
    case 1: gemv_q<TYPE, 1>(a, blocks, stream); break;
    case 2: gemv_q<TYPE, 2>(a, blocks, stream); break;
    case 3: gemv_q<TYPE, 3>(a, blocks, stream); break;
    case 4: gemv_q<TYPE, 4>(a, blocks, stream); break;
    case 5: gemv_q<TYPE, 5>(a, blocks, stream); break;
    case 6: gemv_q<TYPE, 6>(a, blocks, stream); break;
    case 7: gemv_q<TYPE, 7>(a, blocks, stream); break;
    case 8: gemv_q<TYPE, 8>(a, blocks, stream); break;
    default: throw std::invalid_argument("gemv token group must be 1..8");
    }
}

}  // namespace

int32_t gemv_chunk_values(int32_t n_tok, int32_t K) {
    int32_t chunk = (kLdsActBytes / n_tok) / 256 * 256;
    if (chunk < 256) chunk = 256;
    const int32_t k_round = (K + 255) / 256 * 256;
    return chunk < k_round ? chunk : k_round;
}

void launch_gemv(const GemvArgs& a_in, hipStream_t stream) {
    // token groups of at most 8 rows
    for (int t0 = 0; t0 < a_in.n_tok; t0 += 8) {
        GemvArgs a = a_in;
        a.n_tok = a_in.n_tok - t0 < 8 ? a_in.n_tok - t0 : 8;
        a.x.q += static_cast<size_t>(t0) * a.x.stride;
        a.x.d += static_cast<size_t>(t0) * (a.x.stride / 256);
        a.x.s += static_cast<size_t>(t0) * (a.x.stride / 16);
        a.x.f += static_cast<size_t>(t0) * a.x.stride;
        a.y += static_cast<size_t>(t0) * a.y_stride;
        if (a.best) a.best += t0;
        uint32_t total = 0;
        for (int i = 0; i < a.n_mat; ++i) total += a.mat[i].rows;
        const int waves = a.mode == kSwiGLU ? static_cast<int>(a.mat[0].rows) : static_cast<int>((total + 1) / 2);
        const int blocks = (waves + kThreads / kWave - 1) / (kThreads / kWave);
        const uint32_t type = a.mat[0].type;
        if (type == 1 || type == 2) {
            switch (a.n_tok) {
            case 1: hipLaunchKernelGGL(k_gemv_f<1>, dim3(blocks), dim3(kThreads), 0, stream, a); break;
            case 2: hipLaunchKernelGGL(k_gemv_f<2>, dim3(blocks), dim3(kThreads), 0, stream, a); break;
            case 3: case 4: hipLaunchKernelGGL(k_gemv_f<4>, dim3(blocks), dim3(kThreads), 0, stream, a); break;
            default: hipLaunchKernelGGL(k_gemv_f<8>, dim3(blocks), dim3(kThreads), 0, stream, a); break;
            }
            check(hipGetLastError(), "gemv launch");
            continue;
        }
        switch (type) {
        case 11: gemv_q_nt<11>(a, blocks, stream); break;
        case 13: gemv_q_nt<13>(a, blocks, stream); break;
        case 9: gemv_q_nt<9>(a, blocks, stream); break;
        case 7: gemv_q_nt<7>(a, blocks, stream); break;
        default: throw std::invalid_argument("unsupported weight type for gemv");
        }
    }
}

void launch_embed(const DMat& table, const StepDev* step, float* h, int32_t n_rows, int32_t H,
                  unsigned long long* best, int32_t n_best, hipStream_t stream) {
    dim3 grid((H + kThreads - 1) / kThreads, n_rows);
    hipLaunchKernelGGL(k_embed, grid, dim3(kThreads), 0, stream, table, step, h, H, best, n_best);
    check(hipGetLastError(), "embed launch");
}

void launch_norm_quant(const float* h, int32_t h_stride, const float* gain, float eps, int32_t H,
                       const StepDev* step, int32_t select_out, int32_t n_rows, bool quantize, Act x,
                       hipStream_t stream) {
    if (H % 4 != 0) throw std::invalid_argument("hidden size must be a multiple of 4");
    hipLaunchKernelGGL(k_norm_quant, dim3((H + kActBlock - 1) / kActBlock, n_rows), dim3(kWave), 0, stream, h,
                       h_stride, gain, eps, H, step, select_out, quantize ? 1 : 0, x);
    check(hipGetLastError(), "norm launch");
}

void launch_quant(const float* src, int32_t src_stride, int32_t K, int32_t n_rows, bool quantize, Act x,
                  hipStream_t stream) {
    hipLaunchKernelGGL(k_quant, dim3((K + kActBlock - 1) / kActBlock, n_rows), dim3(kWave), 0, stream, src, src_stride,
                       K, quantize ? 1 : 0, x);
    check(hipGetLastError(), "quant launch");
}

void launch_rope_kv(const float* qkv, int32_t n_rows, int32_t n_head, int32_t n_head_kv, int32_t head_dim,
                    const float* rope, const StepDev* step, int32_t layer, float* qout, hipStream_t stream) {
    hipLaunchKernelGGL(k_rope_kv, dim3(n_rows), dim3(kThreads), 0, stream, qkv, n_head, n_head_kv, head_dim, rope,
                       step, layer, qout);
    check(hipGetLastError(), "rope launch");
}

int32_t attention_splits(int32_t capacity) {
    const int32_t s = (capacity + kWave - 1) / kWave;
    return s < 1 ? 1 : (s > kWave ? kWave : s);
}

void launch_attention(const float* q, const StepDev* step, int32_t n_rows, int32_t max_len, int32_t n_seq,
                      int32_t layer, int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits,
                      float* partial, int32_t* counters, Act out, hipStream_t stream) {
    const int G = n_head / n_head_kv;
    const int nq = G * max_len;
    if (head_dim > 2 * kWave || head_dim % 2 != 0) throw std::invalid_argument("attention supports even head dims <= 128");
    if (nq > kAttnWaves * 16) throw std::invalid_argument("attention work-group exceeds its query rows");
    const int qpw = (nq + kAttnWaves - 1) / kAttnWaves;
    dim3 grid(splits, n_head_kv, n_seq), block(kAttnWaves * kWave);
#define JFH_ATTN(QPW)                                                                                          \
    hipLaunchKernelGGL(k_attention<QPW>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, head_dim, \
                       splits, partial, counters, out.f, out.stride)
    if (qpw <= 2) JFH_ATTN(2);
    else if (qpw <= 4) JFH_ATTN(4);
    else if (qpw <= 8) JFH_ATTN(8);
    else JFH_ATTN(16);
#undef JFH_ATTN
    check(hipGetLastError(), "attention launch");
    const int H = n_head * head_dim;
    launch_quant(out.f, out.stride, H, n_rows, H % kActBlock == 0, out, stream);
}

void launch_finish(const unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out,
                   hipStream_t stream) {
    hipLaunchKernelGGL(k_finish, dim3(1), dim3(64), 0, stream, best, step, n_out, out);
    check(hipGetLastError(), "finish launch");
}

void launch_dequant_rows(const DMat& m, int32_t row0, int32_t n_rows, float* out, hipStream_t stream) {
    dim3 grid((m.cols + kThreads - 1) / kThreads, n_rows);
    hipLaunchKernelGGL(k_dequant_rows, grid, dim3(kThreads), 0, stream, m, row0, out);
    check(hipGetLastError(), "dequant launch");
}

}  // namespace jfh::gpu
