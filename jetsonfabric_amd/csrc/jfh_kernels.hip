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

// Load/compute split per block type, so that a wave can issue the loads of
// all of its rows (and two block iterations) before consuming any of them.
template <uint32_t TYPE>
struct QBlock;
template <>
struct QBlock<11> {
    using Regs = Q4KRegs;
    static __device__ __forceinline__ Regs load(const RowRef& r, int gb, int part) { return q4k_load(r, gb, part); }
    template <int NT>
    static __device__ __forceinline__ void dot(const Regs& v, int part, const Staged& x, int lb, float* acc) {
        q4k_compute<NT>(v, part, x, lb, acc);
    }
};
template <>
struct QBlock<13> {
    using Regs = Q6KRegs;
    static __device__ __forceinline__ Regs load(const RowRef& r, int gb, int part) { return q6k_load(r, gb, part); }
    template <int NT>
    static __device__ __forceinline__ void dot(const Regs& v, int part, const Staged& x, int lb, float* acc) {
        q6k_compute<NT>(v, part, x, lb, acc);
    }
};
template <>
struct QBlock<9> {
    using Regs = Q2KRegs;
    static __device__ __forceinline__ Regs load(const RowRef& r, int gb, int part) { return q2k_load(r, gb, part); }
    template <int NT>
    static __device__ __forceinline__ void dot(const Regs& v, int part, const Staged& x, int lb, float* acc) {
        q2k_compute<NT>(v, part, x, lb, acc);
    }
};
template <>
struct QBlock<7> {
    using Regs = Q80Regs;
    static __device__ __forceinline__ Regs load(const RowRef& r, int gb, int part) { return q80_load(r, gb, part); }
    template <int NT>
    static __device__ __forceinline__ void dot(const Regs& v, int part, const Staged& x, int lb, float* acc) {
        q80_compute<NT>(v, part, x, lb, acc);
    }
};

__device__ __forceinline__ unsigned long long pack_best(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - idx);
}

// Sum over the 4 lanes of a quad (DPP quad permutations [1,0,3,2], [2,3,0,1]).
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
    return v;
}

__device__ __forceinline__ const float* x_row(const XIn& x, int t) {
    return x.x + static_cast<size_t>(x.gather ? x.gather[t] : t) * x.stride;
}

// 1/sqrt(mean(x^2) + eps) of each token row (qwen2_architecture.cpp:373-376),
// reduced by the whole work-group into rs[t].
template <int NT>
__device__ void row_rms(const XIn& x, int n_tok, int K, float* rs, float* red) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    for (int t = 0; t < n_tok; ++t) {
        const float* xr = x_row(x, t);
        float ss = 0.0F;
        for (int i0 = 4 * threadIdx.x; i0 < K; i0 += 4 * 4 * kThreads) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * 4 * kThreads;
                v[u] = i < K ? *reinterpret_cast<const float4*>(xr + i) : make_float4(0.0F, 0.0F, 0.0F, 0.0F);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[t * (kThreads / kWave) + wave] = ss;
    }
    __syncthreads();
    if (threadIdx.x < static_cast<unsigned>(n_tok)) {
        const int t = threadIdx.x;
        float ss = 0.0F;
        for (int w = 0; w < kThreads / kWave; ++w) ss += red[t * (kThreads / kWave) + w];
        rs[t] = 1.0F / sqrtf(ss / static_cast<float>(K) + x.eps);
    }
    __syncthreads();
}

// Quantizes values [c0, c0 + nb*256) of every token row into the LDS chunk
// (int8, scale per 256 values, int16 sums per 16), one wave per 256-value
// block, loads issued four blocks at a time.
#pragma clang fp contract(off)
template <int NT>
__device__ void stage_chunk(const XIn& x, int n_tok, int c0, int nb, const float* rs, int8_t* sq, float* sd,
                            int16_t* ss, int chunk) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    constexpr int W = kThreads / kWave;
    const int total = n_tok * nb;
    for (int j0 = wave; j0 < total; j0 += 4 * W) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + u * W;
            if (j < total) {
                const int t = j / nb, b = j - t * nb;
                const int c = c0 + b * 256 + 4 * lane;
                v[u] = *reinterpret_cast<const float4*>(x_row(x, t) + c);
                if (x.gain) {
                    const float r = rs[t];
                    const float4 g = *reinterpret_cast<const float4*>(x.gain + c);
                    v[u].x = v[u].x * r * g.x;
                    v[u].y = v[u].y * r * g.y;
                    v[u].z = v[u].z * r * g.z;
                    v[u].w = v[u].w * r * g.w;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + u * W;
            if (j < total) {
                const int t = j / nb, b = j - t * nb;
                const float vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                quant_block_wave(vv, lane, sq + t * chunk + b * 256, sd + t * (chunk / 256) + b,
                                 ss + t * (chunk / 16) + b * 16);
            }
        }
    }
}
#pragma clang fp contract(on)

// Launch geometry of one quantized matmul, fixed by the host.
struct GemvGeom {
    int32_t rows_per_wg;  // rows of one work-group (even; a multiple of 2*kGluGroup for SwiGLU)
    int32_t chunk;        // K values staged per pass (multiple of 256)
    uint64_t nbc_magic;   // ceil(2^32 / nbc), nbc = chunk / 256: f / nbc = (f * magic) >> 32
};

#pragma clang fp contract(off)
__device__ __forceinline__ void qkv_store(const GemvArgs& a, int t, int gr, float va, float vb, bool pair) {
    // gr: first fused row of a rotated pair (q or k) or a v row (pair == false)
    const QkvOut& o = a.qkv;
    const int hd = o.head_dim, half = hd / 2, Hq = o.n_head * hd, kv = o.n_head_kv * hd;
    const StepDev* st = o.step;
    const int pos = st->pos[o.row0 + t];
    const SeqDev& sd = st->seqs[st->seq[o.row0 + t]];
    if (pair) {
        const int region = gr < Hq ? 0 : 1;
        const int g = region == 0 ? gr : gr - Hq;
        const int head = g / hd, i = (g % hd) / 2;
        const float c = o.rope[static_cast<size_t>(pos) * hd + 2 * i];
        const float s = o.rope[static_cast<size_t>(pos) * hd + 2 * i + 1];
        const float r0 = va * c - vb * s;
        const float r1 = va * s + vb * c;
        if (region == 0) {
            float* q = o.q + static_cast<size_t>(t) * Hq + head * hd;
            q[i] = r0;
            q[i + half] = r1;
        } else {
            const size_t row = ((static_cast<size_t>(o.layer) * o.n_head_kv + head) * sd.capacity + pos) * hd;
            sd.k[row + i] = f2h(r0);
            sd.k[row + i + half] = f2h(r1);
        }
    } else {
        const int g = gr - Hq - kv;
        const int head = g / hd, dcol = g % hd;
        const size_t row = ((static_cast<size_t>(o.layer) * o.n_head_kv + head) * sd.capacity + pos) * hd;
        sd.v[row + dcol] = f2h(va);
    }
}
#pragma clang fp contract(on)

// Row results of a work-group (sums in LDS) -> bias / residual / SwiGLU /
// RoPE + cache / greedy argmax. `sum(j, t)` returns the dot of local row j.
template <int NT, typename Sum>
__device__ void gemv_epilogue(const GemvArgs& a, int row0, int nrows, Sum sum, float* lv) {
    const int n = nrows * a.n_tok;
    switch (a.mode) {
    case kStore:
    case kAdd:
        for (int idx = threadIdx.x; idx < n; idx += kThreads) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            float* out = a.y + static_cast<size_t>(t) * a.y_stride + gr;
            if (a.mode == kAdd) *out += sum(j, t);
            else *out = sum(j, t) + (a.mat.bias ? a.mat.bias[gr] : 0.0F);
        }
        break;
    case kSwiGLU: {
        const int half = nrows / 2;
        for (int idx = threadIdx.x; idx < half * a.n_tok; idx += kThreads) {
            const int t = idx / half, jj = idx - t * half;
            const int j = (jj / kGluGroup) * 2 * kGluGroup + jj % kGluGroup;
            const float g = sum(j, t), u = sum(j + kGluGroup, t);
            const int o = (row0 / 2) + jj;
            a.y[static_cast<size_t>(t) * a.y_stride + o] = g / (1.0F + expf(-g)) * u;
        }
        break;
    }
    case kQKV: {
        const int Hq = a.qkv.n_head * a.qkv.head_dim, kv = a.qkv.n_head_kv * a.qkv.head_dim;
        for (int idx = threadIdx.x; idx < n; idx += kThreads) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            const float* bias = a.mat.bias;
            if (gr < Hq + kv) {
                if (gr & 1) continue;
                qkv_store(a, t, gr, sum(j, t) + (bias ? bias[gr] : 0.0F), sum(j + 1, t) + (bias ? bias[gr + 1] : 0.0F),
                          true);
            } else {
                qkv_store(a, t, gr, sum(j, t) + (bias ? bias[gr] : 0.0F), 0.0F, false);
            }
        }
        break;
    }
    case kLogits: {
        for (int idx = threadIdx.x; idx < n; idx += kThreads) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            const float v = sum(j, t) + (a.mat.bias ? a.mat.bias[gr] : 0.0F);
            if (a.store_logits) a.y[static_cast<size_t>(t) * a.y_stride + gr] = v;
            lv[idx] = v;
        }
        __syncthreads();
        // one wave per token: lanes scan rows, then a wave argmax (first maximum)
        const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
        for (int t = wave; t < a.n_tok; t += kThreads / kWave) {
            float bv = -INFINITY;
            int bi = -1;
            for (int j = lane; j < nrows; j += kWave) {
                const float v = lv[t * nrows + j];
                if (bi < 0 || v > bv) {
                    bv = v;
                    bi = j;
                }
            }
            unsigned long long p = bi < 0 ? 0ull : pack_best(bv, static_cast<uint32_t>(row0 + bi));
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned long long q = __shfl_xor(p, o);
                p = q > p ? q : p;
            }
            if (lane == 0 && p != 0ull) atomicMax(a.best + t, p);
        }
        break;
    }
    default:
        break;
    }
}

// Quantized matmul. Work-group w owns rows [w*RW, w*RW + RW) and streams
// their blocks as one flat list (row-major, so contiguous in memory): quad q
// of the 64 lane quads takes flat blocks q, q + 64, ..., two per iteration
// with both loads issued first. Each block's dot (4 lanes, one per quarter)
// is quad-reduced and added to its own LDS slot; rows are then summed over
// their slots in a fixed order, so results do not depend on scheduling.
// The activation is quantized into LDS by the work-group itself (after the
// optional RMSNorm), chunk by chunk when it does not fit at once.
template <uint32_t TYPE, int NT>
__global__ __launch_bounds__(kThreads) void k_gemv_q(GemvArgs a, GemvGeom g) {
    using B = QBlock<TYPE>;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = static_cast<int>(a.mat.cols);
    const int chunk = g.chunk, nbc = chunk / 256, RW = g.rows_per_wg;
    const int n_tok = NT;  // token groups are launched with exactly NT rows
    int8_t* sq = reinterpret_cast<int8_t*>(lds_raw);
    float* sd = reinterpret_cast<float*>(lds_raw + NT * chunk);
    int16_t* ss = reinterpret_cast<int16_t*>(sd + NT * nbc);
    float* part = reinterpret_cast<float*>(ss + NT * (chunk / 16));
    float* small = part + RW * nbc * NT;  // rs[NT], red[NT*4], logits values [RW*NT]
    float* rs = small;
    float* red = small + NT;
    float* lv = red + NT * (kThreads / kWave);

    const int row0 = blockIdx.x * RW;
    const int nrows = min(RW, static_cast<int>(a.mat.rows) - row0);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int part_id = lane & 3, quad = wave * (kWave / 4) + (lane >> 2);
    const Staged st{sq, sd, ss, chunk};

    if (a.x.gain) row_rms<NT>(a.x, n_tok, K, rs, red);
    for (int i = threadIdx.x; i < RW * nbc * NT; i += kThreads) part[i] = 0.0F;

    const size_t rb = a.mat.main_row_bytes, ab = a.mat.aux_row_bytes;
    const uint8_t* main0 = a.mat.main + static_cast<size_t>(row0) * rb;
    const uint8_t* aux0 = a.mat.aux ? a.mat.aux + static_cast<size_t>(row0) * ab : nullptr;
    const int total = nrows * nbc;
    for (int c0 = 0; c0 < K; c0 += chunk) {
        const int nb = min(chunk, K - c0) / 256;
        __syncthreads();
        stage_chunk<NT>(a.x, n_tok, c0, nb, rs, sq, sd, ss, chunk);
        __syncthreads();
        for (int f0 = quad; f0 < total; f0 += 2 * kWave) {
            const int f1 = f0 + kWave;
            const int r0 = static_cast<int>((static_cast<uint64_t>(f0) * g.nbc_magic) >> 32);
            const int r1 = static_cast<int>((static_cast<uint64_t>(f1) * g.nbc_magic) >> 32);
            const int b0 = f0 - r0 * nbc, b1 = f1 - r1 * nbc;
            const bool ok0 = b0 < nb, ok1 = f1 < total && b1 < nb;
            typename B::Regs v0, v1;
            if (ok0) v0 = B::load(RowRef{main0 + r0 * rb, aux0 ? aux0 + r0 * ab : nullptr, true}, c0 / 256 + b0, part_id);
            if (ok1) v1 = B::load(RowRef{main0 + r1 * rb, aux0 ? aux0 + r1 * ab : nullptr, true}, c0 / 256 + b1, part_id);
            float s0[NT], s1[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                s0[t] = 0.0F;
                s1[t] = 0.0F;
            }
            if (ok0) B::template dot<NT>(v0, part_id, st, b0, s0);
            if (ok1) B::template dot<NT>(v1, part_id, st, b1, s1);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                s0[t] = quad_sum(s0[t]);
                s1[t] = quad_sum(s1[t]);
            }
            if (part_id == 0) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (ok0) part[f0 * NT + t] += s0[t];
                    if (ok1) part[f1 * NT + t] += s1[t];
                }
            }
        }
    }
    __syncthreads();
    gemv_epilogue<NT>(a, row0, nrows,
                      [&](int j, int t) {
                          float acc = 0.0F;
                          const float* p = part + j * nbc * NT + t;
                          for (int b = 0; b < nbc; ++b) acc += p[b * NT];
                          return acc;
                      },
                      lv);
}

// Float weights (F32/F16, small models): one wave per row, lanes over K,
// float activations (RMS-normalized in the prologue when a gain is given).
template <int NT>
__global__ __launch_bounds__(kThreads) void k_gemv_f(GemvArgs a, int32_t rows_per_wg) {
    __shared__ float rs[NT], red[NT * (kThreads / kWave)];
    __shared__ float sums[kThreads / kWave * 2][NT];
    extern __shared__ float lv_f[];
    const int K = static_cast<int>(a.mat.cols);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n_tok = a.n_tok < NT ? a.n_tok : NT;
    if (a.x.gain) row_rms<NT>(a.x, n_tok, K, rs, red);
    const int RW = rows_per_wg, row0 = blockIdx.x * RW;
    const int nrows = min(RW, static_cast<int>(a.mat.rows) - row0);
    for (int j = wave; j < RW; j += kThreads / kWave) {
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0.0F;
        if (j < nrows) {
            for (int c = lane; c < K; c += kWave) {
                const float w = dequant_elem(a.mat, static_cast<uint32_t>(row0 + j), static_cast<uint32_t>(c));
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (t < n_tok) {
                        float xv = x_row(a.x, t)[c];
                        if (a.x.gain) xv = xv * rs[t] * a.x.gain[c];
                        acc[t] += w * xv;
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = wave_sum(acc[t]);
        if (lane == 0 && j < nrows) {
#pragma unroll
            for (int t = 0; t < NT; ++t) sums[j][t] = acc[t];
        }
    }
    __syncthreads();
    GemvArgs b = a;
    b.n_tok = n_tok;
    gemv_epilogue<NT>(b, row0, nrows, [&](int j, int t) { return sums[j][t]; }, lv_f);
}

// ------------------------------------------------------------------ attention
// Split-K causal GQA flash attention (qwen2_architecture.cpp:438-464, mask
// 697-708) over the f16 caches. Work-group = (key split, kv head x query
// group, sequence); a query group is up to kAttnQPW of the G*T query rows that
// share the kv head, staged in LDS. Each wave takes 16-key tiles: for Q.K a
// quad of lanes holds one key (a quarter of its dims each) and the score is
// quad-reduced; for P.V the lanes own two head dims each. K and V of a tile
// are loaded together. The four waves' online-softmax states are merged in
// LDS; with several splits the last work-group to finish (atomic counter,
// reset by it) merges the splits' partials.
constexpr int kAttnQPW = 8;
constexpr int kAttnTile = 16;
constexpr int kAttnWgKeys = kAttnTile * (kThreads / kWave);

template <int HD>
__device__ __forceinline__ void attn_load_k(const uint16_t* krow, int hd, int qq, uint4* kr) {
    if constexpr (HD > 0) {
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) kr[c] = *reinterpret_cast<const uint4*>(krow + qq * (HD / 4) + 8 * c);
    }
}

template <int HD>
__global__ __launch_bounds__(kThreads) void k_attention(const float* __restrict__ q, const StepDev* __restrict__ step,
                                                        int32_t layer, int32_t n_head, int32_t n_head_kv,
                                                        int32_t hd_arg, int32_t splits_max, int32_t qgroups,
                                                        float* __restrict__ partial, int32_t* __restrict__ counters,
                                                        float* __restrict__ out) {
    constexpr int QPW = kAttnQPW, W = kThreads / kWave;
    constexpr int QS = (HD > 0 ? HD : 128) + 16;  // LDS row stride of a query (quarters padded by 4)
    __shared__ __align__(16) float Qs[QPW][QS];
    __shared__ __align__(16) float P[W][QPW][kAttnTile];
    __shared__ float Ms[W][QPW], Ls[W][QPW];
    __shared__ __align__(16) float Os[W][QPW][128];
    __shared__ int last;
    const int hd = HD > 0 ? HD : hd_arg;
    const int DQ = hd / 4;
    const int seq = blockIdx.z;
    if (seq >= step->n_seq) return;
    const int32_t pos0 = step->seqs[seq].pos0, len = step->seqs[seq].len, row0 = step->seqs[seq].row0;
    const int32_t capacity = step->seqs[seq].capacity;
    const int G = n_head / n_head_kv, NQ = G * len, H = n_head * hd;
    const int kvh = blockIdx.y / qgroups, qg = blockIdx.y % qgroups;
    const int q_begin = qg * QPW;
    if (q_begin >= NQ) return;
    const int nq = min(QPW, NQ - q_begin);
    const int n_keys = pos0 + len;
    int L = (n_keys + splits_max - 1) / splits_max;
    L = (L + kAttnWgKeys - 1) / kAttnWgKeys * kAttnWgKeys;
    const int n_splits = (n_keys + L - 1) / L;
    const int split = blockIdx.x;
    if (split >= n_splits) return;
    const int k0 = split * L, k1 = min(n_keys, k0 + L);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int kk = lane >> 2, qq = lane & 3;
    const float scale = 1.0F / sqrtf(static_cast<float>(hd));
    const size_t head_base = (static_cast<size_t>(layer) * n_head_kv + kvh) * capacity;
    const uint16_t* kc = step->seqs[seq].k + head_base * hd;
    const uint16_t* vc = step->seqs[seq].v + head_base * hd;

    // queries -> LDS, quarter c of row i at Qs[i][c * (DQ + 4)]
    for (int e = threadIdx.x; e < QPW * hd; e += kThreads) {
        const int i = e / hd, d = e - i * hd;
        const int qi = q_begin + min(i, nq - 1);
        const int t = qi / G, head = kvh * G + qi % G;
        Qs[i][(d / DQ) * (DQ + 4) + d % DQ] = q[static_cast<size_t>(row0 + t) * H + head * hd + d];
    }
    int limit[QPW];
#pragma unroll
    for (int i = 0; i < QPW; ++i) limit[i] = pos0 + (q_begin + min(i, nq - 1)) / G;
    __syncthreads();

    float m[QPW], l[QPW], o0[QPW], o1[QPW];
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0F;
        o0[i] = 0.0F;
        o1[i] = 0.0F;
    }
    for (int t0 = k0 + wave * kAttnTile; t0 < k1; t0 += W * kAttnTile) {
        const int key = t0 + kk;
        const int keyc = min(key, capacity - 1);
        // K quarter of this lane's key and V pairs of the tile's 16 keys, loaded together
        uint4 kr[HD > 0 ? HD / 32 : 1];
        attn_load_k<HD>(kc + static_cast<size_t>(keyc) * hd, hd, qq, kr);
        uint32_t vv[kAttnTile];
#pragma unroll
        for (int u = 0; u < kAttnTile; ++u) {
            const int kj = min(t0 + u, capacity - 1);
            vv[u] = 2 * lane < hd ? *reinterpret_cast<const uint32_t*>(vc + static_cast<size_t>(kj) * hd + 2 * lane) : 0u;
        }
        float sc[QPW];
#pragma unroll
        for (int i = 0; i < QPW; ++i) sc[i] = 0.0F;
        if constexpr (HD > 0) {
#pragma unroll
            for (int c = 0; c < HD / 32; ++c) {
                const float kf[8] = {h2f(kr[c].x), h2f(kr[c].x >> 16), h2f(kr[c].y), h2f(kr[c].y >> 16),
                                     h2f(kr[c].z), h2f(kr[c].z >> 16), h2f(kr[c].w), h2f(kr[c].w >> 16)};
#pragma unroll
                for (int i = 0; i < QPW; ++i) {
                    const float4 qa = *reinterpret_cast<const float4*>(&Qs[i][qq * (DQ + 4) + 8 * c]);
                    const float4 qb = *reinterpret_cast<const float4*>(&Qs[i][qq * (DQ + 4) + 8 * c + 4]);
                    sc[i] += kf[0] * qa.x + kf[1] * qa.y + kf[2] * qa.z + kf[3] * qa.w + kf[4] * qb.x + kf[5] * qb.y +
                             kf[6] * qb.z + kf[7] * qb.w;
                }
            }
        } else {
            const uint16_t* kq = kc + static_cast<size_t>(keyc) * hd + qq * DQ;
            for (int d = 0; d < DQ; ++d) {
                const float kf = h2f(kq[d]);
#pragma unroll
                for (int i = 0; i < QPW; ++i) sc[i] += kf * Qs[i][qq * (DQ + 4) + d];
            }
        }
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            const float full = quad_sum(sc[i]);
            const bool vis = i < nq && key < k1 && key <= limit[i];
            const float sv = vis ? full * scale : -INFINITY;
            const float m_new = fmaxf(m[i], wave_max(sv));
            float p = 0.0F, alpha = 1.0F;
            if (m_new != -INFINITY) {
                alpha = m[i] == -INFINITY ? 0.0F : expf(m[i] - m_new);
                p = vis ? expf(sv - m_new) : 0.0F;
            }
            l[i] = l[i] * alpha + (qq == 0 ? p : 0.0F);
            o0[i] *= alpha;
            o1[i] *= alpha;
            m[i] = m_new;
            if (qq == 0) P[wave][i][kk] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int u4 = 0; u4 < kAttnTile / 4; ++u4) {
            float v0[4], v1[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v0[u] = h2f(vv[4 * u4 + u]);
                v1[u] = h2f(vv[4 * u4 + u] >> 16);
            }
#pragma unroll
            for (int i = 0; i < QPW; ++i) {
                const float4 pv = *reinterpret_cast<const float4*>(&P[wave][i][4 * u4]);
                o0[i] += pv.x * v0[0] + pv.y * v0[1] + pv.z * v0[2] + pv.w * v0[3];
                o1[i] += pv.x * v1[0] + pv.y * v1[1] + pv.z * v1[2] + pv.w * v1[3];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // merge the four waves
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
        const float ls = wave_sum(l[i]);
        if (lane == 0) {
            Ms[wave][i] = m[i];
            Ls[wave][i] = ls;
        }
        if (2 * lane < hd) {
            Os[wave][i][2 * lane] = o0[i];
            Os[wave][i][2 * lane + 1] = o1[i];
        }
    }
    __syncthreads();
    const int half_hd = hd / 2;
    for (int e = threadIdx.x; e < nq * half_hd; e += kThreads) {
        const int i = e / half_hd, dp = e - i * half_hd;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, Ms[w][i]);
        float Lsum = 0.0F, a0 = 0.0F, a1 = 0.0F;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float f = Ms[w][i] == -INFINITY ? 0.0F : expf(Ms[w][i] - M);
                Lsum += f * Ls[w][i];
                a0 += f * Os[w][i][2 * dp];
                a1 += f * Os[w][i][2 * dp + 1];
            }
        }
        const int qi = q_begin + i;
        const int t = qi / G, head = kvh * G + qi % G;
        if (n_splits == 1) {
            float* o = out + static_cast<size_t>(row0 + t) * H + head * hd;
            o[2 * dp] = a0 / Lsum;
            o[2 * dp + 1] = a1 / Lsum;
        } else {
            float* dst = partial + ((static_cast<size_t>(row0 + t) * n_head + head) * splits_max + split) * (hd + 2);
            if (dp == 0) {
                dst[0] = M;
                dst[1] = Lsum;
            }
            dst[2 + 2 * dp] = a0;
            dst[3 + 2 * dp] = a1;
        }
    }
    if (n_splits == 1) return;
    __threadfence();
    __syncthreads();
    int32_t* counter = counters + (static_cast<size_t>(seq) * n_head_kv + kvh) * qgroups + qg;
    if (threadIdx.x == 0) last = atomicAdd(counter, 1) == n_splits - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int e = threadIdx.x; e < nq * half_hd; e += kThreads) {
        const int i = e / half_hd, dp = e - i * half_hd;
        const int qi = q_begin + i;
        const int t = qi / G, head = kvh * G + qi % G;
        const float* base = partial + (static_cast<size_t>(row0 + t) * n_head + head) * splits_max * (hd + 2);
        float M = -INFINITY;
        for (int sp = 0; sp < n_splits; ++sp) M = fmaxf(M, base[sp * (hd + 2)]);
        float Lsum = 0.0F, a0 = 0.0F, a1 = 0.0F;
        for (int sp = 0; sp < n_splits; ++sp) {
            const float* src = base + sp * (hd + 2);
            const float ms = src[0];
            const float f = ms == -INFINITY ? 0.0F : expf(ms - M);
            Lsum += f * src[1];
            a0 += f * src[2 + 2 * dp];
            a1 += f * src[3 + 2 * dp];
        }
        float* o = out + static_cast<size_t>(row0 + t) * H + head * hd;
        o[2 * dp] = a0 / Lsum;
        o[2 * dp + 1] = a1 / Lsum;
    }
    if (threadIdx.x == 0) *counter = 0;
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

// Host-side geometry: the activation chunk fits kGemvActBytes of LDS, the
// per-block partial sums kGemvPartBytes, and the row count per work-group
// aims at kGemvTargetWgs work-groups.
constexpr int kGemvActBytes = 28672;
constexpr int kGemvPartBytes = 16384;
constexpr int kGemvTargetWgs = 512;
constexpr int kGemvFloatRows = 2 * kGluGroup;

GemvGeom gemv_geom(const GemvArgs& a, int nt, size_t& lds) {
    const int K = static_cast<int>(a.mat.cols);
    const double per_value = nt * (1.0 + 4.0 / 256.0 + 2.0 / 16.0);
    int chunk = static_cast<int>(kGemvActBytes / per_value) / 256 * 256;
    if (chunk < 256) chunk = 256;
    const int k_round = (K + 255) / 256 * 256;
    if (chunk > k_round) chunk = k_round;
    const int nbc = chunk / 256;
    const int rows = static_cast<int>(a.mat.rows);
    int rw = (rows + kGemvTargetWgs - 1) / kGemvTargetWgs;
    const int cap = kGemvPartBytes / (nbc * nt * 4);
    if (rw > cap) rw = cap;
    if (rw < 1) rw = 1;
    const int align = a.mode == kSwiGLU ? 2 * kGluGroup : a.mode == kQKV ? 2 : 1;
    rw = (rw + align - 1) / align * align;
    GemvGeom g;
    g.rows_per_wg = rw;
    g.chunk = chunk;
    g.nbc_magic = ((1ull << 32) + static_cast<uint64_t>(nbc) - 1) / static_cast<uint64_t>(nbc);
    lds = static_cast<size_t>(nt) * chunk + static_cast<size_t>(nt) * nbc * 4 + static_cast<size_t>(nt) * chunk / 8 +
          static_cast<size_t>(rw) * nbc * nt * 4 + static_cast<size_t>(nt + nt * (kThreads / kWave) + rw * nt) * 4;
    return g;
}

template <uint32_t TYPE, int NT>
void gemv_q(const GemvArgs& a, hipStream_t stream) {
    size_t lds = 0;
    const GemvGeom g = gemv_geom(a, NT, lds);
    const int grid = (static_cast<int>(a.mat.rows) + g.rows_per_wg - 1) / g.rows_per_wg;
    hipLaunchKernelGGL((k_gemv_q<TYPE, NT>), dim3(grid), dim3(kThreads), lds, stream, a, g);
    check(hipGetLastError(), "gemv launch");
}

template <uint32_t TYPE>
void gemv_q_nt(const GemvArgs& a, hipStream_t stream) {
    switch (a.n_tok) {
    case 1: gemv_q<TYPE, 1>(a, stream); break;
    case 2: gemv_q<TYPE, 2>(a, stream); break;
    case 3: gemv_q<TYPE, 3>(a, stream); break;
    case 4: gemv_q<TYPE, 4>(a, stream); break;
    case 5: gemv_q<TYPE, 5>(a, stream); break;
    case 6: gemv_q<TYPE, 6>(a, stream); break;
    case 7: gemv_q<TYPE, 7>(a, stream); break;
    case 8: gemv_q<TYPE, 8>(a, stream); break;
    default: throw std::invalid_argument("gemv token group must be 1..8");
    }
}

template <int NT>
void gemv_f(const GemvArgs& a, hipStream_t stream) {
    const int grid = (static_cast<int>(a.mat.rows) + kGemvFloatRows - 1) / kGemvFloatRows;
    const size_t lds = static_cast<size_t>(kGemvFloatRows) * NT * sizeof(float);
    hipLaunchKernelGGL((k_gemv_f<NT>), dim3(grid), dim3(kThreads), lds, stream, a, kGemvFloatRows);
    check(hipGetLastError(), "gemv launch");
}

}  // namespace

void launch_gemv(const GemvArgs& a_in, hipStream_t stream) {
    const uint32_t type = a_in.mat.type;
    const bool quantized = type == 7 || type == 9 || type == 11 || type == 13;
    if (quantized && (a_in.mat.cols % kActBlock != 0 || a_in.x.stride % 4 != 0)) {
        throw std::invalid_argument("quantized matmul needs rows of a multiple of 256 values");
    }
    if ((a_in.mode == kSwiGLU && a_in.mat.rows % (2 * kGluGroup) != 0) || (a_in.mode == kQKV && a_in.mat.rows % 2 != 0)) {
        throw std::invalid_argument("matmul rows do not fit the fused row layout");
    }
    // token groups of at most 8 rows
    for (int t0 = 0; t0 < a_in.n_tok; t0 += 8) {
        GemvArgs a = a_in;
        a.n_tok = a_in.n_tok - t0 < 8 ? a_in.n_tok - t0 : 8;
        if (a.x.gather) a.x.gather += t0;
        else a.x.x += static_cast<size_t>(t0) * a.x.stride;
        if (a.y) a.y += static_cast<size_t>(t0) * a.y_stride;
        if (a.best) a.best += t0;
        if (a.mode == kQKV) {
            a.qkv.row0 += t0;
            a.qkv.q += static_cast<size_t>(t0) * a.qkv.n_head * a.qkv.head_dim;
        }
        if (!quantized) {
            switch (a.n_tok) {
            case 1: gemv_f<1>(a, stream); break;
            case 2: gemv_f<2>(a, stream); break;
            case 3: case 4: gemv_f<4>(a, stream); break;
            default: gemv_f<8>(a, stream); break;
            }
            continue;
        }
        switch (type) {
        case 11: gemv_q_nt<11>(a, stream); break;
        case 13: gemv_q_nt<13>(a, stream); break;
        case 9: gemv_q_nt<9>(a, stream); break;
        case 7: gemv_q_nt<7>(a, stream); break;
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

int32_t attention_splits(int32_t capacity) {
    const int32_t s = (capacity + kAttnWgKeys - 1) / kAttnWgKeys;
    return s < 1 ? 1 : (s > 32 ? 32 : s);
}

size_t attention_partial_floats(int32_t rows, int32_t n_head, int32_t head_dim, int32_t splits) {
    return static_cast<size_t>(rows) * n_head * splits * (head_dim + 2);
}

void launch_attention(const float* q, const StepDev* step, int32_t max_len, int32_t n_seq, int32_t layer,
                      int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits, float* partial,
                      int32_t* counters, float* out, hipStream_t stream) {
    const int G = n_head / n_head_kv;
    const int qgroups = (G * max_len + kAttnQPW - 1) / kAttnQPW;
    if (head_dim > 2 * kWave || head_dim % 4 != 0) {
        throw std::invalid_argument("attention supports head dims that are multiples of 4 up to 128");
    }
    if (qgroups > kMaxAttnQGroups) throw std::invalid_argument("attention step has too many query rows per kv head");
    dim3 grid(splits, n_head_kv * qgroups, n_seq), block(kThreads);
    if (head_dim == 128) {
        hipLaunchKernelGGL(k_attention<128>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, head_dim, splits,
                           qgroups, partial, counters, out);
    } else if (head_dim == 64) {
        hipLaunchKernelGGL(k_attention<64>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, head_dim, splits,
                           qgroups, partial, counters, out);
    } else {
        hipLaunchKernelGGL(k_attention<0>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, head_dim, splits,
                           qgroups, partial, counters, out);
    }
    check(hipGetLastError(), "attention launch");
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
