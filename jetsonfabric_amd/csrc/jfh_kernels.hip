// gfx950 kernels for the Qwen2 stage forward (decode, draft verify, prefill).
//
// Graph being implemented: runtime/engines/native/src/qwen2_architecture.cpp:522-598.
// Weights keep their GGML block encodings, rearranged into 16-row x 256-value
// tiles (jfh_kernels.hpp, tile_bytes) so that every wave-wide load covers
// 1 KiB of contiguous memory. The matmuls quantize each activation row to int8
// in 256-value blocks (d = amax/127) and use v_dot4 integer dot products
// against the unpacked codes, the scheme GGML's CPU backend uses for K-quants
// (activation q8 blocks + integer dot).
#include "jfh_kernels.hpp"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace jfh::gpu {
namespace {

constexpr int kWave = 64;

// Pointers read from device memory (the step description) are generic to
// the compiler; routing them through the global address space lets it use
// global (not FLAT) memory instructions, whose completion is tracked apart
// from LDS traffic.
template <typename T>
using global_ptr = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ global_ptr<T> as_global(T* p) {
    return (global_ptr<T>) p;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load_u4(global_ptr<const uint16_t> p) {
    const u32x4 v = *(global_ptr<const u32x4>) p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

__host__ __device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16 & 0xFFFFu)));
}

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// DPP lane exchange within rows of 16 lanes (quad_perm / row_ror controls).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Whole-wave reductions: DPP within each 16-lane row (xor 1, xor 2, rotate 4,
// rotate 8), then the four row results combined from lanes 0/16/32/48 in a
// fixed order, so every lane gets the same value.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over the 4 lanes of a quad (DPP quad permutations [1,0,3,2], [2,3,0,1]).
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), acc, false);
}

__device__ __forceinline__ uint32_t u4_word(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__host__ __device__ __forceinline__ int sext8(uint32_t v) { return static_cast<int>(static_cast<int8_t>(v & 0xFFu)); }

// Q4_K 6-bit scale/min of sub-block j from the header's scale bytes (h.y..w).
__host__ __device__ __forceinline__ void q4k_scale_min(const uint4& h, int j, int& sc, int& m) {
    if (j < 4) {
        sc = (h.y >> (8 * j)) & 63;
        m = (h.z >> (8 * j)) & 63;
    } else {
        const int k = j - 4;
        sc = ((h.w >> (8 * k)) & 0xF) | (((h.y >> (8 * k + 6)) & 3) << 4);
        m = ((h.w >> (8 * k + 4)) & 0xF) | (((h.z >> (8 * k + 6)) & 3) << 4);
    }
}

__host__ __device__ __forceinline__ uint32_t byte_at(const uint8_t* p) { return *p; }

__host__ __device__ __forceinline__ uint32_t u16_at(const uint8_t* p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

__host__ __device__ __forceinline__ uint32_t u32_at(const uint8_t* p) {
    return u16_at(p) | (u16_at(p + 2) << 16);
}

// ------------------------------------------------------------------ element dequantization
// Exact GGML dequantization of value k of row i of one tile; the arithmetic
// order matches the GGML formulas: Q4_K (d*sc)*q - dmin*m, Q6_K
// (d*sc)*(q-32), Q8_0 q*d, Q2_K (d*sc)*q - dmin*m.
__host__ __device__ float tile_value(uint32_t type, const uint8_t* tile, uint32_t i, uint32_t k) {
    const uint32_t g = k / 64, v = k % 64, l = i + 16 * g;
    auto code_dword = [&](uint32_t base, uint32_t idx) { return u32_at(tile + base + ((idx / 4) * 64 + l) * 16 + 4 * (idx % 4)); };
    switch (type) {
    case 11: {
        const uint8_t* hb = tile + 16 * i;
        const float d = h2f(u16_at(hb)), dmin = h2f(u16_at(hb + 2));
        const uint32_t f = byte_at(hb + 4 + 3 * g) | (byte_at(hb + 5 + 3 * g) << 8) | (byte_at(hb + 6 + 3 * g) << 16);
        const uint32_t hi = v >= 32 ? 1u : 0u;
        const int sc = static_cast<int>((f >> (6 * hi)) & 63), mn = static_cast<int>((f >> (12 + 6 * hi)) & 63);
        const uint32_t b = v % 32;
        const uint32_t byte = byte_at(tile + 256 + ((b / 16) * 64 + l) * 16 + b % 16);
        const int q = hi ? static_cast<int>(byte >> 4) : static_cast<int>(byte & 0xF);
        const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(mn);
        return d1 * static_cast<float>(q) - m1;
    }
    case 13: {
        const float d = h2f(u16_at(tile + 2 * i));
        const int sc = sext8(byte_at(tile + 32 + 16 * i + k / 16));
        const uint32_t w = v % 8;
        const uint32_t lbyte = (code_dword(288, v / 8) >> (8 * (w % 4))) & 0xFF;
        const uint32_t low4 = w >= 4 ? (lbyte >> 4) : (lbyte & 0xF);
        const uint32_t m = v / 16, r = (v % 16) / 4, e = v % 4;
        const uint32_t h2 = (code_dword(288, 8 + m) >> (8 * e + 2 * r)) & 3;
        const int q = static_cast<int>(low4 | (h2 << 4)) - 32;
        const float ds = d * static_cast<float>(sc);
        return ds * static_cast<float>(q);
    }
    case 7: {
        const float d = h2f(u16_at(tile + 16 * i + 2 * (k / 32)));
        const int q = sext8(byte_at(tile + 256 + ((v / 16) * 64 + l) * 16 + v % 16));
        return static_cast<float>(q) * d;
    }
    case 9: {
        const float d = h2f(u16_at(tile + 4 * i)), dmin = h2f(u16_at(tile + 4 * i + 2));
        const uint32_t sb = byte_at(tile + 64 + 16 * i + k / 16);
        const uint32_t m = v / 16, r = (v % 16) / 4, e = v % 4;
        const int q = static_cast<int>((code_dword(320, m) >> (8 * e + 2 * r)) & 3);
        const float dl = d * static_cast<float>(sb & 0xF), ml = dmin * static_cast<float>(sb >> 4);
        return dl * static_cast<float>(q) - ml;
    }
    default:
        return 0.0F;
    }
}

__device__ float dequant_elem(const DMat& m, uint32_t row, uint32_t c) {
    if (m.type == 1) return reinterpret_cast<const float*>(m.data + static_cast<size_t>(row) * m.row_bytes)[c];
    if (m.type == 2) return h2f(reinterpret_cast<const uint16_t*>(m.data + static_cast<size_t>(row) * m.row_bytes)[c]);
    const uint32_t nb = m.cols / 256;
    const uint8_t* tile = m.data + (static_cast<size_t>(row / 16) * nb + c / 256) * tile_bytes(m.type);
    return tile_value(m.type, tile, row % 16, c % 256);
}

__global__ __launch_bounds__(256) void k_dequant_rows(DMat m, int32_t row0, float* out) {
    const uint32_t r = blockIdx.y;
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c < m.cols) out[static_cast<size_t>(r) * m.cols + c] = dequant_elem(m, row0 + r, c);
}

// ------------------------------------------------------------------ embedding
__global__ __launch_bounds__(256) void k_embed(DMat table, const StepDev* step, float* h, int32_t H,
                                               unsigned long long* best, int32_t n_best) {
    const int r = blockIdx.y;
    if (blockIdx.x == 0 && r == 0) {
        for (int i = threadIdx.x; i < n_best; i += 256) best[i] = 0ull;
    }
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (r < step->n_rows && c < H) {
        h[static_cast<size_t>(r) * H + c] = dequant_elem(table, static_cast<uint32_t>(step->token[r]), c);
    }
}

// ------------------------------------------------------------------ activation quantization
// Quantizes 256 values held 4 per lane (values 4L..4L+3 in lane L) by one
// wave: d = amax/127, q = roundf(x * (1/d)), plus the sum of every 16 codes.
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
    sum += dpp_i<0xB1>(sum);
    sum += dpp_i<0x4E>(sum);
    if ((lane & 3) == 0) s[lane >> 2] = static_cast<int16_t>(sum);
    if (lane == 0) *d = db;
}

// A float rounded to the nearest f16 value (the stored scale of a 32-value block).
__device__ __forceinline__ float round_f16(float v) { return static_cast<float>(static_cast<_Float16>(v)); }

// Code of one value of a block given id = 1/d' (d' = amax/127): roundf(x * id),
// clamped to +-127 (the 256-value rule per block).
__device__ __forceinline__ int quant_code(float v, float id) {
    const float r = fminf(127.0F, fmaxf(-127.0F, roundf(v * id)));
    return static_cast<int>(r);
}

// The same rule over 32-value blocks: the wave's 256 values (4 per lane) form
// eight blocks of eight lanes (block k = lanes 8k .. 8k+7). d[k] receives
// amax/127, rounded to f16 unless RAW (a normalized row's scale is rounded
// after its rms factor is applied); s the sum of every 16 codes.
template <bool RAW>
__device__ __forceinline__ void quant_block_wave32(const float v[4], int lane, int8_t* q, float* d, int16_t* s) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));
    amax = fmaxf(amax, dpp_f<0x4E>(amax));
    amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror: the other quad of the eight lanes
    const float db = amax / 127.0F;
    const float id = db > 0.0F ? 1.0F / db : 0.0F;
    int qi[4];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qi[i] = quant_code(v[i], id);
        sum += qi[i];
    }
    const uint32_t packed = (qi[0] & 0xFF) | ((qi[1] & 0xFF) << 8) | ((qi[2] & 0xFF) << 16) | ((qi[3] & 0xFF) << 24);
    reinterpret_cast<uint32_t*>(q)[lane] = packed;
    sum += dpp_i<0xB1>(sum);
    sum += dpp_i<0x4E>(sum);
    if ((lane & 3) == 0) s[lane >> 2] = static_cast<int16_t>(sum);
    if ((lane & 7) == 0) d[lane >> 3] = RAW ? db : round_f16(db);
}
#pragma clang fp contract(on)

__device__ __forceinline__ const float* x_row(const XIn& x, int t) {
    return x.x + static_cast<size_t>(x.gather ? x.gather[t] : t) * x.stride;
}

// 1/sqrt(mean(x^2) + eps) of each token row (qwen2_architecture.cpp:373-376),
// reduced by the whole work-group into rs[t]; red holds NT * waves floats.
template <int NT, int NTHR>
__device__ void row_rms(const XIn& x, int n_tok, int K, float* rs, float* red) {
    constexpr int W = NTHR / kWave;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    for (int t = 0; t < n_tok; ++t) {
        const float* xr = x_row(x, t);
        float ss = 0.0F;
        for (int i0 = 4 * threadIdx.x; i0 < K; i0 += 4 * 4 * NTHR) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * 4 * NTHR;
                v[u] = i < K ? *reinterpret_cast<const float4*>(xr + i) : make_float4(0.0F, 0.0F, 0.0F, 0.0F);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[t * W + wave] = ss;
    }
    __syncthreads();
    if (threadIdx.x < static_cast<unsigned>(n_tok)) {
        const int t = threadIdx.x;
        float ss = 0.0F;
        for (int w = 0; w < W; ++w) ss += red[t * W + w];
        rs[t] = 1.0F / sqrtf(ss / static_cast<float>(K) + x.eps);
    }
    __syncthreads();
}

// Quantizes values [c0, c0 + nb*256) of every token row into the LDS chunk
// (q [t][chunk] permuted per block, d [t][chunk/ABLK], s [t][chunk/16]), one
// wave per 256 values, loads issued kStageBatch blocks at a time; A32 puts the
// values in 32-value blocks (eight scales per 256 values). With a gain
// (RMSNorm input) the codes are those of x * gain and ssq[t][b] receives the
// 256 values' sum of x^2; the block scales are multiplied by the row's 1/rms
// afterwards (finish_norm), so one pass over x serves both.
//
// The first batch of a pass is loaded ahead (stage_f32_load) and handed in:
// a wave's loads complete in issue order, so activations requested before the
// weight prefetch are not held up behind the weight tiles.
constexpr int kStageBatch = 4;        // blocks per wave of a staging batch (normalized rows: values + gains)
constexpr int kStageBatchFloat = 10;  // blocks per wave of a batch of plain float rows

typedef float f32x4 __attribute__((ext_vector_type(4)));

// A staging batch of NB blocks per wave lives in f32x4 r[2 NB]: the lane's 4
// values of each block, then (GAIN) the matching gains. Loads the blocks j0,
// j0 + W, ... (indices clamped so that every load is issued unconditionally).
template <int NTHR, int NB, bool GAIN>
__device__ __forceinline__ void stage_f32_load(const XIn& x, int n_tok, int c0, int nb, int j0, f32x4 (&r)[2 * NB]) {
    constexpr int W = NTHR / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int total = n_tok * nb;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int j = min(j0 + u * W, total - 1);
        const int t = j / nb, b = j - t * nb;
        const int c = c0 + b * 256 + 4 * lane;
        r[u] = *reinterpret_cast<const f32x4*>(x_row(x, t) + c);
        if constexpr (GAIN) r[NB + u] = *reinterpret_cast<const f32x4*>(x.gain + c);
    }
}

#pragma clang fp contract(off)
template <int NTHR, int NB, bool GAIN, bool A32>
__device__ __forceinline__ void stage_f32_store(int n_tok, int nb, int j0, const f32x4 (&r)[2 * NB], int8_t* sq,
                                                float* sd, int16_t* ss, float* ssq, int chunk) {
    constexpr int W = NTHR / kWave;
    constexpr int DB = A32 ? 8 : 1;  // scales per 256 values
    const int lane = threadIdx.x & (kWave - 1);
    const int total = n_tok * nb;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int j = j0 + u * W;
        if (j < total) {
            const int t = j / nb, b = j - t * nb;
            float vv[4] = {r[u].x, r[u].y, r[u].z, r[u].w};
            if constexpr (GAIN) {
                const float sq2 = wave_sum(vv[0] * vv[0] + vv[1] * vv[1] + vv[2] * vv[2] + vv[3] * vv[3]);
                if (lane == 0) ssq[t * nb + b] = sq2;
                vv[0] = vv[0] * r[NB + u].x;
                vv[1] = vv[1] * r[NB + u].y;
                vv[2] = vv[2] * r[NB + u].z;
                vv[3] = vv[3] * r[NB + u].w;
            }
            float* dst_d = sd + t * (chunk / 256 * DB) + b * DB;
            if constexpr (A32) {
                quant_block_wave32<GAIN>(vv, lane, sq + t * chunk + b * 256, dst_d, ss + t * (chunk / 16) + b * 16);
            } else {
                quant_block_wave(vv, lane, sq + t * chunk + b * 256, dst_d, ss + t * (chunk / 16) + b * 16);
            }
        }
    }
}
#pragma clang fp contract(on)

// Stages a pass whose first batch (blocks wave, wave + W, ...) is already loaded.
template <int NTHR, int NB, bool GAIN, bool A32>
__device__ __forceinline__ void stage_f32(const XIn& x, int n_tok, int c0, int nb, int8_t* sq, float* sd, int16_t* ss,
                                          float* ssq, int chunk, const f32x4 (&first)[2 * NB]) {
    constexpr int W = NTHR / kWave;
    const int wave = threadIdx.x / kWave;
    const int total = n_tok * nb;
    stage_f32_store<NTHR, NB, GAIN, A32>(n_tok, nb, wave, first, sq, sd, ss, ssq, chunk);
    for (int j0 = wave + NB * W; j0 < total; j0 += NB * W) {
        f32x4 r[2 * NB];
        stage_f32_load<NTHR, NB, GAIN>(x, n_tok, c0, nb, j0, r);
        stage_f32_store<NTHR, NB, GAIN, A32>(n_tok, nb, j0, r, sq, sd, ss, ssq, chunk);
    }
}

// After stage_f32 with a gain over the whole row (nb 256-value pieces): rs =
// 1/sqrt(sum(x^2)/K + eps) per token (piece sums added in order) scales the
// token's block scales (qwen2_architecture.cpp:373-376); 32-value block scales
// are then rounded to f16. Every thread that scales a block computes its
// token's rs itself (the same sums in the same order), so one barrier
// separates the staging from the scaling and the matmul's own barrier the
// scaling from the first dot.
#pragma clang fp contract(off)
template <int NTHR, bool A32>
__device__ void finish_norm(int n_tok, int nb, int K, float eps, const float* ssq, float* sd, int chunk) {
    constexpr int DB = A32 ? 8 : 1;
    __syncthreads();
    for (int i = threadIdx.x; i < n_tok * nb * DB; i += NTHR) {
        const int t = i / (nb * DB), b = i - t * (nb * DB);
        float sum = 0.0F;
        for (int c = 0; c < nb; ++c) sum += ssq[t * nb + c];
        const float rs = 1.0F / sqrtf(sum / static_cast<float>(K) + eps);
        const float v = sd[t * (chunk / 256 * DB) + b] * rs;
        sd[t * (chunk / 256 * DB) + b] = A32 ? round_f16(v) : v;
    }
}
#pragma clang fp contract(on)

// Copies values [c0, c0 + nb*256) of pre-quantized rows into the LDS chunk.
// Batch b of a thread holds code pieces tid + (P b + u) NTHR (uint4, u < P),
// sum piece tid + b NTHR (uint4 of 8 int16) and block scale tid + b NTHR (A32:
// scale piece tid + b NTHR, a uint4 of four 32-value block scales); indices
// are clamped so that every load is issued unconditionally. As with
// stage_f32, the first batch is loaded ahead of the weights.
template <int P>
using StageA8Regs = u32x4[P + 2];

template <int NTHR, int P, bool A32>
__device__ __forceinline__ void stage_act8_load(const Act8& xq, int n_tok, int c0, int nb, int batch,
                                                StageA8Regs<P>& r) {
    const int tid = threadIdx.x, n16 = nb * 16, nq = n_tok * n16, ns = n_tok * nb * 2, nd = n_tok * nb;
#pragma unroll
    for (int u = 0; u < P; ++u) {
        const int i = min(tid + (P * batch + u) * NTHR, nq - 1);
        const int t = i / n16, k = i - t * n16;
        r[u] = *reinterpret_cast<const u32x4*>(xq.q + static_cast<size_t>(t) * xq.K + c0 + 16 * k);
    }
    {
        const int i = min(tid + batch * NTHR, ns - 1);
        const int t = i / (2 * nb), k = i - t * 2 * nb;
        r[P] = *reinterpret_cast<const u32x4*>(xq.s + static_cast<size_t>(t) * (xq.K / 16) + c0 / 16 + 8 * k);
        if constexpr (A32) {
            r[P + 1] = *reinterpret_cast<const u32x4*>(xq.d + static_cast<size_t>(t) * (xq.K / 32) + c0 / 32 + 4 * k);
        }
    }
    if constexpr (!A32) {
        const int i = min(tid + batch * NTHR, nd - 1);
        const int t = i / nb, b = i - t * nb;
        r[P + 1].x = __float_as_uint(xq.d[static_cast<size_t>(t) * (xq.K / 256) + c0 / 256 + b]);
    }
}

template <int NTHR, int P, bool A32>
__device__ __forceinline__ void stage_act8_store(int n_tok, int nb, int batch, const StageA8Regs<P>& r, int8_t* sq,
                                                 float* sd, int16_t* ss, int chunk) {
    const int tid = threadIdx.x, n16 = nb * 16, nq = n_tok * n16, ns = n_tok * nb * 2, nd = n_tok * nb;
#pragma unroll
    for (int u = 0; u < P; ++u) {
        const int i = tid + (P * batch + u) * NTHR;
        if (i < nq) {
            const int t = i / n16, k = i - t * n16;
            reinterpret_cast<u32x4*>(sq + t * chunk)[k] = r[u];
        }
    }
    const int i = tid + batch * NTHR;
    if (i < ns) {
        const int t = i / (2 * nb), k = i - t * 2 * nb;
        reinterpret_cast<u32x4*>(ss + t * (chunk / 16))[k] = r[P];
        if constexpr (A32) reinterpret_cast<u32x4*>(sd + t * (chunk / 32))[k] = r[P + 1];
    }
    if constexpr (!A32) {
        if (i < nd) {
            const int t = i / nb, b = i - t * nb;
            sd[t * (chunk / 256) + b] = __uint_as_float(r[P + 1].x);
        }
    }
}

template <int NTHR, int P, bool A32>
__device__ __forceinline__ void stage_act8(const Act8& xq, int n_tok, int c0, int nb, int8_t* sq, float* sd,
                                           int16_t* ss, int chunk, const StageA8Regs<P>& first) {
    const int nq = n_tok * nb * 16, ns = n_tok * nb * 2;
    stage_act8_store<NTHR, P, A32>(n_tok, nb, 0, first, sq, sd, ss, chunk);
    for (int batch = 1; batch * P * NTHR < nq || batch * NTHR < ns; ++batch) {
        StageA8Regs<P> r;
        stage_act8_load<NTHR, P, A32>(xq, n_tok, c0, nb, batch, r);
        stage_act8_store<NTHR, P, A32>(n_tok, nb, batch, r, sq, sd, ss, chunk);
    }
}

// ------------------------------------------------------------------ tile dot products
// Lane (i = lane % 16, g = lane / 16) of a wave holds row i's values
// 64 g .. 64 g + 63 of one tile (whole sub-blocks of every type); for every
// token it computes the integer dots of those codes with the int8
// activation values 64 g .. 64 g + 63 of the block (LDS) and adds its share
// of the block's scaled sum to acc[t].
struct XLds {
    const int8_t* q;    // token 0, block start + 64 g
    const float* d;     // token 0 block scale
    const int16_t* s;   // token 0 block sums (16 per block)
    int32_t q_stride;   // bytes between tokens
    int32_t d_stride;   // floats between tokens
    int32_t s_stride;   // int16 between tokens
};

__device__ __forceinline__ void load_x(const XLds& x, int t, uint32_t (&xw)[16]) {
    const uint4* p = reinterpret_cast<const uint4*>(x.q + t * x.q_stride);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint4 v = p[u];
        xw[4 * u] = v.x;
        xw[4 * u + 1] = v.y;
        xw[4 * u + 2] = v.z;
        xw[4 * u + 3] = v.w;
    }
}

__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }


template <uint32_t TYPE>
struct Tile;

// The float step of a Q4_K / Q2_K tile for one token: acc + xd * (d * isum -
// dmin * msum), with the fused products as written, applied once per tile to
// the integer totals over all of the tile's sub-blocks (GGML's super-block
// sums, ggml_vec_dot_q4_K_q8_K / _q2_K_q8_K; Q6_K likewise sums sc * dot over
// its sixteen sub-blocks before its one step). The decode, token quad and wide
// matmuls all use it, so they round alike.
__device__ __forceinline__ float q4k_term(float acc, float xd, float d, float dmin, int isum, int msum) {
    const float t = __builtin_fmaf(d, static_cast<float>(isum), -(dmin * static_cast<float>(msum)));
    return __builtin_fmaf(xd, t, acc);
}

// q4k_term with the min sum given as the float of that integer
__device__ __forceinline__ float q4k_term_f(float acc, float xd, float d, float dmin, int isum, float msum) {
    const float t = __builtin_fmaf(d, static_cast<float>(isum), -(dmin * msum));
    return __builtin_fmaf(xd, t, acc);
}


// The term of one 32-value activation block b of a Q8_0 tile (GGML block b of
// the row's 256 values) for one (row, token), from its integer dot A:
// A * (dw * xd) (GGML's q8_0 x q8_0 product). Lane group g's partial is
// term(2 g) + term(2 g + 1) and the tile's total (p0 + p1) + (p2 + p3), added
// to the running sum once per tile. Every path (decode dot, token quads,
// wide) evaluates these expressions as written, so their rows agree bit for
// bit.
#pragma clang fp contract(off)
__device__ __forceinline__ float q8_term32(float xd, float dw, int A) { return static_cast<float>(A) * (dw * xd); }
__device__ __forceinline__ float pair_sum(float a, float b) { return a + b; }
__device__ __forceinline__ float tile_total(float p0, float p1, float p2, float p3) { return (p0 + p1) + (p2 + p3); }
// The decode lane's partial p (lane group g = lane / 16) -> the tile's total
// in lane group 0's lanes: lanes i, i + 16, i + 32, i + 48 hold p0 .. p3 of row i.
__device__ __forceinline__ float lane_tile_total(float p) {
    const float h = p + __shfl_xor(p, 16);  // p0 + p1 (lane groups 0, 1), p2 + p3 (2, 3)
    return h + __shfl_xor(h, 32);
}
#pragma clang fp contract(on)

// Q4_K: header of row i | codes: the lane's 32 qs bytes (sub-blocks 2g, 2g+1).
// The lane reads d|dmin and the 8 header bytes that hold its 24-bit scale
// field (header byte 4 + 3g) starting at the enclosing word.
template <>
struct Tile<11> {
    struct Regs {
        uint4 w0, w1;
        uint2 f;
        uint32_t dd;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        const int i = lane & 15, g = lane >> 4;
        r.dd = *reinterpret_cast<const uint32_t*>(t + 16 * i);
        r.f = *reinterpret_cast<const uint2*>(t + 16 * i + 4 + 4 * ((3 * g) >> 2));
        r.w0 = *reinterpret_cast<const uint4*>(t + 256 + 16 * lane);
        r.w1 = *reinterpret_cast<const uint4*>(t + 1280 + 16 * lane);
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int g, const XLds& x, int nt, float* acc) {
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        // the lane group's 24-bit field: sc 2g | sc 2g+1 | m 2g | m 2g+1
        const uint32_t f = __builtin_amdgcn_alignbyte(r.f.y, r.f.x, (3 * g) & 3);
        const int sca = f & 63, scb = (f >> 6) & 63, ma = (f >> 12) & 63, mb = (f >> 18) & 63;
        const uint32_t pw[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            lo[k] = pw[k] & 0x0F0F0F0Fu;
            hi[k] = (pw[k] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            {
                // token slots past nt repeat the last token (straight-line code keeps
                // the load waits exact); their sums are never read
                const int tc = min(t, nt - 1);
                uint32_t xw[16];
                load_x(x, tc, xw);
                int da = 0, db = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    da = sdot4(lo[k], xw[k], da);
                    db = sdot4(hi[k], xw[8 + k], db);
                }
                const int16_t* s = x.s + tc * x.s_stride + 4 * g;
                const int isum = mul24(sca, da) + mul24(scb, db);
                const int msum = mul24(ma, s[0] + s[1]) + mul24(mb, s[2] + s[3]);
                // the tile's integer totals over the four lane groups (lanes i, i + 16, i + 32,
                // i + 48); lane group 0 takes the float step, the others keep exact zeros
                int it = isum + __shfl_xor(isum, 16);
                it += __shfl_xor(it, 32);
                int mt = msum + __shfl_xor(msum, 16);
                mt += __shfl_xor(mt, 32);
                if (g == 0) acc[t] = q4k_term(acc[t], x.d[tc * x.d_stride], d, dmin, it, mt);
            }
        }
    }
};

// Q6_K: d[16] | scales[16][16] | codes (8 low-nibble + 4 high-bit dwords per lane).
template <>
struct Tile<13> {
    struct Regs {
        uint4 c0, c1, c2;
        uint32_t scw, d;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        r.c0 = *reinterpret_cast<const uint4*>(t + 288 + 16 * lane);
        r.c1 = *reinterpret_cast<const uint4*>(t + 1312 + 16 * lane);
        r.c2 = *reinterpret_cast<const uint4*>(t + 2336 + 16 * lane);
        r.scw = *reinterpret_cast<const uint32_t*>(t + 32 + 16 * (lane & 15) + 4 * (lane >> 4));
        r.d = *reinterpret_cast<const uint16_t*>(t + 2 * (lane & 15));
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int g, const XLds& x, int nt, float* acc) {
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        const float d = h2f(r.d);
        const uint32_t L[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
        const uint32_t Hb[4] = {r.c2.x, r.c2.y, r.c2.z, r.c2.w};
        constexpr uint32_t M4 = 0x0F0F0F0Fu, M30 = 0x30303030u;
        uint32_t w[16];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            w[4 * m] = (L[2 * m] & M4) | ((Hb[m] << 4) & M30);
            w[4 * m + 1] = ((L[2 * m] >> 4) & M4) | ((Hb[m] << 2) & M30);
            w[4 * m + 2] = (L[2 * m + 1] & M4) | (Hb[m] & M30);
            w[4 * m + 3] = ((L[2 * m + 1] >> 4) & M4) | ((Hb[m] >> 2) & M30);
        }
        int sc[4];  // scales of sub-blocks 4g .. 4g+3
#pragma unroll
        for (int m = 0; m < 4; ++m) sc[m] = sext8(r.scw >> (8 * m));
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            {
                // token slots past nt repeat the last token (straight-line code keeps
                // the load waits exact); their sums are never read
                const int tc = min(t, nt - 1);
                uint32_t xw[16];
                load_x(x, tc, xw);
                const int16_t* s = x.s + tc * x.s_stride + 4 * g;
                int isum = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    int dm = 0;
#pragma unroll
                    for (int q = 0; q < 4; ++q) dm = sdot4(w[4 * m + q], xw[4 * m + q], dm);
                    isum += mul24(sc[m], dm - 32 * s[m]);
                }
                // the tile's integer total over the four lane groups; lane group 0
                // takes the float step, the others keep exact zeros
                isum += __shfl_xor(isum, 16);
                isum += __shfl_xor(isum, 32);
                if (g == 0) acc[t] = __builtin_fmaf(x.d[tc * x.d_stride], d * static_cast<float>(isum), acc[t]);
            }
        }
    }
};

// Q8_0: d[16][8] | codes (the int8 values of GGML blocks 2g, 2g+1).
template <>
struct Tile<7> {
    struct Regs {
        uint4 c[4];
        uint32_t dd;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
#pragma unroll
        for (int u = 0; u < 4; ++u) r.c[u] = *reinterpret_cast<const uint4*>(t + 256 + 1024 * u + 16 * lane);
        r.dd = *reinterpret_cast<const uint32_t*>(t + 16 * (lane & 15) + 4 * (lane >> 4));
        return r;
    }
    // Q8_0 inputs always come in 32-value blocks (GGML's q8_0 x q8_0 rule)
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int g, const XLds& x, int nt, float* acc) {
        static_assert(A32, "Q8_0 matrices take 32-value activation blocks");
        const float da = h2f(r.dd), db = h2f(r.dd >> 16);
        const uint32_t w[16] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w,
                                r.c[2].x, r.c[2].y, r.c[2].z, r.c[2].w, r.c[3].x, r.c[3].y, r.c[3].z, r.c[3].w};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            {
                // token slots past nt repeat the last token (straight-line code keeps
                // the load waits exact); their sums are never read
                const int tc = min(t, nt - 1);
                uint32_t xw[16];
                load_x(x, tc, xw);
                int ia = 0, ib = 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    ia = sdot4(w[k], xw[k], ia);
                    ib = sdot4(w[8 + k], xw[8 + k], ib);
                }
                const float* xd = x.d + tc * x.d_stride + 2 * g;
                const float p = pair_sum(q8_term32(xd[0], da, ia), q8_term32(xd[1], db, ib));
                const float tot = lane_tile_total(p);
                if (g == 0) acc[t] = pair_sum(acc[t], tot);
            }
        }
    }
};

// Q2_K: (d, dmin)[16] | scales[16][16] | codes (4 dwords per lane).
template <>
struct Tile<9> {
    struct Regs {
        uint4 c;
        uint32_t scw, dd;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        r.c = *reinterpret_cast<const uint4*>(t + 320 + 16 * lane);
        r.scw = *reinterpret_cast<const uint32_t*>(t + 64 + 16 * (lane & 15) + 4 * (lane >> 4));
        r.dd = *reinterpret_cast<const uint32_t*>(t + 4 * (lane & 15));
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int g, const XLds& x, int nt, float* acc) {
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const uint32_t Q[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        int sc[4], mn[4];  // scale bytes of sub-blocks 4g .. 4g+3
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            sc[m] = (r.scw >> (8 * m)) & 0xF;
            mn[m] = (r.scw >> (8 * m + 4)) & 0xF;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            {
                // token slots past nt repeat the last token (straight-line code keeps
                // the load waits exact); their sums are never read
                const int tc = min(t, nt - 1);
                uint32_t xw[16];
                load_x(x, tc, xw);
                const int16_t* s = x.s + tc * x.s_stride + 4 * g;
                int isum = 0, msum = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    int dm = 0;
#pragma unroll
                    for (int q = 0; q < 4; ++q) dm = sdot4((Q[m] >> (2 * q)) & 0x03030303u, xw[4 * m + q], dm);
                    isum += mul24(sc[m], dm);
                    msum += mul24(mn[m], s[m]);
                }
                // the tile's integer totals over the four lane groups; lane group 0
                // takes the float step, the others keep exact zeros
                isum += __shfl_xor(isum, 16);
                isum += __shfl_xor(isum, 32);
                msum += __shfl_xor(msum, 16);
                msum += __shfl_xor(msum, 32);
                if (g == 0) acc[t] = q4k_term(acc[t], x.d[tc * x.d_stride], d, dmin, isum, msum);
            }
        }
    }
};

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Q4_K tiles x 4..8 int8 token rows on matrix cores, one token quad per
// v_mfma_i32_16x16x32_i8: the A operand's 16 rows are (token t', lane group
// G') pairs, 4 t' + G', and row 4 t' + G' carries token t''s activation codes
// only in lane group G''s K slots (zero elsewhere), so D[4 t' + G'][i] is the
// integer dot of weight row i's sub-block with token t' over lane group G''s
// values alone — the same integer the decode dot computes for that lane
// group. Four MFMAs (chunks of 8 values) per sub-block parity give the dots of
// sub-blocks 2 G' (low nibbles) and 2 G' + 1 (high nibbles). Lane (row i,
// lane group L) then holds token 4 q + L's dots for all four lane groups,
// sums them with their scales into the tile's integer totals and applies
// q4k_term once into acc[4 q] (acc[4 q + 1 .. 3] stay exact zeros, so the
// lane-group reduction ((g0 + g1) + (g2 + g3)) returns the decode dot's sum).
struct TileQ4Quad {
    struct Regs {
        uint4 w0, w1, hdr;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        r.hdr = *reinterpret_cast<const uint4*>(t + 16 * (lane & 15));
        r.w0 = *reinterpret_cast<const uint4*>(t + 256 + 16 * lane);
        r.w1 = *reinterpret_cast<const uint4*>(t + 1280 + 16 * lane);
        return r;
    }
    // acc[4 q + G']: running sum of (row lane % 16, token 4 q + lane / 16,
    // lane group G'); zero: 64 zero bytes of LDS (the masked A slots).
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int L, const XLds& x, int nt, float* acc,
                                               const int8_t* zero) {
        static_assert(NT % 4 == 0, "token quads");
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        constexpr int NQ = NT / 4;
        const int i = threadIdx.x & 15;
        const float d = h2f(r.hdr.x), dmin = h2f(r.hdr.x >> 16);
        // row i's 24-bit fields sc 2g | sc 2g+1 | m 2g | m 2g+1 of the four lane groups
        const uint32_t F[4] = {r.hdr.y & 0xFFFFFFu, (r.hdr.y >> 24) | ((r.hdr.z & 0xFFFFu) << 8),
                               (r.hdr.z >> 16) | ((r.hdr.w & 0xFFu) << 16), r.hdr.w >> 8};
        const uint32_t pw[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
        long bl[4], bh[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t l0 = pw[2 * c] & 0x0F0F0F0Fu, l1 = pw[2 * c + 1] & 0x0F0F0F0Fu;
            const uint32_t h0 = (pw[2 * c] >> 4) & 0x0F0F0F0Fu, h1 = (pw[2 * c + 1] >> 4) & 0x0F0F0F0Fu;
            bl[c] = static_cast<long>(static_cast<uint64_t>(l0) | (static_cast<uint64_t>(l1) << 32));
            bh[c] = static_cast<long>(static_cast<uint64_t>(h0) | (static_cast<uint64_t>(h1) << 32));
        }
        const bool own = (i & 3) == L;  // this lane's A slots carry codes
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            // token slots past nt repeat the last token; their sums are never read
            const int ta = min(4 * q + (i >> 2), nt - 1);
            const u32x4* src = reinterpret_cast<const u32x4*>(own ? x.q + ta * x.q_stride : zero);
            const u32x4 c0 = src[0], c1 = src[1], c2 = src[2], c3 = src[3];
            const u32x2 al[4] = {{c0.x, c0.y}, {c0.z, c0.w}, {c1.x, c1.y}, {c1.z, c1.w}};
            const u32x2 ah[4] = {{c2.x, c2.y}, {c2.z, c2.w}, {c3.x, c3.y}, {c3.z, c3.w}};
            i32x4 dl = {0, 0, 0, 0}, dh = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, al[c]), bl[c], dl, 0, 0, 0);
                dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, ah[c]), bh[c], dh, 0, 0, 0);
            }
            const int tk = min(4 * q + L, nt - 1);
            const u32x4* sp = reinterpret_cast<const u32x4*>(x.s + tk * x.s_stride);
            const u32x4 s03 = sp[0], s47 = sp[1];  // the block's 16 code sums (int16 pairs)
            const uint32_t sw[8] = {s03.x, s03.y, s03.z, s03.w, s47.x, s47.y, s47.z, s47.w};
            const float xd = x.d[tk * x.d_stride];
            // the tile's integer totals over the four lane groups, one float step into
            // acc[4 q]; acc[4 q + 1 .. 3] keep exact zeros (the decode dot's layout)
            int isum = 0, msum = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t f = F[g];
                const int sca = f & 63, scb = (f >> 6) & 63, ma = (f >> 12) & 63, mb = (f >> 18) & 63;
                const uint32_t s01 = sw[2 * g], s23 = sw[2 * g + 1];
                const int s0 = static_cast<int16_t>(s01 & 0xFFFFu), s1 = static_cast<int16_t>(s01 >> 16);
                const int s2 = static_cast<int16_t>(s23 & 0xFFFFu), s3 = static_cast<int16_t>(s23 >> 16);
                isum += mul24(sca, dl[g]) + mul24(scb, dh[g]);
                msum += mul24(ma, s0 + s1) + mul24(mb, s2 + s3);
            }
            acc[4 * q] = q4k_term(acc[4 * q], xd, d, dmin, isum, msum);
        }
    }
};

// Q6_K tiles x 4..8 int8 token rows on matrix cores, with the operand layout
// of TileQ4Quad: one MFMA per 8-value chunk, two chunks per 16-value
// sub-block, so D holds sub-block dots of lane group G' per (token, row). The
// B operand carries the signed codes q - 32 (bytewise (q + 0x60) ^ 0x80 for
// q in 0..63), so D is Tile<13>::dot's dm - 32 * s exactly (integer
// arithmetic) and the code sums are not read; the scale arithmetic per lane
// group is Tile<13>::dot's.
struct TileQ6Quad {
    struct Regs {
        uint4 c0, c1, c2, sc;
        uint32_t d;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        r.c0 = *reinterpret_cast<const uint4*>(t + 288 + 16 * lane);
        r.c1 = *reinterpret_cast<const uint4*>(t + 1312 + 16 * lane);
        r.c2 = *reinterpret_cast<const uint4*>(t + 2336 + 16 * lane);
        r.sc = *reinterpret_cast<const uint4*>(t + 32 + 16 * (lane & 15));
        r.d = *reinterpret_cast<const uint16_t*>(t + 2 * (lane & 15));
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int L, const XLds& x, int nt, float* acc,
                                               const int8_t* zero) {
        static_assert(NT % 4 == 0, "token quads");
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        constexpr int NQ = NT / 4;
        const int i = threadIdx.x & 15;
        const float d = h2f(r.d);
        const uint32_t Lw[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
        const uint32_t Hb[4] = {r.c2.x, r.c2.y, r.c2.z, r.c2.w};
        const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // row i's scales of lane groups 0..3
        constexpr uint32_t M4 = 0x0F0F0F0Fu, M30 = 0x30303030u;
        long b[8];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t w0 = (Lw[2 * m] & M4) | ((Hb[m] << 4) & M30);
            const uint32_t w1 = ((Lw[2 * m] >> 4) & M4) | ((Hb[m] << 2) & M30);
            const uint32_t w2 = (Lw[2 * m + 1] & M4) | (Hb[m] & M30);
            const uint32_t w3 = ((Lw[2 * m + 1] >> 4) & M4) | ((Hb[m] >> 2) & M30);
            // q - 32 per byte: q + 0x60 stays below 0x100, the xor moves the bias to -0x80
            constexpr uint32_t B60 = 0x60606060u, S80 = 0x80808080u;
            const uint32_t s0 = (w0 + B60) ^ S80, s1 = (w1 + B60) ^ S80;
            const uint32_t s2 = (w2 + B60) ^ S80, s3 = (w3 + B60) ^ S80;
            b[2 * m] = static_cast<long>(static_cast<uint64_t>(s0) | (static_cast<uint64_t>(s1) << 32));
            b[2 * m + 1] = static_cast<long>(static_cast<uint64_t>(s2) | (static_cast<uint64_t>(s3) << 32));
        }
        const bool own = (i & 3) == L;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int ta = min(4 * q + (i >> 2), nt - 1);
            const u32x4* src = reinterpret_cast<const u32x4*>(own ? x.q + ta * x.q_stride : zero);
            const u32x4 c0 = src[0], c1 = src[1], c2 = src[2], c3 = src[3];
            const u32x2 a[8] = {{c0.x, c0.y}, {c0.z, c0.w}, {c1.x, c1.y}, {c1.z, c1.w},
                                {c2.x, c2.y}, {c2.z, c2.w}, {c3.x, c3.y}, {c3.z, c3.w}};
            i32x4 D[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const i32x4 z = {0, 0, 0, 0};
                D[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[2 * m]), b[2 * m], z, 0, 0, 0);
                D[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[2 * m + 1]), b[2 * m + 1], D[m],
                                                            0, 0, 0);
            }
            const int tk = min(4 * q + L, nt - 1);
            const float xd = x.d[tk * x.d_stride];
            // the tile's integer total over the four lane groups, one float step into acc[4 q]
            int isum = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int m = 0; m < 4; ++m) isum += mul24(sext8(scw[g] >> (8 * m)), D[m][g]);
            }
            acc[4 * q] = __builtin_fmaf(xd, d * static_cast<float>(isum), acc[4 * q]);
        }
    }
};

// Q8_0 tiles x 4..8 int8 token rows on matrix cores, with the operand layout
// of TileQ4Quad: the lane group's 64 codes are eight 8-value chunks, chunks
// 0..3 (GGML block 2 G') accumulate into D0 and chunks 4..7 (block 2 G' + 1)
// into D1; the terms and the tile total are Tile<7>::dot's.
struct TileQ8Quad {
    struct Regs {
        uint4 c[4];
        uint4 sc;  // row i's eight block scales (f16)
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
#pragma unroll
        for (int u = 0; u < 4; ++u) r.c[u] = *reinterpret_cast<const uint4*>(t + 256 + 1024 * u + 16 * lane);
        r.sc = *reinterpret_cast<const uint4*>(t + 16 * (lane & 15));
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int L, const XLds& x, int nt, float* acc,
                                               const int8_t* zero) {
        static_assert(NT % 4 == 0, "token quads");
        static_assert(A32, "Q8_0 matrices take 32-value activation blocks");
        constexpr int NQ = NT / 4;
        const int i = threadIdx.x & 15;
        const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // (da, db) of lane groups 0..3
        long b[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            b[2 * u] = static_cast<long>(static_cast<uint64_t>(r.c[u].x) | (static_cast<uint64_t>(r.c[u].y) << 32));
            b[2 * u + 1] =
                static_cast<long>(static_cast<uint64_t>(r.c[u].z) | (static_cast<uint64_t>(r.c[u].w) << 32));
        }
        const bool own = (i & 3) == L;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int ta = min(4 * q + (i >> 2), nt - 1);
            const u32x4* src = reinterpret_cast<const u32x4*>(own ? x.q + ta * x.q_stride : zero);
            const u32x4 c0 = src[0], c1 = src[1], c2 = src[2], c3 = src[3];
            const u32x2 a[8] = {{c0.x, c0.y}, {c0.z, c0.w}, {c1.x, c1.y}, {c1.z, c1.w},
                                {c2.x, c2.y}, {c2.z, c2.w}, {c3.x, c3.y}, {c3.z, c3.w}};
            i32x4 D0 = {0, 0, 0, 0}, D1 = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                D0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[c]), b[c], D0, 0, 0, 0);
                D1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[4 + c]), b[4 + c], D1, 0, 0, 0);
            }
            const int tk = min(4 * q + L, nt - 1);
            const float* xd = x.d + tk * x.d_stride;
            const f32x4 xa = *reinterpret_cast<const f32x4*>(xd), xb = *reinterpret_cast<const f32x4*>(xd + 4);
            const float x8[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            float p[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float da = h2f(scw[g]), db = h2f(scw[g] >> 16);
                p[g] = pair_sum(q8_term32(x8[2 * g], da, D0[g]), q8_term32(x8[2 * g + 1], db, D1[g]));
            }
            acc[4 * q] = pair_sum(acc[4 * q], tile_total(p[0], p[1], p[2], p[3]));
        }
    }
};

// Q2_K tiles x 4..8 int8 token rows on matrix cores, with the operand layout
// of TileQ4Quad: chunk c (values 8 c .. 8 c + 7 of the lane group) is the
// 2-bit fields 4 (c % 2) and 4 (c % 2) + 2 of code word c / 2, two chunks per
// 16-value sub-block, so D[m] holds sub-block m's dot of lane group G' per
// (token, row); the scale and minimum arithmetic per lane group is
// Tile<9>::dot's.
struct TileQ2Quad {
    struct Regs {
        uint4 c, sc;
        uint32_t dd;
    };
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) {
        Regs r;
        r.c = *reinterpret_cast<const uint4*>(t + 320 + 16 * lane);
        r.sc = *reinterpret_cast<const uint4*>(t + 64 + 16 * (lane & 15));
        r.dd = *reinterpret_cast<const uint32_t*>(t + 4 * (lane & 15));
        return r;
    }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int L, const XLds& x, int nt, float* acc,
                                               const int8_t* zero) {
        static_assert(NT % 4 == 0, "token quads");
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        constexpr int NQ = NT / 4;
        const int i = threadIdx.x & 15;
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const uint32_t Q[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // row i's scale bytes of lane groups 0..3
        constexpr uint32_t M2 = 0x03030303u;
        long b[8];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t lo = (Q[m] >> (4 * h)) & M2, hi = (Q[m] >> (4 * h + 2)) & M2;
                b[2 * m + h] = static_cast<long>(static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32));
            }
        }
        const bool own = (i & 3) == L;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int ta = min(4 * q + (i >> 2), nt - 1);
            const u32x4* src = reinterpret_cast<const u32x4*>(own ? x.q + ta * x.q_stride : zero);
            const u32x4 c0 = src[0], c1 = src[1], c2 = src[2], c3 = src[3];
            const u32x2 a[8] = {{c0.x, c0.y}, {c0.z, c0.w}, {c1.x, c1.y}, {c1.z, c1.w},
                                {c2.x, c2.y}, {c2.z, c2.w}, {c3.x, c3.y}, {c3.z, c3.w}};
            i32x4 D[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const i32x4 z = {0, 0, 0, 0};
                D[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[2 * m]), b[2 * m], z, 0, 0, 0);
                D[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a[2 * m + 1]), b[2 * m + 1], D[m],
                                                            0, 0, 0);
            }
            const int tk = min(4 * q + L, nt - 1);
            const u32x4* sp = reinterpret_cast<const u32x4*>(x.s + tk * x.s_stride);
            const u32x4 s03 = sp[0], s47 = sp[1];
            const uint32_t sw[8] = {s03.x, s03.y, s03.z, s03.w, s47.x, s47.y, s47.z, s47.w};
            const float xd = x.d[tk * x.d_stride];
            // the tile's integer totals over the four lane groups, one float step into acc[4 q]
            int isum = 0, msum = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int j = 4 * g + m;  // sub-block of the block
                    const int sj = static_cast<int16_t>((sw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
                    const uint32_t byte = scw[g] >> (8 * m);
                    isum += mul24(static_cast<int>(byte & 0xF), D[m][g]);
                    msum += mul24(static_cast<int>((byte >> 4) & 0xF), sj);
                }
            }
            acc[4 * q] = q4k_term(acc[4 * q], xd, d, dmin, isum, msum);
        }
    }
};

// Q2_K tiles x 4..16 int8 token rows on matrix cores with the sub-block
// scales folded into the weight operand: a Q2_K scale (4 bits) times a code
// (2 bits) is at most 45, an int8, so one v_mfma_i32_16x16x64_i8 per 64
// values contracts sc * code against the tokens' codes and four of them give
// every (token, row) the tile's integer total sum_j sc_j dot_j over all
// sixteen sub-blocks, with no per-sub-block arithmetic. Lane (i, G) brings
// token i's codes of lane group G's chunk c (activation words 4 c .. 4 c + 3
// of its slice) and row i's codes of sub-block 4 G + c at the same positions
// (the 2-bit fields at shift 2 q of Q[c] pair with word 4 c + q, as in the
// decode dot), times that sub-block's scale. The min sums sum_j m_j S_j are
// exact integers below 2^24 from four v_mfma_f32_16x16x4f32 (K = lane group
// G: sub-block 4 c + G). D gives lane (i, G) tokens 4 G + r, r < 4, of row
// i: the lane keeps them in acc[0..3] (token-major, one lane group per
// token) and takes the decode dot's one float step per tile on the same
// integers, so rows equal the decode rows bit for bit.
struct TileQ2Fold {
    using Regs = TileQ2Quad::Regs;
    static __device__ __forceinline__ Regs load(const uint8_t* t, int lane) { return TileQ2Quad::load(t, lane); }
    template <int NT, bool A32>
    static __device__ __forceinline__ void dot(const Regs& r, int G, const XLds& x, int nt, float* acc) {
        static_assert(NT % 4 == 0 && NT <= 16, "token groups of up to 16 rows");
        static_assert(!A32, "K-quant matrices take 256-value activation blocks");
        const int i = threadIdx.x & 15;
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const uint32_t Q[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // row i's scale bytes, sub-blocks 4 g + m
        const uint32_t own = G == 0 ? scw[0] : G == 1 ? scw[1] : G == 2 ? scw[2] : scw[3];
        constexpr uint32_t M2 = 0x03030303u;
        const int ta = min(i, nt - 1);  // token rows past the step repeat its last row (never stored)
        const u32x4* src = reinterpret_cast<const u32x4*>(x.q + ta * x.q_stride);
        i32x4 D = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4 av = src[c];
            const uint16_t sc = static_cast<uint16_t>((own >> (8 * c)) & 0xFu);
            const u16x2 sv = {sc, sc};
            u32x4 bv;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                bv[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, (Q[c] >> (2 * q)) & M2) * sv);
            D = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, av), __builtin_bit_cast(i32x4, bv), D,
                                                      0, 0, 0);
        }
        f32x4 ms = {0.0F, 0.0F, 0.0F, 0.0F};
        const int16_t* srow = x.s + ta * x.s_stride;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float sa = static_cast<float>(srow[4 * c + G]);
            const float mb = static_cast<float>((scw[c] >> (8 * G + 4)) & 0xFu);
            ms = __builtin_amdgcn_mfma_f32_16x16x4f32(sa, mb, ms, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int t = min(4 * G + q, nt - 1);
            acc[q] = q4k_term_f(acc[q], x.d[t * x.d_stride], d, dmin, D[q], ms[q]);
        }
    }
};

// The token-quad tile of a weight format (void: none).
template <uint32_t TYPE>
struct QuadTile {
    using type = void;
};
template <>
struct QuadTile<7> {
    using type = TileQ8Quad;
};
template <>
struct QuadTile<9> {
    using type = TileQ2Quad;
};
template <>
struct QuadTile<11> {
    using type = TileQ4Quad;
};
template <>
struct QuadTile<13> {
    using type = TileQ6Quad;
};
template <uint32_t TYPE>
constexpr bool kHasQuads = !std::is_void_v<typename QuadTile<TYPE>::type>;

__device__ __forceinline__ unsigned long long pack_best(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - idx);
}

// ------------------------------------------------------------------ matmul epilogues
// Step fields the QKV epilogue needs for one token row: its position and its
// sequence's cache.
struct QkvRow {
    int32_t pos;
    int32_t capacity;
    uint16_t* k;
    uint16_t* v;
};

__device__ __forceinline__ QkvRow qkv_row(const QkvOut& o, int t) {
    const StepDev* st = o.step;
    const SeqDev& sd = st->seqs[st->seq[o.row0 + t]];
    return QkvRow{st->pos[o.row0 + t], sd.capacity, sd.k, sd.v};
}

#pragma clang fp contract(off)
__device__ __forceinline__ void qkv_store(const GemvArgs& a, int t, int gr, float va, float vb, bool pair,
                                          const QkvRow& sd) {
    // gr: first fused row of a rotated pair (q or k) or a v row (pair == false)
    const QkvOut& o = a.qkv;
    const int hd = o.head_dim, half = hd / 2, Hq = o.n_head * hd, kv = o.n_head_kv * hd;
    const int pos = sd.pos;
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
            global_ptr<uint16_t> kc = as_global(sd.k);
            kc[row + i] = f2h(r0);
            kc[row + i + half] = f2h(r1);
        }
    } else {
        const int g = gr - Hq - kv;
        const int head = g / hd, dcol = g % hd;
        // V is stored in 16-position tiles, transposed within a tile:
        // [layer][kv head][position / 16][dim][position % 16]
        const size_t at = ((static_cast<size_t>(o.layer) * o.n_head_kv + head) * sd.capacity + (pos & ~15)) * hd +
                          static_cast<size_t>(dcol) * 16 + (pos & 15);
        as_global(sd.v)[at] = f2h(va);
    }
}
#pragma clang fp contract(on)

// Row results of a work-group -> bias / residual / SwiGLU / RoPE + cache /
// greedy argmax. `sum(j, t)` returns the dot of local row j for token t;
// lv holds nrows * n_tok floats of scratch.
// Which modes an instantiation handles: every mode, every mode but kLogits,
// or kLogits alone (kernels that never see a mode do not carry its code or
// its registers).
enum EpilogueModes : int { kAllModes = 0, kNoLogits = 1, kLogitsOnly = 2 };

template <int NTHR, int MODES = kAllModes, typename Sum>
__device__ void gemv_epilogue(const GemvArgs& a, int row0, int nrows, Sum sum, float* lv,
                              unsigned long long* best_lds = nullptr) {
    constexpr int W = NTHR / kWave;
    const int n = nrows * a.n_tok;
    const int mode = MODES == kLogitsOnly ? kLogits : (MODES == kNoLogits && a.mode == kLogits ? -1 : a.mode);
    switch (mode) {
    case kStore:
    case kAdd:
        if constexpr (MODES == kLogitsOnly) break;
        for (int idx = threadIdx.x; idx < n; idx += NTHR) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            float* out = a.y + static_cast<size_t>(t) * a.y_stride + gr;
            if (a.mode == kAdd) *out += sum(j, t);
            else *out = sum(j, t) + (a.mat.bias ? a.mat.bias[gr] : 0.0F);
        }
        break;
    case kSwiGLU: {
        if constexpr (MODES == kLogitsOnly) break;
        const int half = nrows / 2;
        for (int idx = threadIdx.x; idx < half * a.n_tok; idx += NTHR) {
            const int t = idx / half, jj = idx - t * half;
            const int j = (jj / kGluGroup) * 2 * kGluGroup + jj % kGluGroup;
            const float g = sum(j, t), u = sum(j + kGluGroup, t);
            const int o = (row0 / 2) + jj;
            a.y[static_cast<size_t>(t) * a.y_stride + o] = g / (1.0F + expf(-g)) * u;
        }
        break;
    }
    case kQKV: {
        if constexpr (MODES == kLogitsOnly) break;
        const int Hq = a.qkv.n_head * a.qkv.head_dim, kv = a.qkv.n_head_kv * a.qkv.head_dim;
        for (int idx = threadIdx.x; idx < n; idx += NTHR) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            const float* bias = a.mat.bias;
            const QkvRow rw = qkv_row(a.qkv, t);
            if (gr < Hq + kv) {
                if (gr & 1) continue;
                qkv_store(a, t, gr, sum(j, t) + (bias ? bias[gr] : 0.0F), sum(j + 1, t) + (bias ? bias[gr + 1] : 0.0F),
                          true, rw);
            } else {
                qkv_store(a, t, gr, sum(j, t) + (bias ? bias[gr] : 0.0F), 0.0F, false, rw);
            }
        }
        break;
    }
    case kLogits: {
        if constexpr (MODES == kNoLogits) break;
        for (int idx = threadIdx.x; idx < n; idx += NTHR) {
            const int t = idx / nrows, j = idx - t * nrows, gr = row0 + j;
            const float v = sum(j, t) + (a.mat.bias ? a.mat.bias[gr] : 0.0F);
            if (a.store_logits) a.y[static_cast<size_t>(t) * a.y_stride + gr] = v;
            lv[idx] = v;
        }
        __syncthreads();
        // one wave per token: lanes scan rows, then a wave argmax (first maximum)
        const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
        for (int t = wave; t < a.n_tok; t += W) {
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
            // best_lds: a work-group's running best per token, merged into a.best once at its end
            if (lane == 0 && p != 0ull) {
                if (best_lds != nullptr) {
                    best_lds[t] = p > best_lds[t] ? p : best_lds[t];
                } else {
                    // the slot only grows: a best at or below its current value needs no atomic
                    if (p > __hip_atomic_load(a.best + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                        atomicMax(a.best + t, p);
                }
            }
        }
        break;
    }
    default:
        break;
    }
}

// ------------------------------------------------------------------ quantized matmul
// Work-group = kMmWaves waves owning `rgw` consecutive 16-row groups. For
// every staged K chunk, wave w takes the chunk's tiles b = w, w + W, ... of
// each of the group's row groups, as one flat item stream with the next
// kMmDepth tiles' loads in flight (the first ones issued before the
// activation prologue). A lane accumulates its share of a row group's 16
// rows; when the stream leaves a row group, the four lane groups are summed
// and the wave's partial row sums added to its own LDS slot. Row results are
// the sum of the waves' slots in wave order, so they do not depend on
// scheduling.
constexpr int kMmWaves = 8;
constexpr int kMmThreads = kMmWaves * kWave;
constexpr int kMmDepth = 2;

struct MmGeom {
    int32_t rgw;    // row groups per work-group
    int32_t chunk;  // K values staged per pass (multiple of 256)
};

// Kinds of matmul input: pre-quantized rows (a.xq), float rows RMS-normalized
// with a gain in the prologue (a.x with a.x.gain), plain float rows (a.x).
// A32: the activations are (or are staged) in 32-value blocks.
enum MmInput : int { kInAct8 = 0, kInNormed = 1, kInFloat = 2 };

template <uint32_t TYPE, int NT, int IN, bool A32>
__global__ __launch_bounds__(kMmThreads) void k_mm(GemvArgs a, MmGeom geo) {
    constexpr bool A8 = IN == kInAct8;
    constexpr bool GAIN = IN == kInNormed;
    constexpr int DB = A32 ? 8 : 1;  // activation scales per 256 values
    constexpr int NB = GAIN ? kStageBatch : kStageBatchFloat;  // blocks per wave of a float staging batch
    // int8 code pieces per thread of a staging batch (a later batch waits
    // behind the weight tiles in flight): five take two rows of the down
    // projection (2 x 18944 values) in one batch, six take five in two
    constexpr int A8P = NT == 4 ? 5 : NT == 8 ? 6 : 4;
    // int8 or normalized rows of a format with a token-quad tile, in token quads, run on matrix cores;
    // Q2_K token groups on the folded-scale tile (token-major: lane group G holds tokens 4 G .. 4 G + 3)
    constexpr bool FOLD = TYPE == 9 && (A8 || GAIN) && NT % 4 == 0;
    constexpr bool QUAD = kHasQuads<TYPE> && (A8 || GAIN) && NT % 4 == 0 && !FOLD;
    using T = std::conditional_t<FOLD, TileQ2Fold,
                                 std::conditional_t<QUAD, typename QuadTile<TYPE>::type, Tile<TYPE>>>;
    using Regs = typename T::Regs;
    constexpr int W = kMmWaves;
    constexpr uint32_t TB = tile_bytes(TYPE);
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int K = static_cast<int>(a.mat.cols), nb = K / 256;
    const int chunk = geo.chunk, nbc = chunk / 256, rgw = geo.rgw;
    const int n_tok = a.n_tok;
    // staging for the step's n_tok rows (token slots past them are never read)
    int8_t* sq = reinterpret_cast<int8_t*>(lds_raw);
    float* sd = reinterpret_cast<float*>(lds_raw + n_tok * chunk);
    int16_t* ss = reinterpret_cast<int16_t*>(sd + ((n_tok * nbc * DB + 3) & ~3));  // 16-byte aligned
    // Row partials. One pass over K: each wave stores its finished row-group
    // sums with the four lane groups already combined, [rgw][W][16 rows][NT].
    // Several passes: every lane keeps running sums, [rgw][W][64 lanes][PS]
    // (the folded Q2_K tile keeps four per lane: lane group G's tokens 4 G + q).
    constexpr int PS = FOLD ? 4 : NT;
    const bool single = NT <= 2 || nbc >= nb;  // one- and two-token groups always run one pass (mm_geom)
    float* part = reinterpret_cast<float*>(ss + n_tok * (chunk / 16));
    float* ssq = part + (single ? rgw * W * 16 * NT : rgw * W * 64 * PS);  // [n_tok][nbc] sums of squares (normed)
    float* lv = ssq + n_tok * nbc;  // [rgw * 16 * NT]
    // 64 zero bytes (16-byte aligned) for the masked operand slots of TileQ4Quad
    int8_t* zero = reinterpret_cast<int8_t*>(lds_raw) +
                   ((reinterpret_cast<uint8_t*>(lv + rgw * 16 * NT) - lds_raw + 15) & ~static_cast<ptrdiff_t>(15));

    const int n_rg = (static_cast<int>(a.mat.rows) + 15) / 16;
    const int rg0 = blockIdx.x * rgw;
    const int rgn = min(rgw, n_rg - rg0);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int grp = lane >> 4;
    const uint8_t* base = a.mat.data + static_cast<size_t>(rg0) * nb * TB;
    const int row0 = rg0 * 16;
    const int nrows = min(rgn * 16, static_cast<int>(a.mat.rows) - row0);

    // items of the wave in a chunk of nbcur tiles: per row group the tiles w, w+W, ...
    auto per_rg = [&](int nbcur) { return nbcur > wave ? (nbcur - wave + W - 1) / W : 0; };

    // The wave's stream of (row group r, tile m) items keeps kMmDepth tile
    // loads in flight: slot u is consumed, then refilled with the item
    // kMmDepth ahead. The load cursor stops at the stream's last item, so
    // every load is issued unconditionally and the compiler counts
    // outstanding loads exactly.
    Regs ring[kMmDepth];
    int nbcur = min(nbc, nb);
    int pr = per_rg(nbcur);
    int total = pr * rgn;
    // load cursor: byte offset of the next item, its tile index in the row
    // group and the number of items still to be loaded after it
    uint32_t loff = 0;
    int lm = 0, lleft = 0;
    auto load_next = [&](Regs& slot) {
        slot = T::load(base + loff, lane);
        if (lleft > 0) {
            --lleft;
            if (lm + 1 < pr) {
                ++lm;
                loff += W * TB;
            } else {
                lm = 0;
                loff += (nb - (pr - 1) * W) * TB;
            }
        }
    };
    // A wave without tiles in the pass (total == 0) loads its ring from the
    // pass's last tile and never uses it: loads stay unconditional.
    auto prefetch = [&](int c0b) {
        loff = static_cast<uint32_t>(c0b + min(wave, nbcur - 1)) * TB;
        lm = 0;
        lleft = total - 1;
#pragma unroll
        for (int u = 0; u < kMmDepth; ++u) load_next(ring[u]);
    };
    // the first staging batch is requested before the weights (loads complete
    // in issue order, so the activations do not wait behind weight tiles)
    f32x4 f0[2 * NB];
    StageA8Regs<A8P> q0;
    if constexpr (A8) stage_act8_load<kMmThreads, A8P, A32>(a.xq, n_tok, 0, nbcur, 0, q0);
    else stage_f32_load<kMmThreads, NB, GAIN>(a.x, n_tok, 0, nbcur, wave, f0);
    prefetch(0);
    // the residual the epilogue adds to is fetched with the first weights
    // (issued unconditionally from a clamped index, so that the compiler's
    // count of outstanding loads stays exact)
    float y_pre;
    {
        const int idx = min(static_cast<int>(threadIdx.x), nrows * n_tok - 1);
        const int t = idx / nrows, j = idx - t * nrows;
        const float* src = a.mode == kAdd ? a.y + static_cast<size_t>(t) * a.y_stride + row0 + j
                                          : reinterpret_cast<const float*>(a.mat.data);
        y_pre = *src;
    }
    // zero partials (waves without tiles, when the row has fewer blocks than waves, add nothing)
    for (int i = threadIdx.x; i < (single ? rgw * W * 16 * NT : rgw * W * 64 * PS); i += kMmThreads) part[i] = 0.0F;
    if constexpr (QUAD) {
        if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(zero)[threadIdx.x] = 0u;
    }
    if constexpr (A8) {
        stage_act8<kMmThreads, A8P, A32>(a.xq, n_tok, 0, nbcur, sq, sd, ss, chunk, q0);
    } else {
        stage_f32<kMmThreads, NB, GAIN, A32>(a.x, n_tok, 0, nbcur, sq, sd, ss, ssq, chunk, f0);
        if constexpr (GAIN) finish_norm<kMmThreads, A32>(n_tok, nbcur, K, a.x.eps, ssq, sd, chunk);
    }

    for (int c0b = 0;;) {
        __syncthreads();
        if (total > 0) {
            float acc[NT];
            int cm = 0;                                             // tile of the row group being computed
            float* slot = part + (wave * 64 + lane) * PS;          // the lane's running sums of that row group
            float* done = part + (wave * 16 + (lane & 15)) * NT;   // its finished sums (one pass)
            const int8_t* xq0 = sq + wave * 256 + 64 * grp;         // its activation slice
            // one item of the wave's stream (its tile cm of the current row group) from slot u of the ring
            auto consume = [&](const Regs& tile_regs) {
                if (cm == 0) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t] = single || t >= PS ? 0.0F : slot[t];
                }
                const int bl = wave + W * cm;
                XLds x;
                x.q = xq0 + W * 256 * cm;
                x.d = sd + bl * DB;
                x.s = ss + bl * 16;
                x.q_stride = chunk;
                x.d_stride = nbc * DB;
                x.s_stride = chunk / 16;
                if constexpr (QUAD) T::template dot<NT, A32>(tile_regs, grp, x, n_tok, acc, zero);
                else T::template dot<NT, A32>(tile_regs, grp, x, n_tok, acc);
                if (++cm == pr) {
                    cm = 0;
                    if (single) {
                        // (g0 + g1) + (g2 + g3) of the row's four lane-group sums
                        if constexpr (FOLD) {
                            // one lane group per token: its value is the sum
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                if (4 * grp + q < NT) done[4 * grp + q] = acc[q];
                            }
                        } else if constexpr (QUAD) {
#pragma unroll
                            for (int q = 0; q < NT / 4; ++q) {
                                done[4 * q + grp] =
                                    (acc[4 * q] + acc[4 * q + 1]) + (acc[4 * q + 2] + acc[4 * q + 3]);
                            }
                        } else {
#pragma unroll
                            for (int t = 0; t < NT; ++t) {
                                float v = acc[t];
                                v += __shfl_xor(v, 16);
                                v += __shfl_xor(v, 32);
                                if (grp == 0) done[t] = v;
                            }
                        }
                        done += W * 16 * NT;
                    } else {
#pragma unroll
                        for (int t = 0; t < PS; ++t) slot[t] = acc[t];
                        slot += W * 64 * PS;
                    }
                }
            };
            // Items whose ring slot is refilled with a later item; the last
            // kMmDepth items are consumed without further loads.
            int n0 = 0;
            for (; n0 + kMmDepth < total; n0 += kMmDepth) {
#pragma unroll
                for (int u = 0; u < kMmDepth; ++u) {
                    consume(ring[u]);
                    load_next(ring[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < kMmDepth; ++u) {
                if (n0 + u < total) consume(ring[u]);
            }
        }
        c0b += nbc;
        if (c0b >= nb) break;
        // next pass (rows that are not normalized): activations first, then weights
        nbcur = min(nbc, nb - c0b);
        pr = per_rg(nbcur);
        total = pr * rgn;
        if constexpr (A8) {
            StageA8Regs<A8P> qn;
            stage_act8_load<kMmThreads, A8P, A32>(a.xq, n_tok, c0b * 256, nbcur, 0, qn);
            prefetch(c0b);
            __syncthreads();  // every wave is done with the previous pass's activations
            stage_act8<kMmThreads, A8P, A32>(a.xq, n_tok, c0b * 256, nbcur, sq, sd, ss, chunk, qn);
        } else {
            f32x4 fn[2 * NB];
            stage_f32_load<kMmThreads, NB, GAIN>(a.x, n_tok, c0b * 256, nbcur, wave, fn);
            prefetch(c0b);
            __syncthreads();
            stage_f32<kMmThreads, NB, GAIN, A32>(a.x, n_tok, c0b * 256, nbcur, sq, sd, ss, ssq, chunk, fn);
        }
    }
    __syncthreads();
    // row sum: over waves in order of ((g0 + g1) + (g2 + g3)) per wave, on every layout
    auto sum = [&](int j, int t) {
        const int r = j >> 4, i = j & 15;
        float v = 0.0F;
        if (single) {
#pragma unroll
            for (int w = 0; w < W; ++w) v += part[((r * W + w) * 16 + i) * NT + t];
            return v;
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
            float p[4];
            if constexpr (FOLD) {
                // token t's running sum sits in lane group t / 4, slot t % 4 alone
                v += part[((r * W + w) * 64 + i + 16 * (t >> 2)) * PS + (t & 3)];
                continue;
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                p[g] = QUAD ? part[((r * W + w) * 64 + i + 16 * (t & 3)) * NT + 4 * (t >> 2) + g]
                            : part[((r * W + w) * 64 + i + 16 * g) * NT + t];
            }
            v += (p[0] + p[1]) + (p[2] + p[3]);
        }
        return v;
    };
    if (a.mode == kAdd) {
        // residual add with the prefetched values
        const int n = nrows * n_tok;
        for (int idx = threadIdx.x; idx < n; idx += kMmThreads) {
            const int t = idx / nrows, j = idx - t * nrows;
            float* out = a.y + static_cast<size_t>(t) * a.y_stride + row0 + j;
            *out = (idx == static_cast<int>(threadIdx.x) ? y_pre : *out) + sum(j, t);
        }
        return;
    }
    gemv_epilogue<kMmThreads>(a, row0, nrows, sum, lv);
}

// ------------------------------------------------------------------ wide matmul on matrix cores
// Quantized tiles x int8 rows for steps of 9 .. kWideRows tokens (prefill
// chunks, long drafts, large batches). Work-group = one 16-row group and one
// 16-token tile; wave w takes the K tiles w, w + W, ... as the decode matmul
// does. Each v_mfma_i32_16x16x32_i8 contracts one 32-value stretch of a tile:
// lane (i, G) brings token i's activation codes 32 s + 8 G .. + 7 (the A
// operand) and row i's codes at the same positions (the B operand), so the
// product is one GGML block (Q8_0), one sub-block (Q4_K), or, with the lane
// groups of the other half zeroed, one 16-value sub-block (Q6_K, Q2_K). D
// gives lane (i, G) the integer dots of row i with tokens 4 G + j for every
// block, and the lane applies the decode matmul's scale arithmetic in the
// same order (Q4_K and Q2_K: q4k_term per (tile, token) on the tile's
// integer totals, Q6_K one step on its integer scale sum; Q8_0 q8_term per
// (tile, lane group, token)). The min sums Σ m · (code sum) are exact integers below 2^24 and
// come from v_mfma_f32_16x16x4f32 as exact floats. Sums run over waves, then
// lane groups, in the decode order: every row equals that row computed alone,
// bit for bit.
__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return static_cast<long>(static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32));
}

__device__ __forceinline__ i32x4 mfma_i8(long a, long b) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, i32x4{0, 0, 0, 0}, 0, 0, 0);
}


// Per-format operands of one tile for lane (row i, lane group G) and the
// scale arithmetic of its 16 (lane group g, token 4 G + j) terms.
template <uint32_t TYPE>
struct WideTile;

// Q4_K: c[g] = code chunk G of lane group g (values 64 g + 8 G .. + 7 of
// sub-block 2 g in the low nibbles, 64 g + 32 + 8 G .. of 2 g + 1 in the high
// ones). The min sum ma · S(2 g) + mb · S(2 g + 1) is a K = 2 product over
// lane groups 0 and 1 (S: a 32-value code sum of the token).
template <>
struct WideTile<11> {
    static constexpr bool kSums = true;
    struct Wt {
        uint4 hdr;
        uint2 c[4];
    };
    struct Xt {
        float s[4];
    };
    static __device__ __forceinline__ Wt load_w(const uint8_t* t, int i, int G) {
        Wt w;
        w.hdr = *reinterpret_cast<const uint4*>(t + 16 * i);
#pragma unroll
        for (int g = 0; g < 4; ++g)
            w.c[g] = *reinterpret_cast<const uint2*>(t + 256 + 1024 * (G >> 1) + 16 * (16 * g + i) + 8 * (G & 1));
        return w;
    }
    // xs: the token's 16-value code sums of this block (16 int16, in LDS)
    static __device__ __forceinline__ Xt load_x(const uint32_t* xs, int G) {
        Xt x;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t v = xs[2 * g + (G & 1)];  // sums 4 g + 2 G, + 1: sub-block 2 g + G
            const int S = static_cast<int16_t>(v & 0xFFFFu) + (static_cast<int32_t>(v) >> 16);
            x.s[g] = G < 2 ? static_cast<float>(S) : 0.0F;
        }
        return x;
    }
    static __device__ __forceinline__ void accumulate(const Wt& w, const long (&av)[8], const Xt& x,
                                                      const float (&xd)[4], int G, float (&acc)[4][4]) {
        const float d = h2f(w.hdr.x), dmin = h2f(w.hdr.x >> 16);
        // row i's 24-bit fields sc 2g | sc 2g+1 | m 2g | m 2g+1 of the four lane groups
        const uint32_t F[4] = {w.hdr.y & 0xFFFFFFu, (w.hdr.y >> 24) | ((w.hdr.z & 0xFFFFu) << 8),
                               (w.hdr.z >> 16) | ((w.hdr.w & 0xFFu) << 16), w.hdr.w >> 8};
        // the tile's totals over the four lane groups: integer dots, and the min
        // sums accumulated on the f32 MFMA (exact integers below 2^24); one float
        // step per token into acc[0], acc[1 .. 3] keep exact zeros (the decode dot's order)
        int isum[4] = {0, 0, 0, 0};
        f32x4 ms = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t f = F[g];
            const int sca = f & 63, scb = (f >> 6) & 63;
            const uint2 c = w.c[g];
            const long lo = pack2(c.x & 0x0F0F0F0Fu, c.y & 0x0F0F0F0Fu);
            const long hi = pack2((c.x >> 4) & 0x0F0F0F0Fu, (c.y >> 4) & 0x0F0F0F0Fu);
            const i32x4 da = mfma_i8(av[2 * g], lo), db = mfma_i8(av[2 * g + 1], hi);
            const float mB = G < 2 ? static_cast<float>((f >> (12 + 6 * G)) & 63u) : 0.0F;
            ms = __builtin_amdgcn_mfma_f32_16x16x4f32(x.s[g], mB, ms, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) isum[j] += mul24(sca, da[j]) + mul24(scb, db[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][j] = q4k_term_f(acc[0][j], xd[j], d, dmin, isum[j], ms[j]);
    }
};

// Q8_0: c[2 g + e] = values 8 G .. + 7 of GGML block 2 g + e (signed codes).
template <>
struct WideTile<7> {
    static constexpr bool kSums = false;
    struct Wt {
        uint4 dd;
        uint2 c[8];
    };
    struct Xt {};
    static __device__ __forceinline__ Wt load_w(const uint8_t* t, int i, int G) {
        Wt w;
        w.dd = *reinterpret_cast<const uint4*>(t + 16 * i);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int e = 0; e < 2; ++e)
                w.c[2 * g + e] = *reinterpret_cast<const uint2*>(t + 256 + 1024 * (2 * e + (G >> 1)) + 16 * (16 * g + i) +
                                                                 8 * (G & 1));
        }
        return w;
    }
    static __device__ __forceinline__ Xt load_x(const uint32_t*, int) { return {}; }
    // xd holds the token tile's 32-value block scales ([token][8]); the lane's
    // tokens are 4 G + j. The terms and the tile total are the decode dot's
    // (q8_term32, tile_total).
    static __device__ __forceinline__ void accumulate32(const Wt& w, const long (&av)[8], const uint32_t*,
                                                        const float* xd, int G, float (&acc)[4][4]) {
        const uint32_t D[4] = {w.dd.x, w.dd.y, w.dd.z, w.dd.w};
        i32x4 I[4][2];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            I[g][0] = mfma_i8(av[2 * g], pack2(w.c[2 * g].x, w.c[2 * g].y));
            I[g][1] = mfma_i8(av[2 * g + 1], pack2(w.c[2 * g + 1].x, w.c[2 * g + 1].y));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = 4 * G + j;
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(xd + 8 * tok), x1 = *reinterpret_cast<const f32x4*>(xd + 8 * tok + 4);
            const float x8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            float p[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float da = h2f(D[g]), db = h2f(D[g] >> 16);
                p[g] = pair_sum(q8_term32(x8[2 * g], da, I[g][0][j]), q8_term32(x8[2 * g + 1], db, I[g][1][j]));
            }
            acc[0][j] = pair_sum(acc[0][j], tile_total(p[0], p[1], p[2], p[3]));
        }
    }
};

// Q6_K: per 32-value stretch h = 2 g + e (sub-blocks 4 g + 2 e, + 1), L[h] /
// H[h] = the low-nibble and high-bit words that hold values 32 e + 8 G .. + 7
// of lane group g. The codes enter as q - 32, so the dot is the decode's
// dm - 32 · (code sum) without the sums.
template <>
struct WideTile<13> {
    static constexpr bool kSums = false;
    struct Wt {
        uint4 sc;
        uint32_t d;
        uint32_t L[8], H[8];
    };
    struct Xt {};
    static __device__ __forceinline__ Wt load_w(const uint8_t* t, int i, int G) {
        Wt w;
        w.d = *reinterpret_cast<const uint16_t*>(t + 2 * i);
        w.sc = *reinterpret_cast<const uint4*>(t + 32 + 16 * i);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int lane_off = 16 * (16 * g + i);
                w.L[2 * g + e] = *reinterpret_cast<const uint32_t*>(t + 288 + 1024 * e + lane_off + 4 * G);
                w.H[2 * g + e] = *reinterpret_cast<const uint32_t*>(t + 2336 + lane_off + 4 * (2 * e + (G >> 1)));
            }
        }
        return w;
    }
    static __device__ __forceinline__ Xt load_x(const uint32_t*, int) { return {}; }
    static __device__ __forceinline__ void accumulate(const Wt& w, const long (&av)[8], const Xt&,
                                                      const float (&xd)[4], int G, float (&acc)[4][4]) {
        constexpr uint32_t M4 = 0x0F0F0F0Fu, M30 = 0x30303030u;
        const float d = h2f(w.d);
        const uint32_t SC[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
        const int hshift = (G & 1) ? 0 : 4;
        const bool low = G < 2;  // lane groups 0, 1: the stretch's first sub-block
        int isum[4] = {0, 0, 0, 0};  // the tile's integer totals over the lane groups, per token
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            i32x4 dm[4];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t Lw = w.L[2 * g + e], H1 = w.H[2 * g + e] << hshift;
                uint32_t w0 = (Lw & M4) | (H1 & M30), w1 = ((Lw >> 4) & M4) | ((H1 >> 2) & M30);
                // q - 32 per byte (q < 64: no carry between bytes)
                w0 = (w0 + 0x60606060u) ^ 0x80808080u;
                w1 = (w1 + 0x60606060u) ^ 0x80808080u;
                const long B = pack2(w0, w1);
                dm[2 * e] = mfma_i8(av[2 * g + e], low ? B : 0L);
                dm[2 * e + 1] = mfma_i8(av[2 * g + e], low ? 0L : B);
            }
            int sc[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) sc[m] = sext8(SC[g] >> (8 * m));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int m = 0; m < 4; ++m) isum[j] += mul24(sc[m], dm[m][j]);
            }
        }
        // one float step per token into acc[0]; acc[1 .. 3] keep exact zeros
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][j] = __builtin_fmaf(xd[j], d * static_cast<float>(isum[j]), acc[0][j]);
    }
};

// Q2_K: Q[2 g + e] = the code word of sub-block 4 g + 2 e + G / 2; the min
// sum Σ mn · (16-value code sum) is a K = 4 product over the lane groups.
template <>
struct WideTile<9> {
    static constexpr bool kSums = true;
    struct Wt {
        uint32_t dd;
        uint4 sc;
        uint32_t Q[8];
    };
    struct Xt {
        float s[4];
    };
    static __device__ __forceinline__ Wt load_w(const uint8_t* t, int i, int G) {
        Wt w;
        w.dd = *reinterpret_cast<const uint32_t*>(t + 4 * i);
        w.sc = *reinterpret_cast<const uint4*>(t + 64 + 16 * i);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int e = 0; e < 2; ++e)
                w.Q[2 * g + e] = *reinterpret_cast<const uint32_t*>(t + 320 + 16 * (16 * g + i) + 4 * (2 * e + (G >> 1)));
        }
        return w;
    }
    static __device__ __forceinline__ Xt load_x(const uint32_t* xs, int G) {
        Xt x;
        const int16_t* s = reinterpret_cast<const int16_t*>(xs);
#pragma unroll
        for (int g = 0; g < 4; ++g) x.s[g] = static_cast<float>(s[4 * g + G]);
        return x;
    }
    static __device__ __forceinline__ void accumulate(const Wt& w, const long (&av)[8], const Xt& x,
                                                      const float (&xd)[4], int G, float (&acc)[4][4]) {
        const float d = h2f(w.dd), dmin = h2f(w.dd >> 16);
        const uint32_t SC[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
        const int qshift = 4 * (G & 1);
        const bool low = G < 2;
        // the tile's totals over the lane groups: integer dots, and the min sums
        // accumulated on the f32 MFMA (exact integers below 2^24)
        int isum[4] = {0, 0, 0, 0};
        f32x4 ms = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            i32x4 dm[4];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t q = w.Q[2 * g + e] >> qshift;
                const long B = pack2(q & 0x03030303u, (q >> 2) & 0x03030303u);
                dm[2 * e] = mfma_i8(av[2 * g + e], low ? B : 0L);
                dm[2 * e + 1] = mfma_i8(av[2 * g + e], low ? 0L : B);
            }
            ms = __builtin_amdgcn_mfma_f32_16x16x4f32(x.s[g], static_cast<float>((SC[g] >> (8 * G + 4)) & 0xFu), ms, 0,
                                                      0, 0);
            int sc[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) sc[m] = (SC[g] >> (8 * m)) & 0xF;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int m = 0; m < 4; ++m) isum[j] += mul24(sc[m], dm[m][j]);
            }
        }
        // one float step per token into acc[0]; acc[1 .. 3] keep exact zeros
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][j] = q4k_term_f(acc[0][j], xd[j], d, dmin, isum[j], ms[j]);
    }
};

// The arguments of tokens t0 .. t0 + nt - 1 of a step, as token 0 .. nt - 1.
__device__ __forceinline__ GemvArgs token_slice(const GemvArgs& a, int t0, int nt) {
    GemvArgs b = a;
    b.n_tok = nt;
    if (b.y != nullptr) b.y += static_cast<size_t>(t0) * b.y_stride;
    if (b.best != nullptr) b.best += t0;
    b.qkv.row0 += t0;
    if (b.qkv.q != nullptr) b.qkv.q += static_cast<size_t>(t0) * b.qkv.n_head * b.qkv.head_dim;
    return b;
}

// One wave's activation loads for one (token tile, K tile) item: lane
// (i, G)'s natural bytes 64 G .. 64 G + 63 of token i, and its share of the
// token tile's code sums and scales (lanes 0..31: token lane / 2, half
// lane % 2 of its 16 sums; lanes 32..47: the scale of token lane - 32),
// which the wave passes through LDS.
struct WideAct {
    uint4 xa[4];
    u32x4 st;
};

// The loads of one (token tile tt, K tile b) item. Lanes 0..31 bring half
// lane % 2 of token lane / 2's 16 code sums (SUMS); lanes 32..47 the scale of
// token lane - 32, or with A32 lanes 32..63 half lane % 2 of token
// (lane - 32) / 2's eight 32-value block scales. Token rows past the step
// repeat its last row (their sums are never stored).
template <bool SUMS, bool A32>
__device__ __forceinline__ WideAct wide_load_act(const Act8& xq, int tt, int b, int n_tok, int K, int lane) {
    const int i = lane & 15, G = lane >> 4;
    const size_t tok = static_cast<size_t>(min(16 * tt + i, n_tok - 1));
    WideAct r;
    const uint4* xa = reinterpret_cast<const uint4*>(xq.q + tok * K + b * 256 + 64 * G);
#pragma unroll
    for (int u = 0; u < 4; ++u) r.xa[u] = xa[u];
    const int tl = lane < 32 ? lane >> 1 : (A32 ? (lane - 32) >> 1 : lane - 32);
    const size_t tk = static_cast<size_t>(min(16 * tt + (tl & 15), n_tok - 1));
    if (lane >= 32) {
        if constexpr (A32) r.st = reinterpret_cast<const u32x4*>(xq.d + tk * (K / 32) + 8 * b)[lane & 1];
        else r.st.x = __float_as_uint(xq.d[tk * (K / 256) + b]);
    } else if (SUMS) {
        r.st = reinterpret_cast<const u32x4*>(xq.s + tk * (K / 16) + 16 * b)[lane & 1];
    }
    return r;
}

// Writes a wave's item loads to its LDS slots: sums [token][2] (u32x4),
// scales [token] or (A32) [token][8].
template <bool SUMS, bool A32>
__device__ __forceinline__ void wide_stage(const WideAct& r, int lane, u32x4* sums, float* scales) {
    if (lane < 32) {
        if (SUMS) sums[lane] = r.st;
    } else if (A32) {
        reinterpret_cast<u32x4*>(scales)[lane - 32] = r.st;
    } else if (lane < 48) {
        scales[lane - 32] = __uint_as_float(r.st.x);
    }
}

// A operands from natural activation bytes: stretch s = 2 h + e (values
// 32 s .. 32 s + 31) of lane group G is chunk 4 e + G of lane group h, so
// for each e and 32-bit half the (chunk, lane group) 4 x 4 block is
// transposed with two rounds of lane-group swaps.
__device__ __forceinline__ void wide_a_operands(const uint4 (&xa)[4], long (&av)[8]) {
    const uint32_t n[16] = {xa[0].x, xa[0].y, xa[0].z, xa[0].w, xa[1].x, xa[1].y, xa[1].z, xa[1].w,
                            xa[2].x, xa[2].y, xa[2].z, xa[2].w, xa[3].x, xa[3].y, xa[3].z, xa[3].w};
    uint32_t t[2][2][4];  // [e][half][h]
#pragma unroll
    for (int e = 0; e < 2; ++e) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            // X_r = word 8 e + 2 r + hf (chunk 4 e + r); after the swaps register r holds Y_r
            uint32_t x0 = n[8 * e + hf], x1 = n[8 * e + 2 + hf], x2 = n[8 * e + 4 + hf], x3 = n[8 * e + 6 + hf];
            const auto p02 = __builtin_amdgcn_permlane32_swap(x0, x2, false, false);
            const auto p13 = __builtin_amdgcn_permlane32_swap(x1, x3, false, false);
            const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
            const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
            t[e][hf][0] = q01[0];
            t[e][hf][1] = q01[1];
            t[e][hf][2] = q23[0];
            t[e][hf][3] = q23[1];
        }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
#pragma unroll
        for (int e = 0; e < 2; ++e) av[2 * h + e] = pack2(t[e][0][h], t[e][1][h]);
    }
}

// Work-group = `rpw` 16-row groups (rg, rg + 8, ..., all on one XCD; more
// than one only for the logits head, which then merges one running best per
// token into the step's argmax instead of one per row group) and up to
// kWideTpw consecutive 16-token tiles (`tpw`). A wave keeps each of its K
// tiles' weight operands in registers while it runs that tile for every
// token tile of the group, with one accumulator set per token tile.
constexpr int kWideTpw = 2;

template <uint32_t TYPE, bool MERGED, bool A32>
__global__ __launch_bounds__(kMmThreads) void k_mm_wide(GemvArgs a, int32_t n_rg, int32_t tpw, int32_t rpw) {
    using T = WideTile<TYPE>;
    constexpr int W = kMmWaves;
    constexpr uint32_t TB = tile_bytes(TYPE);
    constexpr int NTOK = 16 * kWideTpw;  // a work-group's token rows
    __shared__ float red[W][4][16][16];  // [wave][lane group][token][row] of one token tile
    __shared__ float vals[NTOK][16];
    __shared__ u32x4 stage_s[W][16][2];
    __shared__ float stage_d[W][A32 ? 16 * 8 : 16];  // scales [token] (A32: [token][8])
    __shared__ unsigned long long best[NTOK];
    float* lv = &red[0][0][0][0];  // the epilogue's scratch (NTOK x 16 floats) once red is read
    static_assert(sizeof(red) >= sizeof(float) * NTOK * 16, "epilogue scratch");
    const int n_tok = a.n_tok, n_tt = (n_tok + 15) / 16, n_grp = (n_tt + tpw - 1) / tpw;
    // work-group k runs on XCD k % 8: the token groups of one row group share an XCD (and its L2)
    const int q = static_cast<int>(blockIdx.x) >> 3;
    const int grp = q % n_grp, rg_first = (q / n_grp) * 8 * rpw + static_cast<int>(blockIdx.x & 7u);
    if (rg_first >= n_rg) return;
    const int K = static_cast<int>(a.mat.cols), nb = K / 256;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int i = lane & 15, G = lane >> 4;
    const int tt0 = grp * tpw, ntl = min(n_tt, tt0 + tpw) - tt0;
    const int t0 = 16 * tt0, nt = min(16 * (tt0 + ntl), n_tok) - t0;
    const GemvArgs out = token_slice(a, t0, nt);
    if (MERGED && threadIdx.x < NTOK) best[threadIdx.x] = 0ull;
    const Act8 xq = a.xq;
    auto load_act = [&](int tt, int b) { return wide_load_act<T::kSums, A32>(xq, tt, b, n_tok, K, lane); };
    for (int rr = 0; rr < (MERGED ? rpw : 1); ++rr) {
        const int rg = rg_first + 8 * rr;
        if (rg >= n_rg) break;
        const uint8_t* base = a.mat.data + static_cast<size_t>(rg) * nb * TB;
        float acc[kWideTpw][4][4];
#pragma unroll
        for (int tl = 0; tl < kWideTpw; ++tl) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[tl][g][j] = 0.0F;
            }
        }
        for (int b = wave; b < nb; b += W) {
            const typename T::Wt w = T::load_w(base + static_cast<size_t>(b) * TB, i, G);
#pragma unroll
            for (int tl = 0; tl < kWideTpw; ++tl) {
                if (tl < ntl) {
                    const WideAct r = load_act(tt0 + tl, b);
                    wide_stage<T::kSums, A32>(r, lane, &stage_s[wave][0][0], stage_d[wave]);
                    __builtin_amdgcn_wave_barrier();
                    long av[8];
                    wide_a_operands(r.xa, av);
                    if constexpr (A32) {
                        T::accumulate32(w, av, reinterpret_cast<const uint32_t*>(&stage_s[wave][0][0]), stage_d[wave],
                                        G, acc[tl]);
                    } else {
                        float xd[4];  // scales of tokens 4 G + j
#pragma unroll
                        for (int j = 0; j < 4; ++j) xd[j] = stage_d[wave][4 * G + j];
                        const typename T::Xt x = T::load_x(reinterpret_cast<const uint32_t*>(&stage_s[wave][i][0]), G);
                        T::accumulate(w, av, x, xd, G, acc[tl]);
                    }
                    __builtin_amdgcn_wave_barrier();
                }
            }
        }
        // per token tile: sum over waves of ((g0 + g1) + (g2 + g3)) (the decode matmul's order)
#pragma unroll
        for (int tl = 0; tl < kWideTpw; ++tl) {
            if (tl < ntl) {
                __syncthreads();
#pragma unroll
                for (int g = 0; g < 4; ++g) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) red[wave][g][4 * G + j][i] = acc[tl][g][j];
                }
                __syncthreads();
                if (threadIdx.x < 256) {
                    const int tk = threadIdx.x >> 4, r = threadIdx.x & 15;
                    float v = 0.0F;
#pragma unroll
                    for (int w = 0; w < W; ++w)
                        v += (red[w][0][tk][r] + red[w][1][tk][r]) + (red[w][2][tk][r] + red[w][3][tk][r]);
                    vals[16 * tl + tk][r] = v;
                }
            }
        }
        __syncthreads();
        const int row0 = rg * 16;
        const int nrows = min(16, static_cast<int>(a.mat.rows) - row0);
        gemv_epilogue<kMmThreads, MERGED ? kLogitsOnly : kNoLogits>(
            out, row0, nrows, [&](int j, int t) { return vals[t][j]; }, lv, MERGED ? best : nullptr);
    }
    if (MERGED) {
        __syncthreads();
        if (threadIdx.x < nt && best[threadIdx.x] != 0ull) atomicMax(out.best + threadIdx.x, best[threadIdx.x]);
    }
}

// The wide matmul of the K-quant formats (Q4_K, Q6_K, Q2_K, whose tiles keep
// one accumulator per (row, token): the integer totals of a tile take one
// float step) over R consecutive 16-row groups per work-group: a wave loads
// its K tile's activations once for the group's token tiles and runs them
// against the R row groups' weight tiles (the next row group's tile in flight
// while the current one is multiplied), so the activation rows are read from
// L2 once per R row groups instead of once per row group. Per (row, token) the
// sum is the one-row-group kernel's: each wave's tiles in K order, the waves
// in order (the lane groups' other accumulators are exact zeros, and adding
// them to a sum that starts at +0 changes no bit), so rows stay bit-identical
// to decode rows.
template <uint32_t TYPE, int R, int TP, bool A32>
__global__ __launch_bounds__(kMmThreads) void k_mm_wide_rg(GemvArgs a, int32_t n_rg, int32_t tpw) {
    using T = WideTile<TYPE>;
    constexpr int W = kMmWaves;
    constexpr uint32_t TB = tile_bytes(TYPE);
    __shared__ float red[W][TP][16][16];  // [wave][token tile][token][row] of one row group
    __shared__ float vals[16 * TP][16 * R];
    __shared__ u32x4 stage_s[W][TP][16][2];
    __shared__ float stage_d[W][TP][A32 ? 16 * 8 : 16];  // scales [token] (A32: [token][8])
    const int n_tok = a.n_tok, n_tt = (n_tok + 15) / 16, n_grp = (n_tt + tpw - 1) / tpw;
    // work-group k runs on XCD k % 8: the token groups of one row-group set share an XCD (and its L2)
    const int q = static_cast<int>(blockIdx.x) >> 3;
    const int grp = q % n_grp, set = (q / n_grp) * 8 + static_cast<int>(blockIdx.x & 7u);
    const int rg0 = set * R;
    if (rg0 >= n_rg) return;
    const int nrg = min(R, n_rg - rg0);
    const int K = static_cast<int>(a.mat.cols), nb = K / 256;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int i = lane & 15, G = lane >> 4;
    const int tt0 = grp * tpw, ntl = min(TP, min(n_tt, tt0 + tpw) - tt0);
    const int t0 = 16 * tt0, nt = min(16 * (tt0 + ntl), n_tok) - t0;
    const GemvArgs out = token_slice(a, t0, nt);
    const Act8 xq = a.xq;
    auto load_act = [&](int tt, int b) { return wide_load_act<T::kSums, A32>(xq, tt, b, n_tok, K, lane); };
    const uint8_t* base = a.mat.data + static_cast<size_t>(rg0) * nb * TB;
    float acc[R][TP][4][4];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
#pragma unroll
        for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[rr][tl][g][j] = 0.0F;
            }
        }
    }
    for (int b = wave; b < nb; b += W) {
        // the first row group's tile, then the token tiles' activations (clamped: issued unconditionally)
        typename T::Wt w = T::load_w(base + static_cast<size_t>(b) * TB, i, G);
        long av[TP][8];
        float xd[TP][4];
        typename T::Xt x[TP];
#pragma unroll
        for (int tl = 0; tl < TP; ++tl) {
            const WideAct r = load_act(tt0 + min(tl, ntl - 1), b);
            wide_stage<T::kSums, A32>(r, lane, &stage_s[wave][tl][0][0], stage_d[wave][tl]);
            wide_a_operands(r.xa, av[tl]);
        }
        __builtin_amdgcn_wave_barrier();
        if constexpr (!A32) {
#pragma unroll
            for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
                for (int j = 0; j < 4; ++j) xd[tl][j] = stage_d[wave][tl][4 * G + j];
                x[tl] = T::load_x(reinterpret_cast<const uint32_t*>(&stage_s[wave][tl][i][0]), G);
            }
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            // the next row group's tile (clamped to the group's last) is requested before this one runs
            const typename T::Wt wn =
                T::load_w(base + (static_cast<size_t>(min(rr + 1, nrg - 1)) * nb + b) * TB, i, G);
            if (rr < nrg) {
#pragma unroll
                for (int tl = 0; tl < TP; ++tl) {
                    if (tl < ntl) {
                        if constexpr (A32) {
                            T::accumulate32(w, av[tl], reinterpret_cast<const uint32_t*>(&stage_s[wave][tl][0][0]),
                                            stage_d[wave][tl], G, acc[rr][tl]);
                        } else {
                            T::accumulate(w, av[tl], x[tl], xd[tl], G, acc[rr][tl]);
                        }
                    }
                }
            }
            w = wn;
        }
        // the staged sums and scales are read until the last row group has run
        if constexpr (A32) __builtin_amdgcn_wave_barrier();
    }
    // per row group and token tile: the sum over waves in wave order
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        if (rr < nrg) {
            __syncthreads();
#pragma unroll
            for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
                for (int j = 0; j < 4; ++j) red[wave][tl][4 * G + j][i] = acc[rr][tl][0][j];
            }
            __syncthreads();
            for (int e = threadIdx.x; e < ntl * 256; e += kMmThreads) {
                const int tl = e >> 8, tk = (e >> 4) & 15, r = e & 15;
                float v = 0.0F;
#pragma unroll
                for (int w2 = 0; w2 < W; ++w2) v += red[w2][tl][tk][r];
                vals[16 * tl + tk][16 * rr + r] = v;
            }
        }
    }
    __syncthreads();
    const int row0 = rg0 * 16;
    const int nrows = min(16 * nrg, static_cast<int>(a.mat.rows) - row0);
    gemv_epilogue<kMmThreads, kNoLogits>(out, row0, nrows, [&](int j, int t) { return vals[t][j]; },
                                         &red[0][0][0][0]);
}

// The wide Q4_K matmul for steps with many row groups (the gate / up matrix
// of a prefill chunk): the sub-block scales are folded into the weight
// operand, each wave owns one 16-row group over the whole of K, and the
// work-group's waves share every activation tile through LDS.
//
// Scale fold: a Q4_K scale sc (6 bits) times a code (4 bits) does not fit an
// int8, but sc = 8 sh + sl with sh, sl < 8 does: sl * code and sh * code are
// at most 105, so two chains of v_mfma_i32_16x16x64_i8 give every (row,
// token) the tile's totals L = sum_j sl_j dot_j and H = sum_j sh_j dot_j, and
// L + 8 H is the integer total sum_j sc_j dot_j of the decode dot. Lane (i,
// G) brings row i's codes of sub-block pair G (chunks 0, 1: the low nibbles,
// sub-block 2 G; chunks 2, 3: the high ones, 2 G + 1), each word folded with
// its sub-block's sl or sh by one packed 16-bit multiply (the byte products
// stay below 256, so no carry crosses a byte), against token i's activation
// bytes 64 G .. 64 G + 63 at the same positions. The folded operands are made
// once per K tile and serve every token tile of the work-group. The min sums
// sum_j m_j S_j (exact integers below 2^24) come from two
// v_mfma_f32_16x16x4f32 (K = lane group G: sub-blocks 2 G, 2 G + 1). With the
// weights as the first operand D gives lane (i, G) rows 4 G + r of token i.
//
// Order: the decode matmul's wave w sums the tiles w, w + 8, ... with one
// q4k_term_f step each and the eight partials are added in wave order. A wave
// here walks the tiles in that order (0, 8, 16, ..., then 1, 9, ..., ...),
// keeps the running partial of the current chain and adds it to the total
// when the chain ends, so every row equals the decode row bit for bit with no
// cross-wave reduction.
//
// Staging: the work-group's token rows of the next K tile (codes, 16-value
// sums, scales) are written to the other of two LDS buffers; one barrier per
// tile. With four token tiles per work-group (long steps) the next tile's
// staging loads are issued after the current tile's work and a wave loads
// its weight tile when the tile starts: no register is held across a tile
// for the next one, so four work-groups fit on a CU (128 VGPRs, 39 KB of LDS
// each), whose waves hide each other's load latency. With one or two token
// tiles (9..32-row steps) a tile's work is short, and both loads are issued
// one tile ahead.
constexpr int kStageRow = 272;  // bytes per staged token row: 256 codes + 16 bytes of padding (banks)

template <int NW, int TP>
__global__ __launch_bounds__(NW * kWave) void k_mm_wide_q4k(GemvArgs a, int32_t n_rg, int32_t tpw) {
    constexpr int NTHR = NW * kWave;
    constexpr int NTOK = 16 * TP;
    constexpr uint32_t TB = tile_bytes(11);
    constexpr uint32_t M4 = 0x0F0F0F0Fu;
    constexpr int CODE_CHUNKS = NTOK * 16;  // 16-byte pieces of a staged tile's codes
    static_assert(CODE_CHUNKS % NTHR == 0, "whole code pieces per thread");
    constexpr int CPT = CODE_CHUNKS / NTHR;
    constexpr int VSTRIDE = 16 * NW + 1;  // epilogue row stride (floats)
    __shared__ __align__(16) uint8_t codes[2][NTOK * kStageRow];
    __shared__ __align__(16) f32x4 sums[2][NTOK][2];  // the 32-value code sums of the tile's eight sub-blocks
    __shared__ float scales[2][NTOK];
    static_assert(sizeof(float) * NTOK * VSTRIDE <= sizeof(codes), "epilogue values alias the staging buffers");
    float* vals = reinterpret_cast<float*>(&codes[0][0]);
    const int n_tok = a.n_tok, n_tt = (n_tok + 15) / 16, n_grp = (n_tt + tpw - 1) / tpw;
    const int n_sets = (n_rg + NW - 1) / NW;
    // work-group k runs on XCD k % 8: the token groups of one row-group set share an XCD (and its L2)
    const int q = static_cast<int>(blockIdx.x) >> 3;
    const int grp = q % n_grp, set = (q / n_grp) * 8 + static_cast<int>(blockIdx.x & 7u);
    if (set >= n_sets) return;
    const int K = static_cast<int>(a.mat.cols), nb = K / 256;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int i = lane & 15, G = lane >> 4;
    const int tt0 = grp * tpw, ntl = min(TP, min(n_tt, tt0 + tpw) - tt0);
    const int t0 = 16 * tt0, nt = min(16 * (tt0 + ntl), n_tok) - t0;
    const GemvArgs out = token_slice(a, t0, nt);
    const Act8 xq = a.xq;
    const int rg = set * NW + wave;
    const bool active = rg < n_rg;  // waves past the matrix stage and wait but compute nothing
    const uint8_t* base = a.mat.data + static_cast<size_t>(min(rg, n_rg - 1)) * nb * TB;

    // staging loads of K tile b into registers (token rows past the step repeat its last row)
    struct Stage {
        u32x4 c[CPT];
        u32x4 s;
        float d;
    };
    // element offsets are unsigned 32-bit (rows of at most kWideRows tokens)
    auto stage_load = [&](int b) {
        Stage st;
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const uint32_t e = threadIdx.x + u * NTHR, tk = e >> 4, part = e & 15;
            const uint32_t tok = static_cast<uint32_t>(min(t0 + static_cast<int>(tk), n_tok - 1));
            st.c[u] = *reinterpret_cast<const u32x4*>(xq.q + (tok * static_cast<uint32_t>(K) + 256u * b + 16u * part));
        }
        if (threadIdx.x < 2 * NTOK) {
            const uint32_t tok = static_cast<uint32_t>(min(t0 + static_cast<int>(threadIdx.x >> 1), n_tok - 1));
            st.s = *reinterpret_cast<const u32x4*>(xq.s + (tok * static_cast<uint32_t>(K / 16) + 16u * b + 8u * (threadIdx.x & 1)));
        }
        if (threadIdx.x < NTOK) {
            const uint32_t tok = static_cast<uint32_t>(min(t0 + static_cast<int>(threadIdx.x), n_tok - 1));
            st.d = xq.d[tok * static_cast<uint32_t>(nb) + b];
        }
        return st;
    };
    // the 16-value sums, pairwise: sub-block sums as exact floats
    auto sub_sum = [](uint32_t w) {
        return static_cast<float>(static_cast<int16_t>(w & 0xFFFFu) + (static_cast<int32_t>(w) >> 16));
    };
    auto stage_store = [&](const Stage& st, int buf) {
#pragma unroll
        for (int u = 0; u < CPT; ++u) {
            const int e = threadIdx.x + u * NTHR, tk = e >> 4, part = e & 15;
            *reinterpret_cast<u32x4*>(&codes[buf][tk * kStageRow + 16 * part]) = st.c[u];
        }
        if (threadIdx.x < 2 * NTOK) {
            sums[buf][threadIdx.x >> 1][threadIdx.x & 1] =
                f32x4{sub_sum(st.s.x), sub_sum(st.s.y), sub_sum(st.s.z), sub_sum(st.s.w)};
        }
        if (threadIdx.x < NTOK) scales[buf][threadIdx.x] = st.d;
    };
    // the lane's share of a weight tile: rows 4 G + r's scales, row i's field pair and code words
    struct Raw {
        uint32_t dd[4];
        uint2 fw;
        u32x4 w0, w1;
    };
    auto load_raw = [&](int b) {
        const uint8_t* t = base + static_cast<size_t>(b) * TB;
        Raw r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.dd[j] = *reinterpret_cast<const uint32_t*>(t + 16 * (4 * G + j));
        r.fw = *reinterpret_cast<const uint2*>(t + 16 * i + 4 + 4 * ((3 * G) >> 2));
        r.w0 = *reinterpret_cast<const u32x4*>(t + 256 + 16 * lane);
        r.w1 = *reinterpret_cast<const u32x4*>(t + 1280 + 16 * lane);
        return r;
    };
    // the tile after b in the decode waves' order
    auto next_tile = [&](int b) { return b + 8 < nb ? b + 8 : (b & 7) + 1; };

    float total[TP][4], chain[TP][4];
#pragma unroll
    for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
        for (int j = 0; j < 4; ++j) total[tl][j] = chain[tl][j] = 0.0F;
    }
    // one or two token tiles: the next tile's loads are issued before this tile's work (a short
    // tile hides little latency); four: after it, so that no register is held across a tile
    constexpr bool AHEAD = TP < 4;
    stage_store(stage_load(0), 0);
    Raw ahead{};
    if constexpr (AHEAD) ahead = load_raw(0);
    __syncthreads();
    int b = 0;
    for (int s = 0; s < nb; ++s) {
        const int buf = s & 1;
        const int bn = s + 1 < nb ? next_tile(b) : b;  // clamped: issued unconditionally
        Stage st{};
        Raw nxt{};
        if constexpr (AHEAD) {
            st = stage_load(bn);
            nxt = load_raw(bn);
        }
        const Raw cur = AHEAD ? ahead : load_raw(b);
        if (active) {
            // lane group G's 24-bit field of row i: sc 2G | sc 2G+1 | m 2G | m 2G+1
            const uint32_t f = __builtin_amdgcn_alignbyte(cur.fw.y, cur.fw.x, (3 * G) & 3);
            const uint32_t sca = f & 63u, scb = (f >> 6) & 63u;
            const float ma = static_cast<float>((f >> 12) & 63u), mb = static_cast<float>((f >> 18) & 63u);
            const u16x2 la = {static_cast<uint16_t>(sca & 7u), static_cast<uint16_t>(sca & 7u)};
            const u16x2 ha = {static_cast<uint16_t>(sca >> 3), static_cast<uint16_t>(sca >> 3)};
            const u16x2 lb = {static_cast<uint16_t>(scb & 7u), static_cast<uint16_t>(scb & 7u)};
            const u16x2 hb = {static_cast<uint16_t>(scb >> 3), static_cast<uint16_t>(scb >> 3)};
            auto fold = [](uint32_t c, u16x2 sv) {
                return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, c) * sv);
            };
            float d[4], dmin[4];  // rows 4 G + j
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d[j] = h2f(cur.dd[j]);
                dmin[j] = h2f(cur.dd[j] >> 16);
            }
            u32x4 BL[4], BH[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t l0 = cur.w0[k] & M4, l1 = cur.w1[k] & M4;
                const uint32_t h0 = (cur.w0[k] >> 4) & M4, h1 = (cur.w1[k] >> 4) & M4;
                BL[0][k] = fold(l0, la);
                BL[1][k] = fold(l1, la);
                BL[2][k] = fold(h0, lb);
                BL[3][k] = fold(h1, lb);
                BH[0][k] = fold(l0, ha);
                BH[1][k] = fold(l1, ha);
                BH[2][k] = fold(h0, hb);
                BH[3][k] = fold(h1, hb);
            }
#pragma unroll
            for (int tl = 0; tl < TP; ++tl) {
                if (tl < ntl) {
                    const int r = 16 * tl + i;
                    const u32x4* src = reinterpret_cast<const u32x4*>(&codes[buf][r * kStageRow + 64 * G]);
                    const float2 xs = reinterpret_cast<const float2*>(&sums[buf][r][0])[G];
                    const float xd = scales[buf][r];
                    i32x4 DL = {0, 0, 0, 0}, DH = {0, 0, 0, 0};
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const i32x4 av = __builtin_bit_cast(i32x4, src[m]);
                        DL = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, BL[m]), av, DL, 0, 0, 0);
                        DH = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, BH[m]), av, DH, 0, 0, 0);
                    }
                    // token r's 32-value code sums of sub-blocks 2G, 2G + 1
                    f32x4 ms = {0.0F, 0.0F, 0.0F, 0.0F};
                    ms = __builtin_amdgcn_mfma_f32_16x16x4f32(ma, xs.x, ms, 0, 0, 0);
                    ms = __builtin_amdgcn_mfma_f32_16x16x4f32(mb, xs.y, ms, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        chain[tl][j] = q4k_term_f(chain[tl][j], xd, d[j], dmin[j], DL[j] + 8 * DH[j], ms[j]);
                }
            }
            if (b + 8 >= nb) {
                // the chain of tiles b mod 8 ends: its partial joins the total in wave order
#pragma unroll
                for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        total[tl][j] += chain[tl][j];
                        chain[tl][j] = 0.0F;
                    }
                }
            }
        }
        // the next tile's staging loads after this tile's work (their registers are not held across it)
        if constexpr (AHEAD) {
            if (s + 1 < nb) stage_store(st, buf ^ 1);
            ahead = nxt;
        } else {
            __builtin_amdgcn_sched_barrier(0);
            if (s + 1 < nb) stage_store(stage_load(bn), buf ^ 1);
        }
        b = bn;
        __syncthreads();
    }
    // the staging buffers are free (the loop ends on a barrier): rows and tokens to the epilogue
    if (active) {
#pragma unroll
        for (int tl = 0; tl < TP; ++tl) {
#pragma unroll
            for (int j = 0; j < 4; ++j) vals[(16 * tl + i) * VSTRIDE + 16 * wave + 4 * G + j] = total[tl][j];
        }
    }
    __syncthreads();
    const int row0 = set * NW * 16;
    const int nrows = min(16 * NW, static_cast<int>(a.mat.rows) - row0);
    gemv_epilogue<NTHR, kNoLogits>(out, row0, nrows, [&](int j, int tk) { return vals[tk * VSTRIDE + j]; }, nullptr);
}

// The wide Q4_K matmul for steps with fewer row groups (the down, output
// and qkv matrices of a prefill chunk): the decode matmul's eight waves (wave
// w takes the K tiles w, w + 8, ...), R consecutive row groups and one
// 16-token tile per work-group, and the folded-scale tile arithmetic of
// k_mm_wide_q4k. A wave loads its K tile's activations (lane (i, G): token
// i's bytes 64 G .. 64 G + 63, its code sums and scale) once and runs them
// against the R row groups' folded weight operands, the next weight tile in
// flight while one runs; the waves' partials are summed in wave order through
// LDS, so every row equals the decode row bit for bit.
template <int R>
__global__ __launch_bounds__(kMmThreads) void k_mm_wide_q4r(GemvArgs a, int32_t n_rg) {
    constexpr int W = kMmWaves;
    constexpr uint32_t TB = tile_bytes(11);
    constexpr uint32_t M4 = 0x0F0F0F0Fu;
    __shared__ float red[W][16][16 * R];  // [wave][token][row]
    __shared__ float vals[16][16 * R];
    const int n_tok = a.n_tok, n_tt = (n_tok + 15) / 16;
    // work-group k runs on XCD k % 8: the token tiles of one row-group set share an XCD (and its L2)
    const int q = static_cast<int>(blockIdx.x) >> 3;
    const int tt = q % n_tt, set = (q / n_tt) * 8 + static_cast<int>(blockIdx.x & 7u);
    const int rg0 = set * R;
    if (rg0 >= n_rg) return;
    const int nrg = min(R, n_rg - rg0);
    const int K = static_cast<int>(a.mat.cols), nb = K / 256;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int i = lane & 15, G = lane >> 4;
    const int t0 = 16 * tt, nt = min(16, n_tok - t0);
    const GemvArgs out = token_slice(a, t0, nt);
    const Act8 xq = a.xq;
    // the lane's token (rows past the step repeat its last row; never stored)
    const uint32_t tok = static_cast<uint32_t>(min(t0 + i, n_tok - 1));
    const uint8_t* base = a.mat.data + static_cast<size_t>(rg0) * nb * TB;
    struct Raw {
        uint32_t dd[4];
        uint2 fw;
        u32x4 w0, w1;
    };
    auto load_raw = [&](int rr, int b) {
        const uint8_t* t = base + (static_cast<size_t>(rr) * nb + b) * TB;
        Raw r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.dd[j] = *reinterpret_cast<const uint32_t*>(t + 16 * (4 * G + j));
        r.fw = *reinterpret_cast<const uint2*>(t + 16 * i + 4 + 4 * ((3 * G) >> 2));
        r.w0 = *reinterpret_cast<const u32x4*>(t + 256 + 16 * lane);
        r.w1 = *reinterpret_cast<const u32x4*>(t + 1280 + 16 * lane);
        return r;
    };
    auto sub_sum = [](uint32_t w) {
        return static_cast<float>(static_cast<int16_t>(w & 0xFFFFu) + (static_cast<int32_t>(w) >> 16));
    };
    float acc[R][4];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rr][j] = 0.0F;
    }
    Raw cur = load_raw(0, min(wave, nb - 1));
    for (int b = wave; b < nb; b += W) {
        const u32x4* src = reinterpret_cast<const u32x4*>(xq.q + (tok * static_cast<uint32_t>(K) + 256u * b + 64u * G));
        u32x4 xa[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) xa[m] = src[m];
        const uint2 sw = *reinterpret_cast<const uint2*>(xq.s + (tok * static_cast<uint32_t>(K / 16) + 16u * b + 4u * G));
        const float xd = xq.d[tok * static_cast<uint32_t>(nb) + b];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            // the next weight tile (the next row group's, else the wave's next K tile's first; clamped)
            const Raw nxt = rr + 1 < nrg ? load_raw(rr + 1, b) : load_raw(0, min(b + W, nb - 1));
            if (rr < nrg) {
                float d[4], dmin[4];  // rows 4 G + j
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    d[j] = h2f(cur.dd[j]);
                    dmin[j] = h2f(cur.dd[j] >> 16);
                }
                // lane group G's 24-bit field of row i: sc 2G | sc 2G+1 | m 2G | m 2G+1
                const uint32_t f = __builtin_amdgcn_alignbyte(cur.fw.y, cur.fw.x, (3 * G) & 3);
                const uint32_t sca = f & 63u, scb = (f >> 6) & 63u;
                const float ma = static_cast<float>((f >> 12) & 63u), mb = static_cast<float>((f >> 18) & 63u);
                const u16x2 la = {static_cast<uint16_t>(sca & 7u), static_cast<uint16_t>(sca & 7u)};
                const u16x2 ha = {static_cast<uint16_t>(sca >> 3), static_cast<uint16_t>(sca >> 3)};
                const u16x2 lb = {static_cast<uint16_t>(scb & 7u), static_cast<uint16_t>(scb & 7u)};
                const u16x2 hb = {static_cast<uint16_t>(scb >> 3), static_cast<uint16_t>(scb >> 3)};
                auto fold = [](uint32_t c, u16x2 sv) {
                    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, c) * sv);
                };
                i32x4 DL = {0, 0, 0, 0}, DH = {0, 0, 0, 0};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const u32x4 w = m & 1 ? cur.w1 : cur.w0;
                    const u16x2 sl = m < 2 ? la : lb, sh = m < 2 ? ha : hb;
                    u32x4 bl, bh;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t c = m < 2 ? w[k] & M4 : (w[k] >> 4) & M4;
                        bl[k] = fold(c, sl);
                        bh[k] = fold(c, sh);
                    }
                    const i32x4 av = __builtin_bit_cast(i32x4, xa[m]);
                    DL = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, bl), av, DL, 0, 0, 0);
                    DH = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, bh), av, DH, 0, 0, 0);
                }
                // token i's 32-value code sums of sub-blocks 2G, 2G + 1
                f32x4 ms = {0.0F, 0.0F, 0.0F, 0.0F};
                ms = __builtin_amdgcn_mfma_f32_16x16x4f32(ma, sub_sum(sw.x), ms, 0, 0, 0);
                ms = __builtin_amdgcn_mfma_f32_16x16x4f32(mb, sub_sum(sw.y), ms, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[rr][j] = q4k_term_f(acc[rr][j], xd, d[j], dmin[j], DL[j] + 8 * DH[j], ms[j]);
            }
            cur = nxt;
        }
    }
    // per row group: the sum over waves in wave order
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[wave][i][16 * rr + 4 * G + j] = acc[rr][j];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * 16 * nrg; e += kMmThreads) {
        const int tk = e / (16 * nrg), r = e - tk * 16 * nrg;
        float v = 0.0F;
#pragma unroll
        for (int w2 = 0; w2 < W; ++w2) v += red[w2][tk][r];
        vals[tk][r] = v;
    }
    __syncthreads();
    const int row0 = rg0 * 16;
    const int nrows = min(16 * nrg, static_cast<int>(a.mat.rows) - row0);
    gemv_epilogue<kMmThreads, kNoLogits>(out, row0, nrows, [&](int j, int tk) { return vals[tk][j]; }, nullptr);
}

// Float weights (F32/F16, small models): one wave per row, lanes over K,
// float activations (RMS-normalized in the prologue when a gain is given).
constexpr int kFloatThreads = 256;
constexpr int kGemvFloatRows = 2 * kGluGroup;

template <int NT>
__global__ __launch_bounds__(kFloatThreads) void k_gemv_f(GemvArgs a, int32_t rows_per_wg) {
    constexpr int W = kFloatThreads / kWave;
    __shared__ float rs[NT], red[NT * W];
    __shared__ float sums[kGemvFloatRows][NT];
    extern __shared__ float lv_f[];
    const int K = static_cast<int>(a.mat.cols);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n_tok = a.n_tok < NT ? a.n_tok : NT;
    if (a.x.gain) row_rms<NT, kFloatThreads>(a.x, n_tok, K, rs, red);
    const int RW = rows_per_wg, row0 = blockIdx.x * RW;
    const int nrows = min(RW, static_cast<int>(a.mat.rows) - row0);
    for (int j = wave; j < RW; j += W) {
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
    gemv_epilogue<kFloatThreads>(b, row0, nrows, [&](int j, int t) { return sums[j][t]; }, lv_f);
}

// ------------------------------------------------------------------ activation quantization kernel
// One wave per 256 values: rows [0, n_rows) of x (stride floats apart) into
// the staging layout of `out` (one 256-value block, or eight 32-value blocks).
__global__ __launch_bounds__(256) void k_quantize(const float* x, int32_t stride, Act8 out) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int b = blockIdx.x * 4 + wave, row = blockIdx.y;
    if (b * 256 >= out.K) return;
    const float4 v4 = *reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * stride + b * 256 + 4 * lane);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    int8_t* q = out.q + static_cast<size_t>(row) * out.K + b * 256;
    int16_t* s = out.s + static_cast<size_t>(row) * (out.K / 16) + b * 16;
    if (out.blk == kActBlock32) quant_block_wave32<false>(v, lane, q, out.d + static_cast<size_t>(row) * (out.K / 32) + 8 * b, s);
    else quant_block_wave(v, lane, q, out.d + static_cast<size_t>(row) * (out.K / 256) + b, s);
}

// RMSNorm x gain + quantization of whole rows, one work-group per row: the
// codes and scales the normalized-input matmul prologue stages (stage_f32
// with a gain, then finish_norm), computed the same way (prefill steps).
constexpr int kNormMaxBlocks = 128;
constexpr int kNormThreads = 1024;  // a wave per block for rows up to 4096 values
#pragma clang fp contract(off)
__global__ __launch_bounds__(kNormThreads) void k_quantize_norm(const float* x, int32_t stride, const int32_t* gather,
                                                       const float* gain, float eps, Act8 out) {
    __shared__ float ssq[kNormMaxBlocks], db[kNormMaxBlocks * 8];
    __shared__ float rs;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int row = blockIdx.x, nb = out.K / 256;
    const bool a32 = out.blk == kActBlock32;
    const float* xr = x + static_cast<size_t>(gather ? gather[row] : row) * stride;
    for (int b = wave; b < nb; b += kNormThreads / kWave) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(xr + b * 256 + 4 * lane);
        const f32x4 g4 = *reinterpret_cast<const f32x4*>(gain + b * 256 + 4 * lane);
        float vv[4] = {v4.x, v4.y, v4.z, v4.w};
        const float sq2 = wave_sum(vv[0] * vv[0] + vv[1] * vv[1] + vv[2] * vv[2] + vv[3] * vv[3]);
        if (lane == 0) ssq[b] = sq2;
        vv[0] = vv[0] * g4.x;
        vv[1] = vv[1] * g4.y;
        vv[2] = vv[2] * g4.z;
        vv[3] = vv[3] * g4.w;
        int8_t* q = out.q + static_cast<size_t>(row) * out.K + b * 256;
        int16_t* s = out.s + static_cast<size_t>(row) * (out.K / 16) + b * 16;
        if (a32) quant_block_wave32<true>(vv, lane, q, &db[8 * b], s);
        else quant_block_wave(vv, lane, q, &db[b], s);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0F;
        for (int b = 0; b < nb; ++b) sum += ssq[b];
        rs = 1.0F / sqrtf(sum / static_cast<float>(out.K) + eps);
    }
    __syncthreads();
    // the scales times the row's 1/rms (32-value block scales then rounded to f16, as finish_norm)
    const int nd = a32 ? 8 * nb : nb;
    for (int b = threadIdx.x; b < nd; b += kNormThreads) {
        const float v = db[b] * rs;
        out.d[static_cast<size_t>(row) * nd + b] = a32 ? round_f16(v) : v;
    }
}
#pragma clang fp contract(on)

// ------------------------------------------------------------------ attention
// Split-K causal GQA flash attention (qwen2_architecture.cpp:438-464, mask
// 697-708) over the f16 caches. Work-group = (key split, kv head x query
// group, sequence); a query group is up to kAttnQPW of the G*T query rows that
// share the kv head, staged in LDS. Each wave takes 16-key tiles: for Q.K a
// quad of lanes holds one key (a quarter of its dims each) and the score is
// quad-reduced; for P.V the lanes own two head dims each. K and V of a tile
// are loaded together. The four waves' online-softmax states are merged in
// LDS and written as the split's (max, sum, output) partial;
// k_attention_merge combines the splits.
constexpr int kAttnThreads = 256;
constexpr int kAttnQPW = 8;
constexpr int kAttnTile = 16;
constexpr int kAttnWgKeys = kAttnTile * (kAttnThreads / kWave);
constexpr int kAttnMaxSplits = 32;

constexpr int kAttnPrefillKeys = 512;
// Work-groups of the matrix-core attention resident at once: two per CU
// (four waves each at its two waves per SIMD) on 256 CUs.
constexpr int kAttnResidentWgs = 512;
// Keys per split of a sequence with n_keys keys and len rows in the step: the
// decode rule (about n_keys / splits_max, in whole rounds of the work-group's
// waves), which depends on the position alone, so a verify or batched step
// splits every row's keys exactly as serial decode does; a sequence bringing
// more rows than any verify step (a prefill chunk) takes splits of at least
// kAttnPrefillKeys keys, several tiles per wave. The attention and merge
// kernels use the same rule.
__device__ __forceinline__ int attn_split_len(int n_keys, int len, int splits_max) {
    int L = (n_keys + splits_max - 1) / splits_max;
    L = (L + kAttnWgKeys - 1) / kAttnWgKeys * kAttnWgKeys;
    if (len > kQuadGroupRows) L = max(L, kAttnPrefillKeys);
    return L;
}

// A work-group whose key split lies beyond the sequence's last key marks the
// split empty (max -inf) for its query rows, so that every split slot below
// splits_max holds this step's maximum and the merge reads the slots without
// consulting the step descriptor (it ignores the sum and output of a split
// whose maximum is -inf).
template <int NTHR>
__device__ __forceinline__ void attn_empty_split(float* partial, int q_begin, int nq, int G, int kvh, int row0,
                                                 int n_head, int hd, int splits_max, int split) {
    for (int i = threadIdx.x; i < nq; i += NTHR) {
        const int qi = q_begin + i;
        const int t = qi / G, head = kvh * G + qi % G;
        partial[((static_cast<size_t>(row0 + t) * n_head + head) * splits_max + split) * (hd + 2)] = -INFINITY;
    }
}

// K quarter of the lane's key (HD > 0) and the lane's V pair of all 16 keys of the tile at t0.
template <int HD>
__device__ __forceinline__ void attn_load_tile(global_ptr<const uint16_t> kc, global_ptr<const uint16_t> vc, int t0,
                                               int capacity, int hd, int kk, int qq, int lane, uint4* kr,
                                               uint32_t* vv) {
    if constexpr (HD > 0) {
        global_ptr<const uint16_t> krow = kc + static_cast<size_t>(min(t0 + kk, capacity - 1)) * HD;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) kr[c] = load_u4(krow + qq * (HD / 4) + 8 * c);
    }
    // V is stored in 16-position tiles ([position / 16][dim][position % 16]): the
    // lane's two dims come from two rows of the key's tile
    const int d0 = min(2 * lane, hd - 1), d1 = min(2 * lane + 1, hd - 1);
#pragma unroll
    for (int u = 0; u < kAttnTile; ++u) {
        const int kj = min(t0 + u, capacity - 1);
        const size_t tile = static_cast<size_t>(kj & ~15) * hd + (kj & 15);
        const uint32_t lo = vc[tile + static_cast<size_t>(d0) * 16];
        const uint32_t hi = vc[tile + static_cast<size_t>(d1) * 16];
        vv[u] = 2 * lane < hd ? (lo | (hi << 16)) : 0u;
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void k_attention(const float* __restrict__ q,
                                                            const StepDev* __restrict__ step, int32_t layer,
                                                            int32_t n_head, int32_t n_head_kv, int32_t hd_arg,
                                                            int32_t splits_max, int32_t qgroups,
                                                            float* __restrict__ partial) {
    constexpr int QPW = kAttnQPW, W = kAttnThreads / kWave;
    constexpr int QS = (HD > 0 ? HD : 128) + 16;  // LDS row stride of a query (quarters padded by 4)
    __shared__ __align__(16) float Qs[QPW][QS];
    __shared__ __align__(16) float P[W][QPW][kAttnTile];
    __shared__ float Ms[W][QPW], Ls[W][QPW];
    __shared__ __align__(16) float Os[W][QPW][128];
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
    const int L = attn_split_len(n_keys, len, splits_max);
    const int n_splits = (n_keys + L - 1) / L;
    const int split = blockIdx.x;
    if (split >= n_splits) {
        attn_empty_split<kAttnThreads>(partial, q_begin, nq, G, kvh, row0, n_head, hd, splits_max, split);
        return;
    }
    const int k0 = split * L, k1 = min(n_keys, k0 + L);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int kk = lane >> 2, qq = lane & 3;
    const float scale = 1.0F / sqrtf(static_cast<float>(hd));
    const size_t head_base = (static_cast<size_t>(layer) * n_head_kv + kvh) * capacity;
    global_ptr<const uint16_t> kc = as_global(static_cast<const uint16_t*>(step->seqs[seq].k)) + head_base * hd;
    global_ptr<const uint16_t> vc = as_global(static_cast<const uint16_t*>(step->seqs[seq].v)) + head_base * hd;

    // K and V of the wave's first tile are requested before the queries are
    // staged; every load index is clamped so that the loads are issued
    // unconditionally and overlap
    int t0 = k0 + wave * kAttnTile;
    uint4 kr[HD > 0 ? HD / 32 : 1];
    uint32_t vv[kAttnTile];
    attn_load_tile<HD>(kc, vc, min(t0, k1 - 1), capacity, hd, kk, qq, lane, kr, vv);
    // queries -> LDS, quarter c of row i at Qs[i][c * (DQ + 4)]
    constexpr int QE = (QPW * (HD > 0 ? HD : 128) + kAttnThreads - 1) / kAttnThreads;
    float qv[QE];
#pragma unroll
    for (int u = 0; u < QE; ++u) {
        const int e = min(static_cast<int>(threadIdx.x) + u * kAttnThreads, QPW * hd - 1);
        const int i = e / hd, d = e - i * hd;
        const int qi = q_begin + min(i, nq - 1);
        const int t = qi / G, head = kvh * G + qi % G;
        qv[u] = q[static_cast<size_t>(row0 + t) * H + head * hd + d];
    }
#pragma unroll
    for (int u = 0; u < QE; ++u) {
        const int e = threadIdx.x + u * kAttnThreads;
        if (e < QPW * hd) {
            const int i = e / hd, d = e - i * hd;
            Qs[i][(d / DQ) * (DQ + 4) + d % DQ] = qv[u];
        }
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
    for (; t0 < k1; t0 += W * kAttnTile) {
        const int key = t0 + kk;
        const int keyc = min(key, capacity - 1);
        // next tile's K and V are requested before this tile is consumed
        const int tn = t0 + W * kAttnTile;
        uint4 krn[HD > 0 ? HD / 32 : 1];
        uint32_t vvn[kAttnTile];
        attn_load_tile<HD>(kc, vc, min(tn, k1 - 1), capacity, hd, kk, qq, lane, krn, vvn);
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
            global_ptr<const uint16_t> kq = kc + static_cast<size_t>(keyc) * hd + qq * DQ;
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
#pragma unroll
        for (int c = 0; c < (HD > 0 ? HD / 32 : 1); ++c) kr[c] = krn[c];
#pragma unroll
        for (int u = 0; u < kAttnTile; ++u) vv[u] = vvn[u];
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
    for (int e = threadIdx.x; e < nq * half_hd; e += kAttnThreads) {
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
        float* dst = partial + ((static_cast<size_t>(row0 + t) * n_head + head) * splits_max + split) * (hd + 2);
        if (dp == 0) {
            dst[0] = M;
            dst[1] = Lsum;
        }
        dst[2 + 2 * dp] = a0;
        dst[3 + 2 * dp] = a1;
    }
}

// ------------------------------------------------------------------ attention on matrix cores
// The same split-K causal GQA attention for head dims 64 and 128 on MFMA.
// Work-group = (key split, kv head x group of 16 query rows, sequence); the
// 16 query rows (G heads x tokens) are the N side of both products. Each wave
// takes 16-key tiles:
//   S^T[16 keys][16 rows] = K[16 keys][hd] . Q^T[hd][16 rows]     (16x16x32 f16)
//   O^T[hd][16 rows]     += V^T[hd][16 keys] . P^T[16 keys][16 rows] (16x16x16 f16)
// K is read as stored (position-major rows) and V from its tile-blocked cache
// (per 16 positions, [dim][position]), so every operand is a contiguous
// per-lane load and a tile's V is one contiguous block. The
// queries (scaled by hd^-1/2) and the probabilities enter as f16 hi + lo
// pairs, which keeps the products at about 22 bits. Lane l holds row l % 16
// of the S^T and O^T fragments, so a row's online-softmax state lives in the
// four lanes l % 16 + 16 j. Output: the split's (max, sum, output) partial,
// as from k_attention.
constexpr int kAttnRows = 16;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <int HD>
__device__ __forceinline__ void attn_mfma_load(global_ptr<const uint16_t> kc, global_ptr<const uint16_t> vt, int t0,
                                               int capacity, int r, int grp, u32x4 (&kr)[HD / 32],
                                               u32x2 (&vr)[HD / 16]) {
    // capacity is a multiple of 16, so a clamped tile start keeps all 16 keys in bounds
    const int tl = min(t0, capacity - kAttnRows);
    global_ptr<const uint16_t> krow = kc + static_cast<size_t>(tl + r) * HD + 8 * grp;
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) kr[s] = *(global_ptr<const u32x4>) (krow + 32 * s);
    // the tile's V block (HD dims x 16 positions, 4 KB at HD 128) is contiguous
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) {
        vr[d] = *(global_ptr<const u32x2>) (vt + static_cast<size_t>(tl) * HD + (16 * d + r) * 16 + 4 * grp);
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void k_attention_mfma(const float* __restrict__ q,
                                                                 const StepDev* __restrict__ step, int32_t layer,
                                                                 int32_t n_head, int32_t n_head_kv,
                                                                 int32_t splits_max, int32_t qgroups, int32_t slots,
                                                                 int32_t spw, float* __restrict__ partial) {
    constexpr int W = kAttnThreads / kWave, KS = HD / 32, DB = HD / 16, R = kAttnRows;
    __shared__ float Ms[W][R], Ls[W][R];
    __shared__ float Os[W][HD][R];
    const int seq = blockIdx.z;
    // the sequence's fields are read together with n_seq (seq < gridDim.z <= kMaxSeq keeps the
    // read inside the descriptor), not after the check
    const int32_t pos0 = step->seqs[seq].pos0, len = step->seqs[seq].len, row0 = step->seqs[seq].row0;
    const int32_t capacity = step->seqs[seq].capacity;
    if (seq >= step->n_seq) return;
    const int G = n_head / n_head_kv, NQ = G * len, H = n_head * HD;
    const int kvh = blockIdx.y / qgroups, qg = blockIdx.y % qgroups;
    const int q_begin = qg * R;
    if (q_begin >= NQ) return;
    const int n_keys = pos0 + len;
    const int L = attn_split_len(n_keys, len, splits_max);
    const int n_splits = (n_keys + L - 1) / L;
    // the work-group's splits [s_first, s_end) of the slots; those past the sequence's last key are marked empty
    const int s_first = blockIdx.x * spw, s_end = min(s_first + spw, slots);
    for (int sp = max(s_first, n_splits); sp < s_end; ++sp) {
        attn_empty_split<kAttnThreads>(partial, q_begin, min(R, NQ - q_begin), G, kvh, row0, n_head, HD, splits_max,
                                       sp);
    }
    const int s_stop = min(s_end, n_splits);
    if (s_first >= s_stop) return;
    int split = s_first;
    int k0 = split * L, k1 = min(n_keys, k0 + L);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r = lane & (R - 1), grp = lane >> 4;
    const size_t head_base = static_cast<size_t>(layer) * n_head_kv + kvh;
    global_ptr<const uint16_t> kc =
        as_global(static_cast<const uint16_t*>(step->seqs[seq].k)) + head_base * capacity * HD;
    global_ptr<const uint16_t> vt =
        as_global(static_cast<const uint16_t*>(step->seqs[seq].v)) + head_base * HD * capacity;

    // the wave's first tile is requested before the queries
    int t0 = k0 + R * wave;
    u32x4 kr[KS];
    u32x2 vr[DB];
    attn_mfma_load<HD>(kc, vt, t0, capacity, r, grp, kr, vr);

    // B operand of S^T: the lane's row r, dims 32 s + 8 grp .. + 7, as f16 hi + lo
    const int qi = min(q_begin + r, NQ - 1);
    const bool row_ok = q_begin + r < NQ;
    const int tr = qi / G, head = kvh * G + qi % G;
    const int limit = pos0 + tr;  // last visible key of the row (causal)
    const float* qrow = q + static_cast<size_t>(row0 + tr) * H + head * HD + 8 * grp;
    const float scale = 1.0F / sqrtf(static_cast<float>(HD));
    h8 qhi[KS], qlo[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * s);
        const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * s + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = row_ok ? x[j] * scale : 0.0F;
            qhi[s][j] = static_cast<_Float16>(v);
            qlo[s][j] = static_cast<_Float16>(v - static_cast<float>(qhi[s][j]));
        }
    }

    float m, l;
    f32x4 o[DB];
    // one 16-key tile of the wave at t0 from kr / vr
    auto tile = [&](int t0) {
        f32x4 sc = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const h8 ka = __builtin_bit_cast(h8, kr[s]);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[s], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[s], sc, 0, 0, 0);
        }
        // the lane's keys t0 + 4 grp + j for row r
        float sv[4], tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = t0 + 4 * grp + j;
            const bool vis = row_ok && key < k1 && key <= limit;
            sv[j] = vis ? sc[j] : -INFINITY;
            tmax = fmaxf(tmax, sv[j]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m, tmax);
        float alpha = 1.0F, p[4] = {0.0F, 0.0F, 0.0F, 0.0F};
        if (m_new != -INFINITY) {
            alpha = m == -INFINITY ? 0.0F : expf(m - m_new);
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = sv[j] == -INFINITY ? 0.0F : expf(sv[j] - m_new);
        }
        l = l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        m = m_new;
        h4 phi, plo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            phi[j] = static_cast<_Float16>(p[j]);
            plo[j] = static_cast<_Float16>(p[j] - static_cast<float>(phi[j]));
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const h4 va = __builtin_bit_cast(h4, vr[d]);
            o[d] *= alpha;
            o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, phi, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, plo, o[d], 0, 0, 0);
        }
    };
    const int nq = min(R, NQ - q_begin);
    // The splits of the work-group one after another, each with its own
    // (max, sum, output) state and partial: a wave keeps its next tile in
    // flight, across a split boundary too (the next split's first tile is
    // requested before the current split's last tile and its merge).
    for (;;) {
        m = -INFINITY;
        l = 0.0F;
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d] = f32x4{0.0F, 0.0F, 0.0F, 0.0F};
        u32x4 krn[KS];
        u32x2 vrn[DB];
        for (; t0 + W * R < k1; t0 += W * R) {
            attn_mfma_load<HD>(kc, vt, t0 + W * R, capacity, r, grp, krn, vrn);
            tile(t0);
#pragma unroll
            for (int s = 0; s < KS; ++s) kr[s] = krn[s];
#pragma unroll
            for (int d = 0; d < DB; ++d) vr[d] = vrn[d];
        }
        const bool more = split + 1 < s_stop;
        const int t_next = (split + 1) * L + R * wave;
        if (more) attn_mfma_load<HD>(kc, vt, t_next, capacity, r, grp, krn, vrn);
        if (t0 < k1) tile(t0);
        // the row's sum over its four lanes, then the waves merged in LDS
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (grp == 0) {
            Ms[wave][r] = m;
            Ls[wave][r] = l;
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
            for (int j = 0; j < 4; ++j) Os[wave][16 * d + 4 * grp + j][r] = o[d][j];
        }
        __syncthreads();
        for (int e = threadIdx.x; e < nq * HD; e += kAttnThreads) {
            const int i = e / HD, dim = e - i * HD;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < W; ++w) M = fmaxf(M, Ms[w][i]);
            float Lsum = 0.0F, acc = 0.0F;
            if (M != -INFINITY) {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const float f = Ms[w][i] == -INFINITY ? 0.0F : expf(Ms[w][i] - M);
                    Lsum += f * Ls[w][i];
                    acc += f * Os[w][dim][i];
                }
            }
            const int qrow_i = q_begin + i;
            const int t = qrow_i / G, hh = kvh * G + qrow_i % G;
            float* dst = partial + ((static_cast<size_t>(row0 + t) * n_head + hh) * splits_max + split) * (HD + 2);
            if (dim == 0) {
                dst[0] = M;
                dst[1] = Lsum;
            }
            dst[2 + dim] = acc;
        }
        if (!more) break;
        __syncthreads();  // the merge above has read the waves' states before the next split overwrites them
        ++split;
        k0 = split * L;
        k1 = min(n_keys, k0 + L);
        t0 = t_next;
#pragma unroll
        for (int s = 0; s < KS; ++s) kr[s] = krn[s];
#pragma unroll
        for (int d = 0; d < DB; ++d) vr[d] = vrn[d];
    }
}

// Combines the split partials of every (row, head): one work-group per
// (row, 256 output values); with xq set the 256 values are quantized into xq.
// Every split slot below n_slots (the attention grid's splits) holds this
// step's maximum (-inf for a split past the sequence's last key), so the
// partials are requested at the kernel's start, with no lookup of the step
// descriptor before them; a split whose maximum is -inf adds exactly zero, as
// it did when the merge skipped the splits past the last one.
template <int MAXS>
__global__ __launch_bounds__(256) void k_attention_merge(const float* __restrict__ partial, int32_t n_head,
                                                         int32_t hd, int32_t splits_max, int32_t n_slots,
                                                         float* __restrict__ out, Act8 xq) {
    __shared__ float vals[256];
    const int row = blockIdx.y, H = n_head * hd;
    const int c = blockIdx.x * 256 + threadIdx.x;
    float v = 0.0F;
    if (c < H) {
        const int head = c / hd, dcol = c - head * hd;
        const float* base = partial + (static_cast<size_t>(row) * n_head + head) * splits_max * (hd + 2);
        // every split's (max, sum, value) requested at once
        float pm[MAXS], pl[MAXS], po[MAXS];
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp) {
            const float* p = base + min(sp, n_slots - 1) * (hd + 2);
            const float2 ml = *reinterpret_cast<const float2*>(p);  // hd + 2 is even: 8-byte aligned
            pm[sp] = ml.x;
            pl[sp] = ml.y;
            po[sp] = p[2 + dcol];
        }
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp) {
            if (sp >= n_slots) pm[sp] = -INFINITY;
        }
        float M = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp) M = fmaxf(M, pm[sp]);
        float total = 0.0F, acc = 0.0F;
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp) {
            const float f = pm[sp] == -INFINITY ? 0.0F : expf(pm[sp] - M);
            // a split with maximum -inf adds nothing (its sum and output may be stale)
            total += pm[sp] == -INFINITY ? 0.0F : f * pl[sp];
            acc += pm[sp] == -INFINITY ? 0.0F : f * po[sp];
        }
        v = acc / total;
        out[static_cast<size_t>(row) * H + c] = v;
    }
    if (xq.q == nullptr) return;
    vals[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        const float4 v4 = *reinterpret_cast<const float4*>(&vals[4 * lane]);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
        int8_t* q = xq.q + static_cast<size_t>(row) * xq.K + blockIdx.x * 256;
        int16_t* s = xq.s + static_cast<size_t>(row) * (xq.K / 16) + blockIdx.x * 16;
        if (xq.blk == kActBlock32) {
            quant_block_wave32<false>(vv, lane, q, xq.d + static_cast<size_t>(row) * (xq.K / 32) + 8 * blockIdx.x, s);
        } else {
            quant_block_wave(vv, lane, q, xq.d + static_cast<size_t>(row) * (xq.K / 256) + blockIdx.x, s);
        }
    }
}

// ------------------------------------------------------------------ argmax + acceptance
// Greedy ids of the logits rows (first maximum, qwen2_architecture.cpp:594) and,
// per sequence, the accepted draft prefix: rows are compared in order with the
// next input token until the first mismatch (generation_runner.cpp:512-517).
// The argmax slots are cleared for the next step (stages without an
// embedding kernel rely on it).
__global__ void k_finish(unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out) {
    __shared__ int32_t tok[kMaxRows];
    for (int i = threadIdx.x; i < n_out; i += blockDim.x) {
        const unsigned long long b = best[i];
        const uint32_t low = static_cast<uint32_t>(b & 0xFFFFFFFFull);
        tok[i] = b == 0ull ? -1 : static_cast<int32_t>(0xFFFFFFFFu - low);
        out->token[i] = tok[i];
        best[i] = 0ull;
    }
    __syncthreads();
    // A draft token is accepted while the greedy id after the previous row
    // equals it and is no end-of-generation id
    // (runtime/pipeline_parallel/generation_runner.cpp:512-517).
    const int n_end = step->n_end;
    for (int s = threadIdx.x; s < step->n_seq; s += blockDim.x) {
        int accepted = 0;
        bool open = true;
        for (int i = 0; i < n_out; ++i) {
            const int r = step->out_row[i];
            if (step->seq[r] != s || !open) continue;
            bool end = false;
            for (int e = 0; e < n_end; ++e) end |= tok[i] == step->end_token[e];
            if (step->draft[i] >= 0 && tok[i] == step->draft[i] && !end) ++accepted;
            else open = false;
        }
        out->accepted[s] = accepted;
    }
}

// ------------------------------------------------------------------ static scratch
// Staging of the allocation-free matmul (int8 activation rows, the device
// matrix's full output rows). Kernels reach it only through the per-device
// address that scratch_setup looks up.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

__global__ __launch_bounds__(256) void k_gather_rows(const float* __restrict__ full, int32_t full_stride,
                                                     float* __restrict__ y, int32_t rows, int32_t offset, int32_t kind,
                                                     int32_t head_dim) {
    const int t = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    int dr = offset + r;
    if (kind == 1) {
        const int head = r / head_dim, i = r - head * head_dim, half = head_dim / 2;
        dr = offset + head * head_dim + (i < half ? 2 * i : 2 * (i - half) + 1);
    } else if (kind == 2 || kind == 3) {
        dr = (r / kGluGroup) * 2 * kGluGroup + (kind == 3 ? kGluGroup : 0) + r % kGluGroup;
    }
    y[static_cast<size_t>(t) * rows + r] = full[static_cast<size_t>(t) * full_stride + dr];
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

std::mutex g_scratch_table;
void* g_scratch_address[kScratchDevices] = {};
std::mutex g_scratch_use[kScratchDevices];

// Events of the launch being timed (set_launch_events). The first launch
// records `start` when its dispatch begins; every launch records `stop` when
// it ends, so a launcher that issues several kernels is timed from the first
// dispatch to the last.
thread_local hipEvent_t t_start = nullptr;
thread_local hipEvent_t t_stop = nullptr;

template <typename... KArgs, typename... Args>
void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    if (t_stop != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, t_start, t_stop, 0u,
                              static_cast<KArgs>(args)...);
        t_start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, static_cast<KArgs>(args)...);
    }
}

// Host-side geometry. Rows are staged in one pass or in passes of kMmChunk
// values (longer balanced passes for a grid of one work-group per CU, when
// they fit the LDS); either way every row's partial sums are added in the same order
// for 1 and for 8 tokens, so a draft-verify step reproduces serial decode bit
// for bit. The per-wave row partials take at most kMmPartBytes of LDS, and
// the row groups per work-group follow from kMmTargetWgs (mm_geom).
constexpr int kMmChunk = 8192;
constexpr int kMmPartBytes = 65536;
constexpr int kMmTargetWgs = 256;
constexpr size_t kMmOnePassLds = 64 * 1024;  // largest one-pass staging of a row that is not normalized
constexpr size_t kMmMaxLds = 160 * 1024;

// LDS of k_mm: staging of n rows (db activation scales per 256 values), row
// partials and epilogue values of nt token slots
// ps: running sums per lane of a several-pass matmul (nt; 4 for the folded Q2_K tile).
size_t mm_lds_bytes(int nt, int ps, int n, int chunk, int rgw, int K, int db) {
    const size_t nbc = static_cast<size_t>(chunk) / 256;
    // one pass: combined lane groups, nt sums per row; several: ps per lane (see k_mm)
    const size_t part = chunk >= K ? 16 * static_cast<size_t>(nt) : 64 * static_cast<size_t>(ps);
    return static_cast<size_t>(n) * chunk + (n * nbc * db + 3) / 4 * 16 + static_cast<size_t>(n) * chunk / 8 +
           static_cast<size_t>(rgw) * kMmWaves * part * 4 + n * nbc * 4 +
           static_cast<size_t>(rgw) * 16 * nt * 4 + 16 + 64;  // + the aligned zero bytes
}

MmGeom mm_geom(const GemvArgs& a, int nt, size_t& lds, bool a32) {
    static_assert(kMmChunk % (256 * kMmWaves) == 0, "a chunk must hold whole rounds of the waves' tiles");
    const int K = static_cast<int>(a.mat.cols);
    const int n_rg = (static_cast<int>(a.mat.rows) + 15) / 16;
    const int db = a32 ? 8 : 1;
    // Up to 2 x kMmTargetWgs row groups: one work-group per CU (a few CUs
    // with two work-groups would set the kernel's time); larger matrices: two
    // work-groups per CU.
    const int wgs = n_rg <= 2 * kMmTargetWgs ? kMmTargetWgs : 2 * kMmTargetWgs;
    const int want = (n_rg + wgs - 1) / wgs;
    // running sums per lane of several passes: four on the folded Q2_K tile (int8 or normalized token groups)
    const bool fold = a.mat.type == 9 && (a.xq.q != nullptr || a.x.gain != nullptr) && nt % 4 == 0;
    const int ps = fold ? 4 : nt;
    // row groups per work-group within kMmPartBytes of row partials
    auto rgw_for = [&](int chunk) {
        const int cap = kMmPartBytes / (kMmWaves * (chunk >= K ? 16 * nt : 64 * ps) * 4);
        return std::max(1, std::min(want, cap));
    };
    // The whole row is staged in one pass when it fits (a normalized input
    // always is: its block scales need the full row's rms), else in passes of
    // kMmChunk values. Wave w takes tiles w, w + W, ... of the row either way
    // and adds them in increasing order, so the pass length does not change
    // any sum.
    const bool normed = a.xq.q == nullptr && a.x.gain != nullptr;
    const int n = a.n_tok;
    int chunk = K;
    int rgw = rgw_for(chunk);
    // A grid of at most one work-group per CU may use the whole LDS for one pass.
    const size_t one_pass = (n_rg + rgw - 1) / rgw <= kMmTargetWgs ? kMmMaxLds : kMmOnePassLds;
    if (!normed && K > kMmChunk && mm_lds_bytes(nt, ps, n, K, rgw, K, db) > one_pass) {
        chunk = kMmChunk;
        // One work-group per CU: fewer, longer passes when they fit the LDS
        // (the passes balanced, in whole rounds of the waves' tiles).
        if ((n_rg + rgw_for(chunk) - 1) / rgw_for(chunk) <= kMmTargetWgs) {
            const int round = 256 * kMmWaves;
            for (int passes = 2; passes * kMmChunk < K; ++passes) {
                const int c = ((K + passes - 1) / passes + round - 1) / round * round;
                if (mm_lds_bytes(nt, ps, n, c, rgw_for(c), K, db) <= kMmMaxLds) {
                    chunk = c;
                    break;
                }
            }
        }
    }
    rgw = rgw_for(chunk);
    if (!normed && mm_lds_bytes(nt, ps, n, chunk, rgw, K, db) > kMmMaxLds) {
        // wide token groups: shorter passes, in whole rounds of the waves' tiles, until the staging fits
        const int round = 256 * kMmWaves;
        chunk = std::min(chunk, kMmChunk) / round * round;
        rgw = rgw_for(chunk);
        while (chunk > round && mm_lds_bytes(nt, ps, n, chunk, rgw, K, db) > kMmMaxLds) chunk -= round;
    }
    if (nt <= 2 && chunk < K) throw std::invalid_argument("one- and two-token matmul rows must fit one pass");
    MmGeom g;
    g.rgw = rgw;
    g.chunk = chunk;
    lds = mm_lds_bytes(nt, ps, n, chunk, rgw, K, db);
    if (lds > kMmMaxLds) throw std::invalid_argument("matmul staging does not fit the LDS");
    return g;
}

// Whether the activations of a matmul come in (or are staged in) 32-value
// blocks: Q8_0 matrices take nothing else, the K-quants 256-value blocks.
bool mm_a32(const GemvArgs& a) {
    const bool a32 = a.xq.q != nullptr ? a.xq.blk == kActBlock32 : a.ablk == kActBlock32;
    if (a32 != (a.mat.type == 7)) {
        throw std::invalid_argument("activation block does not fit the weight type (Q8_0: 32 values, K-quants: 256)");
    }
    return a32;
}

template <uint32_t TYPE, int NT>
void mm(const GemvArgs& a, hipStream_t stream) {
    const bool a32 = mm_a32(a);
    size_t lds = 0;
    const MmGeom g = mm_geom(a, NT, lds, a32);
    const int n_rg = (static_cast<int>(a.mat.rows) + 15) / 16;
    const int grid = (n_rg + g.rgw - 1) / g.rgw;
    const dim3 gd(grid), bd(kMmThreads);
    if constexpr (TYPE == 7) {
        if (a.xq.q != nullptr) launch(k_mm<TYPE, NT, kInAct8, true>, gd, bd, lds, stream, a, g);
        else if (a.x.gain != nullptr) launch(k_mm<TYPE, NT, kInNormed, true>, gd, bd, lds, stream, a, g);
        else launch(k_mm<TYPE, NT, kInFloat, true>, gd, bd, lds, stream, a, g);
    } else {
        if (a.xq.q != nullptr) launch(k_mm<TYPE, NT, kInAct8, false>, gd, bd, lds, stream, a, g);
        else if (a.x.gain != nullptr) launch(k_mm<TYPE, NT, kInNormed, false>, gd, bd, lds, stream, a, g);
        else launch(k_mm<TYPE, NT, kInFloat, false>, gd, bd, lds, stream, a, g);
    }
    check(hipGetLastError(), "matmul launch");
}

template <uint32_t TYPE>
void mm_nt(const GemvArgs& a, hipStream_t stream) {
    if constexpr (kHasQuads<TYPE>) {
        // int8 or normalized rows from kQuadMinRows tokens on: token quads on matrix cores
        if ((a.xq.q != nullptr || a.x.gain != nullptr) && a.n_tok >= kQuadMinRows) {
            if (a.n_tok <= 4) mm<TYPE, 4>(a, stream);
            else if (a.n_tok <= 8) mm<TYPE, 8>(a, stream);
            else mm<TYPE, kQuadGroupRows>(a, stream);
            return;
        }
    }
    switch (a.n_tok) {
    case 1: mm<TYPE, 1>(a, stream); break;
    case 2: mm<TYPE, 2>(a, stream); break;
    case 3: case 4: mm<TYPE, 4>(a, stream); break;
    case 5: case 6: mm<TYPE, 6>(a, stream); break;
    case 7: case 8: mm<TYPE, 8>(a, stream); break;
    default: throw std::invalid_argument("matmul token group must be 1..8");
    }
}

template <int NT>
void gemv_f(const GemvArgs& a, hipStream_t stream) {
    const int grid = (static_cast<int>(a.mat.rows) + kGemvFloatRows - 1) / kGemvFloatRows;
    const size_t lds = static_cast<size_t>(kGemvFloatRows) * NT * sizeof(float);
    launch(k_gemv_f<NT>, dim3(grid), dim3(kFloatThreads), lds, stream, a, kGemvFloatRows);
    check(hipGetLastError(), "gemv launch");
}

}  // namespace

void scratch_setup(int device) {
    if (device < 0 || device >= kScratchDevices) throw std::invalid_argument("device ordinal outside the scratch table");
    std::lock_guard lock(g_scratch_table);
    if (g_scratch_address[device] != nullptr) return;
    void* p = nullptr;
    check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch symbol address");
    if (p == nullptr) throw std::runtime_error("scratch symbol address is null");
    g_scratch_address[device] = p;
}

void* scratch_address(int device) {
    if (device < 0 || device >= kScratchDevices) return nullptr;
    std::lock_guard lock(g_scratch_table);
    return g_scratch_address[device];
}

std::mutex& scratch_lock(int device) {
    if (device < 0 || device >= kScratchDevices) throw std::invalid_argument("device ordinal outside the scratch table");
    return g_scratch_use[device];
}

void launch_gather_rows(const float* full, int32_t full_stride, float* y, int32_t rows, int32_t n_tok, int32_t offset,
                        int32_t kind, int32_t head_dim, hipStream_t stream) {
    if (rows <= 0 || n_tok <= 0 || (kind == 1 && (head_dim <= 0 || head_dim % 2 != 0))) {
        throw std::invalid_argument("row gather shape is invalid");
    }
    launch(k_gather_rows, dim3((rows + 255) / 256, n_tok), dim3(256), 0, stream, full, full_stride, y, rows, offset,
           kind, head_dim);
    check(hipGetLastError(), "row gather launch");
}

void set_launch_events(hipEvent_t start, hipEvent_t stop) {
    t_start = start;
    t_stop = stop;
}

float dequant_tile_value(uint32_t type, const uint8_t* tile, uint32_t row, uint32_t k) {
    return tile_value(type, tile, row, k);
}

void launch_gemv(const GemvArgs& a_in, hipStream_t stream) {
    const uint32_t type = a_in.mat.type;
    const bool quantized = tile_bytes(type) != 0;
    if (quantized && (a_in.mat.cols % kActBlock != 0 || (a_in.xq.q == nullptr && a_in.x.stride % 4 != 0))) {
        throw std::invalid_argument("quantized matmul needs rows of a multiple of 256 values");
    }
    if (!quantized && a_in.xq.q != nullptr) throw std::invalid_argument("float matmuls take float activations");
    if (a_in.xq.q != nullptr && (a_in.xq.K != static_cast<int32_t>(a_in.mat.cols) || a_in.x.gain != nullptr)) {
        throw std::invalid_argument("pre-quantized activations must match the matrix and carry no norm");
    }
    if ((a_in.mode == kSwiGLU && a_in.mat.rows % (2 * kGluGroup) != 0) || (a_in.mode == kQKV && a_in.mat.rows % 2 != 0)) {
        throw std::invalid_argument("matmul rows do not fit the fused row layout");
    }
    // token groups of at most 8 rows; int8 or normalized rows of the quantized
    // formats run on matrix cores in groups of up to kQuadGroupRows
    const bool quads = quantized && (a_in.xq.q != nullptr || a_in.x.gain != nullptr) && a_in.n_tok >= kQuadMinRows;
    const int group = quads ? kQuadGroupRows : 8;
    for (int t0 = 0; t0 < a_in.n_tok; t0 += group) {
        GemvArgs a = a_in;
        a.n_tok = a_in.n_tok - t0 < group ? a_in.n_tok - t0 : group;
        if (a.xq.q) {
            a.xq.q += static_cast<size_t>(t0) * a.xq.K;
            a.xq.d += static_cast<size_t>(t0) * (a.xq.K / a.xq.blk);
            a.xq.s += static_cast<size_t>(t0) * (a.xq.K / 16);
        } else if (a.x.gather) {
            a.x.gather += t0;
        } else {
            a.x.x += static_cast<size_t>(t0) * a.x.stride;
        }
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
        case 11: mm_nt<11>(a, stream); break;
        case 13: mm_nt<13>(a, stream); break;
        case 9: mm_nt<9>(a, stream); break;
        case 7: mm_nt<7>(a, stream); break;
        default: throw std::invalid_argument("unsupported weight type for gemv");
        }
    }
}

void launch_quantize(const float* x, int32_t stride, int32_t n_rows, const Act8& out, hipStream_t stream) {
    if (out.K % 256 != 0 || stride % 4 != 0) throw std::invalid_argument("quantized rows need multiples of 256 values");
    if (out.blk != kActBlock && out.blk != kActBlock32) throw std::invalid_argument("activation blocks are 256 or 32 values");
    dim3 grid((out.K / 256 + 3) / 4, n_rows);
    launch(k_quantize, grid, dim3(256), 0, stream, x, stride, out);
    check(hipGetLastError(), "quantize launch");
}

void launch_quantize_norm(const float* x, int32_t stride, const int32_t* gather, const float* gain, float eps,
                          int32_t n_rows, const Act8& out, hipStream_t stream) {
    if (out.K % 256 != 0 || out.K / 256 > kNormMaxBlocks || stride % 4 != 0 || gain == nullptr ||
        (out.blk != kActBlock && out.blk != kActBlock32)) {
        throw std::invalid_argument("normalized quantization needs rows of a multiple of 256 values and a gain");
    }
    launch(k_quantize_norm, dim3(n_rows), dim3(kNormThreads), 0, stream, x, stride, gather, gain, eps, out);
    check(hipGetLastError(), "normalized quantize launch");
}

constexpr int kWideMinWgs = 512;
constexpr int kWideRgMinWgs = 256;  // one work-group per CU
constexpr int kWideLogitsWgs = 1024;
constexpr int kWideQ4kWaves = 4;
constexpr int kWideQ4kMinWgs = 256;

bool wide_matmul_supported(uint32_t type) { return type == 7 || type == 9 || type == 11 || type == 13; }

// Measured on 7B-shaped layers: Q4_K and Q8_0 from 9 rows; Q6_K and Q2_K,
// whose 16-value sub-blocks take two half-masked MFMAs per 32 values, only
// beyond one 16-slot token-quad group.
constexpr int32_t kWideFromRows = 9;
int32_t wide_min_rows(uint32_t type) {
    switch (type) {
    case 7:
    case 11: return kWideFromRows;
    case 9:
    case 13: return kQuadGroupRows + 1;
    default: return 0;
    }
}

void launch_gemv_wide(const GemvArgs& a_in, hipStream_t stream) {
    if (!wide_matmul_supported(a_in.mat.type) || a_in.xq.q == nullptr || a_in.xq.K != static_cast<int32_t>(a_in.mat.cols) ||
        a_in.mat.cols % kActBlock != 0 || a_in.n_tok < 1 || a_in.n_tok > kWideRows) {
        throw std::invalid_argument("wide matmul takes Q4_K / Q6_K / Q8_0 / Q2_K weights and up to kWideRows pre-quantized token rows");
    }
    if ((a_in.mode == kSwiGLU && a_in.mat.rows % (2 * kGluGroup) != 0) || (a_in.mode == kQKV && a_in.mat.rows % 2 != 0) ||
        (a_in.mode == kLogits && a_in.best == nullptr)) {
        throw std::invalid_argument("wide matmul mode or row layout not supported");
    }
    mm_a32(a_in);  // validates the activation block for the weight type
    const GemvArgs& a = a_in;
    const int n_rg = (static_cast<int>(a.mat.rows) + 15) / 16, n_tt = (a.n_tok + 15) / 16;
    // as many token tiles per work-group as still leave kWideMinWgs work-groups
    int tpw = min(n_tt, kWideTpw);
    while (tpw > 1 && n_rg * ((n_tt + tpw - 1) / tpw) < kWideMinWgs) --tpw;
    const bool merged = a.mode == kLogits;  // the head kernel: the only one with the argmax epilogue
    if (a.mat.type == 11 && !merged) {
        // Q4_K matrices with many row groups: whole-K waves over all of the
        // step's token tiles, while that still leaves kWideQ4kMinWgs work-groups
        const int n_sets = (n_rg + kWideQ4kWaves - 1) / kWideQ4kWaves;
        if (n_sets >= kWideQ4kMinWgs) {
            // up to four token tiles per work-group; longer steps run as several token groups
            const int tpw4 = min(n_tt, 4), n_grp4 = (n_tt + tpw4 - 1) / tpw4;
            const dim3 g((n_sets + 7) / 8 * 8 * n_grp4), b(kWideQ4kWaves * kWave);
            if (tpw4 > 2) launch(k_mm_wide_q4k<kWideQ4kWaves, 4>, g, b, 0, stream, a, n_rg, tpw4);
            else if (tpw4 == 2) launch(k_mm_wide_q4k<kWideQ4kWaves, 2>, g, b, 0, stream, a, n_rg, tpw4);
            else launch(k_mm_wide_q4k<kWideQ4kWaves, 1>, g, b, 0, stream, a, n_rg, tpw4);
            check(hipGetLastError(), "wide matmul launch");
            return;
        }
        // fewer row groups: two row groups and one token tile per work-group, the decode
        // waves' K split, while one work-group per CU remains
        if ((n_rg + 1) / 2 * n_tt >= kWideRgMinWgs) {
            const dim3 g(((n_rg + 1) / 2 + 7) / 8 * 8 * n_tt), b(kMmThreads);
            launch(k_mm_wide_q4r<2>, g, b, 0, stream, a, n_rg);
            check(hipGetLastError(), "wide matmul launch");
            return;
        }
    }
    // K-quant layer matrices: one token tile and several row groups per work-group, every
    // activation load shared by the row groups: four (Q4_K only: the other formats'
    // operands take the registers) while kWideMinWgs work-groups remain, else two while
    // one work-group per CU remains (Q6_K and Q2_K matrices, and Q4_K ones too small for
    // the folded-scale kernels above)
    int rgs = 1;
    if (!merged && a.mat.type != 7) {
        if (a.mat.type == 11 && (n_rg + 3) / 4 * n_tt >= kWideMinWgs) rgs = 4;
        else if ((n_rg + 1) / 2 * n_tt >= kWideRgMinWgs) rgs = 2;
    }
    if (rgs > 1) {
        const int tp1 = 1;
        const dim3 g(((n_rg + rgs - 1) / rgs + 7) / 8 * 8 * n_tt), b(kMmThreads);
        switch (a.mat.type * 8 + rgs) {
        case 11 * 8 + 4: launch(k_mm_wide_rg<11, 4, 1, false>, g, b, 0, stream, a, n_rg, tp1); break;
        case 11 * 8 + 2: launch(k_mm_wide_rg<11, 2, 1, false>, g, b, 0, stream, a, n_rg, tp1); break;
        case 13 * 8 + 2: launch(k_mm_wide_rg<13, 2, 1, false>, g, b, 0, stream, a, n_rg, tp1); break;
        default: launch(k_mm_wide_rg<9, 2, 1, false>, g, b, 0, stream, a, n_rg, tp1); break;
        }
        check(hipGetLastError(), "wide matmul launch");
        return;
    }
    // the head: row groups per work-group so that about kWideLogitsWgs work-groups merge their argmax
    const int rpw = a.mode == kLogits ? std::max(1, n_rg / kWideLogitsWgs) : 1;
    const int grid = (n_rg + 8 * rpw - 1) / (8 * rpw) * 8 * ((n_tt + tpw - 1) / tpw);
    const dim3 g(grid), b(kMmThreads);
    auto go = [&](auto kernel) { launch(kernel, g, b, 0, stream, a, n_rg, tpw, rpw); };
    switch (a.mat.type) {
    case 7:
        if (merged) go(k_mm_wide<7, true, true>);
        else go(k_mm_wide<7, false, true>);
        break;
    case 9:
        if (merged) go(k_mm_wide<9, true, false>);
        else go(k_mm_wide<9, false, false>);
        break;
    case 11:
        if (merged) go(k_mm_wide<11, true, false>);
        else go(k_mm_wide<11, false, false>);
        break;
    default:
        if (merged) go(k_mm_wide<13, true, false>);
        else go(k_mm_wide<13, false, false>);
        break;
    }
    check(hipGetLastError(), "wide matmul launch");
}

void launch_embed(const DMat& table, const StepDev* step, float* h, int32_t n_rows, int32_t H,
                  unsigned long long* best, int32_t n_best, hipStream_t stream) {
    dim3 grid((H + 255) / 256, n_rows);
    launch(k_embed, grid, dim3(256), 0, stream, table, step, h, H, best, n_best);
    check(hipGetLastError(), "embed launch");
}

int32_t attention_max_rows(int32_t head_dim) {
    // the matrix-core kernel takes any number of 16-row groups; the generic one up to kMaxAttnQGroups groups of 8
    return (head_dim == 128 || head_dim == 64) ? kMaxRows * 64 : kMaxAttnQGroups * kAttnQPW;
}

int32_t attention_splits(int32_t capacity) {
    const int32_t s = (capacity + kAttnWgKeys - 1) / kAttnWgKeys;
    return s < 1 ? 1 : (s > kAttnMaxSplits ? kAttnMaxSplits : s);
}

size_t attention_partial_floats(int32_t rows, int32_t n_head, int32_t head_dim, int32_t splits) {
    return static_cast<size_t>(rows) * n_head * splits * (head_dim + 2);
}

int32_t attention_slots(int32_t splits, int32_t capacity, int32_t n_rows, int32_t n_seq) {
    if (n_seq != 1 || n_rows <= kQuadGroupRows) return splits;
    return std::max(1, std::min(splits, (capacity + kAttnPrefillKeys - 1) / kAttnPrefillKeys));
}

void launch_attention(const float* q, const StepDev* step, int32_t max_len, int32_t n_seq, int32_t layer,
                      int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t splits, float* partial,
                      hipStream_t stream, int32_t slots) {
    if (slots <= 0) slots = splits;
    if (slots > splits) throw std::invalid_argument("attention slots exceed the split stride");
    const int G = n_head / n_head_kv;
    if (head_dim > 2 * kWave || head_dim % 4 != 0) {
        throw std::invalid_argument("attention supports head dims that are multiples of 4 up to 128");
    }
    if (n_seq < 1 || n_seq > kMaxSeq) throw std::invalid_argument("attention step needs 1..kMaxSeq sequences");
    const bool mfma = head_dim == 128 || head_dim == 64;
    const int group_rows = mfma ? kAttnRows : kAttnQPW;
    const int qgroups = (G * max_len + group_rows - 1) / group_rows;
    if (G * max_len > attention_max_rows(head_dim)) {
        throw std::invalid_argument("attention step has too many query rows per kv head");
    }
    dim3 grid(slots, n_head_kv * qgroups, n_seq), block(kAttnThreads);
    // On matrix cores a work-group of a decode or verify step walks spw
    // consecutive splits when the step's (split, kv head x query group,
    // sequence) work-groups would exceed one resident round: every split keeps
    // its own partial, so the results do not depend on spw. (Prefill chunks,
    // whose splits already hold kAttnPrefillKeys keys or more, run one split per
    // work-group: two per work-group made 64-row chunks 16 -> 20 us.)
    int spw = 1;
    if (mfma && max_len <= kQuadGroupRows) {
        const int cols = n_head_kv * qgroups * n_seq;
        spw = std::min(slots, (slots * cols + kAttnResidentWgs - 1) / kAttnResidentWgs);
        grid.x = (slots + spw - 1) / spw;
    }
    if (head_dim == 128) {
        launch(k_attention_mfma<128>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, splits, qgroups,
               slots, spw, partial);
    } else if (head_dim == 64) {
        launch(k_attention_mfma<64>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, splits, qgroups,
               slots, spw, partial);
    } else {
        launch(k_attention<0>, grid, block, 0, stream, q, step, layer, n_head, n_head_kv, head_dim, splits, qgroups,
               partial);
    }
    check(hipGetLastError(), "attention launch");
}

void launch_attention_merge(const float* partial, const StepDev* step, int32_t n_rows, int32_t n_head,
                            int32_t head_dim, int32_t splits, float* out, const Act8& xq, hipStream_t stream,
                            int32_t slots) {
    if (slots <= 0) slots = splits;
    if (slots > splits) throw std::invalid_argument("attention slots exceed the split stride");
    const int H = n_head * head_dim;
    if (xq.q != nullptr && (H % 256 != 0 || xq.K != H)) throw std::invalid_argument("merge quantization shape mismatch");
    dim3 grid((H + 255) / 256, n_rows);
    (void) step;
    // the merge requests MAXS >= slots partials per value at once (MAXS a multiple of 4)
    static_assert(kAttnMaxSplits == 32, "merge instantiations");
    switch ((slots + 3) / 4) {
    case 1: launch(k_attention_merge<4>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 2: launch(k_attention_merge<8>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 3: launch(k_attention_merge<12>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 4: launch(k_attention_merge<16>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 5: launch(k_attention_merge<20>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 6: launch(k_attention_merge<24>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    case 7: launch(k_attention_merge<28>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    default: launch(k_attention_merge<32>, grid, dim3(256), 0, stream, partial, n_head, head_dim, splits, slots, out, xq); break;
    }
    check(hipGetLastError(), "attention merge launch");
}

void launch_finish(unsigned long long* best, const StepDev* step, int32_t n_out, StepOut* out,
                   hipStream_t stream) {
    launch(k_finish, dim3(1), dim3(64), 0, stream, best, step, n_out, out);
    check(hipGetLastError(), "finish launch");
}

void launch_dequant_rows(const DMat& m, int32_t row0, int32_t n_rows, float* out, hipStream_t stream) {
    dim3 grid((m.cols + 255) / 256, n_rows);
    launch(k_dequant_rows, grid, dim3(256), 0, stream, m, row0, out);
    check(hipGetLastError(), "dequant launch");
}

}  // namespace jfh::gpu
