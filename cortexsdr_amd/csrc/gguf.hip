// gguf.hip — the GGUF block formats the reference inference engine decodes, as device
// dequant-matmuls on gfx950 (W never materialised in fp32).
//
// Reference path (cortexSDR tree): SparseInferenceEngine.cpp decodeSupportedGGUFQuantized
// (:276-469) dequantises a strategy-0 GGUF tensor to fp32 at layer load (block sizes
// ggufBlockBytesForFormat / ggufBlockElementsForFormat :181-231), then Kernels::linear_forward
// (kernels/blas_kernels.cpp:264-293) computes out (M x R) = in (M x C) . W^T. Every format is
// decoded here with the reference's own element order and arithmetic, including where they
// differ from ggml's: q4_0/q4_1/q5_0/q5_1 take element i from byte i/2 (low nibble for even i),
// q6_k uses scales[0], [2], [4], [6] of each 128-element half for its four 32-element
// quarters, q8_1 reads its scale as fp32 and q8_k as fp16 at the block start. Formats the
// reference has no exact decoder for (q2_k, q3_k, q5_k, the iq and tq families, the
// q4_0_x_y repacks) take its generic rule (:439-465): `bits` per element packed LSB-first at
// the end of the block, centred on 2^(bits-1), times the fp16 scale at the block start (1
// when that is not finite or below 1e-12). q4_k is served by q4k.hip and also here.
//
// Kernels (a template per format, so each decode is straight-line code)
//   gguf_gemv_lds_kernel (M == 1): one wave per row; the row's blocks staged in LDS with
//     coalesced loads, then lane l takes elements l, l + 64, ... of the row, decodes each from
//     its block and multiplies by x in fp32; gguf_gemv_kernel is the same from memory, for
//     the 8-bit formats and rows longer than the LDS budget.
//   gguf_mfma_kernel (M > 1, fp16 X): 16 rows per workgroup, the 4 waves stride over 16-wide k
//     steps; each lane decodes 4 consecutive values of its row in fp32, splits them into fp16
//     hi + lo and issues two v_mfma_f32_16x16x16f16 per 16 output columns (fp32 accumulate).
//   gguf_dequant_kernel: one thread per element.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <string>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h16(const uint8_t* p) {
    return csdr::h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}
__device__ __forceinline__ float nib(const uint8_t* qs, int e) {
    const uint8_t b = qs[e >> 1];
    return (float)((e & 1) ? (b >> 4) : (b & 0x0Fu));
}

// ---- one struct per format: BB bytes and BE elements per block, at(block, e) = value e
struct Q4_0 {  // :398-406
    static constexpr int BB = 18, BE = 32;
    __device__ static float at(const uint8_t* p, int e) { return (nib(p + 2, e) - 8.0f) * h16(p); }
};
struct Q4_1 {  // :408-417
    static constexpr int BB = 20, BE = 32;
    __device__ static float at(const uint8_t* p, int e) {
        return fmaf(nib(p + 4, e), h16(p), h16(p + 2));
    }
};
template <bool HAS_M>
struct Q5 {  // q5_0 / q5_1, :419-436
    static constexpr int BB = HAS_M ? 24 : 22, BE = 32;
    __device__ static float at(const uint8_t* p, int e) {
        const uint8_t* qh = p + (HAS_M ? 4 : 2);
        const uint8_t* qs = p + (HAS_M ? 8 : 6);
        const uint8_t b = qs[e >> 1];
        const uint32_t lo = (e & 1) ? (b >> 4) : (b & 0x0Fu);
        const uint32_t hi = (qh[e >> 3] >> (e & 7)) & 1u;
        const float q = (float)(lo | (hi << 4));
        return HAS_M ? fmaf(q, h16(p), h16(p + 2)) : (q - 16.0f) * h16(p);
    }
};
struct Q8_0 {  // :310-316
    static constexpr int BB = 34, BE = 32;
    __device__ static float at(const uint8_t* p, int e) {
        return (float)(int8_t)p[2 + e] * h16(p);
    }
};
struct Q8_1 {  // :319-326: the scale is read as fp32
    static constexpr int BB = 40, BE = 32;
    __device__ static float at(const uint8_t* p, int e) {
        const uint32_t u = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                           ((uint32_t)p[3] << 24);
        return (float)(int8_t)p[8 + e] * __builtin_bit_cast(float, u);
    }
};
struct Q8_K {  // :387-395: fp16 scale, quants at +4
    static constexpr int BB = 292, BE = 256;
    __device__ static float at(const uint8_t* p, int e) {
        return (float)(int8_t)p[4 + e] * h16(p);
    }
};
struct Q6_K {  // :329-359
    static constexpr int BB = 210, BE = 256;
    __device__ static float at(const uint8_t* p, int e) {
        const int half = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
        const uint8_t* ql = p + half * 64;
        const uint8_t qh = p[128 + half * 32 + l];
        const uint8_t lb = ql[l + ((t & 1) ? 32 : 0)];
        const int lo = (t < 2) ? (lb & 0x0F) : (lb >> 4);
        const int q = (lo | (((qh >> (2 * t)) & 3) << 4)) - 32;
        const int sc = (int)(int8_t)p[192 + half * 8 + 2 * t];
        return h16(p + 208) * (float)(sc * q);
    }
};
struct Q4_K {  // :362-384 (ggml order; see q4k.hip)
    static constexpr int BB = 144, BE = 256;
    __device__ static float at(const uint8_t* p, int e) {
        const int sb = e >> 5;
        const uint8_t* s12 = p + 4;
        uint32_t sc, mn;
        if (sb < 4) {
            sc = s12[sb] & 63u;
            mn = s12[sb + 4] & 63u;
        } else {
            sc = (s12[sb + 4] & 0xFu) | ((s12[sb - 4] >> 6) << 4);
            mn = (s12[sb + 4] >> 4) | ((s12[sb] >> 6) << 4);
        }
        const uint8_t b = p[16 + (sb >> 1) * 32 + (e & 31)];
        const float q = (float)((sb & 1) ? (b >> 4) : (b & 0xFu));
        const float d0 = h16(p) * (float)sc, m0 = h16(p + 2) * (float)mn;
        return d0 * q - m0;
    }
};
template <int BB_, int BE_, int BITS>
struct Packed {  // generic rule, :439-465
    static constexpr int BB = BB_, BE = BE_;
    static constexpr int kData = BB - (BE * BITS + 7) / 8;
    static_assert(kData >= 0, "packed data larger than the block");
    __device__ static float at(const uint8_t* p, int e) {
        float d = h16(p);
        if (!isfinite(d) || fabsf(d) < 1e-12f) d = 1.0f;
        const int bit = e * BITS, byte = kData + (bit >> 3), sh = bit & 7;
        uint32_t v = p[byte];
        if (sh + BITS > 8) v |= (uint32_t)p[byte + 1] << 8;  // (only inside the block)
        const int q = (int)((v >> sh) & ((1u << BITS) - 1u)) - (1 << (BITS - 1));
        return (float)q * d;
    }
};

// ---- kernels
template <class F, typename XT>
__global__ __launch_bounds__(kThreads) void gguf_gemv_kernel(const uint8_t* __restrict__ W,
                                                             int R, int C,
                                                             const XT* __restrict__ x,
                                                             float* __restrict__ y) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x * (kThreads / 64) + wave;
    if (r >= R) return;  // (no barriers below)
    const uint8_t* rowp = W + (size_t)r * (C / F::BE) * F::BB;
    float acc = 0.0f;
    const int nit = (C + 63) >> 6;
#pragma unroll 4
    for (int it = 0; it < nit; ++it) {
        const int e = min(it * 64 + lane, C - 1);  // unconditional loads, masked contribution
        const int b = e / F::BE;
        const float w = F::at(rowp + (size_t)b * F::BB, e - b * F::BE);
        const float xv = csdr::to_f32(x[e]);
        if (it * 64 + lane < C) acc = fmaf(w, xv, acc);
    }
    acc = csdr::wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

constexpr int kMaxNT = 4;  // 16-column tiles per workgroup (grid.y covers more columns)

template <class F>
__global__ __launch_bounds__(kThreads) void gguf_mfma_kernel(const uint8_t* __restrict__ W,
                                                             int R, int C,
                                                             const _Float16* __restrict__ X,
                                                             int M, float* __restrict__ Y) {
    __shared__ floatx4 red[3][kMaxNT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 16;
    const int n0 = blockIdx.y * 16 * kMaxNT;
    const int arow = min(r0 + (lane & 15), R - 1);  // A operand row of this lane
    const int kq = lane >> 4;                        // 4-value k quad within a 16-k step
    const uint8_t* rowp = W + (size_t)arow * (C / F::BE) * F::BB;
    floatx4 acc[kMaxNT];
#pragma unroll
    for (int t = 0; t < kMaxNT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int nt_live = min(kMaxNT, (M - n0 + 15) / 16);
    for (int k0 = wave * 16; k0 < C; k0 += (kThreads / 64) * 16) {
        const int e0 = k0 + kq * 4;
        half4 ahi, alo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = e0 + i, b = e / F::BE;
            const float wv = F::at(rowp + (size_t)b * F::BB, e - b * F::BE);
            const _Float16 h = (_Float16)wv;
            ahi[i] = h;
            alo[i] = (_Float16)(wv - (float)h);
        }
        for (int t = 0; t < nt_live; ++t) {
            const int n = n0 + t * 16 + (lane & 15);
            half4 bv = half4{0, 0, 0, 0};
            if (n < M) bv = *reinterpret_cast<const half4*>(X + (size_t)n * C + e0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ahi, bv, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(alo, bv, acc[t], 0, 0, 0);
        }
    }
    // the 4 waves' tiles: waves 1..3 park theirs in LDS, wave 0 adds and stores
    if (wave > 0)
        for (int t = 0; t < nt_live; ++t) red[wave - 1][t][lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
        for (int t = 0; t < nt_live; ++t) {
            floatx4 s = acc[t];
#pragma unroll
            for (int w = 0; w < 3; ++w) s += red[w][t][lane];
            // D[i][j] of the 16x16 tile: lane holds rows (lane/16)*4 + i, column lane%16
            const int n = n0 + t * 16 + (lane & 15);
            if (n >= M) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = r0 + (lane >> 4) * 4 + i;
                if (r < R) Y[(size_t)n * R + r] = s[i];
            }
        }
    }
}

template <class F>
__global__ __launch_bounds__(kThreads) void gguf_dequant_kernel(const uint8_t* __restrict__ W,
                                                                size_t nblocks,
                                                                float* __restrict__ out) {
    const size_t total = nblocks * F::BE;
    for (size_t g = (size_t)blockIdx.x * kThreads + threadIdx.x; g < total;
         g += (size_t)gridDim.x * kThreads) {
        const size_t b = g / F::BE;
        out[g] = F::at(W + b * F::BB, (int)(g - b * F::BE));
    }
}

// M == 1 with the row staged in LDS: each wave copies its row's blocks with coalesced dword
// loads (byte loads when the row is not 4-byte aligned), then decodes from LDS as
// gguf_gemv_kernel does from memory (the per-element header and quant bytes are LDS reads
// instead of scattered vector-memory loads).
constexpr size_t kGemvLdsMax = 64 * 1024;

// Whether a format's M == 1 product stages its rows in LDS: yes where an element's decode reads
// several scattered bytes (measured at 4096 x 4096: q5_k 36.7 -> 20.4 us, q6_k 25.8 -> 24.5,
// q4_0 16.4 -> 15.5), no for the 8-bit formats (one byte and the scale per element; q8_0
// 15.1 -> 18.0 us staged).
template <class F>
struct StageRow {
    static constexpr bool value = true;
};
template <>
struct StageRow<Q8_0> {
    static constexpr bool value = false;
};
template <>
struct StageRow<Q8_1> {
    static constexpr bool value = false;
};
template <>
struct StageRow<Q8_K> {
    static constexpr bool value = false;
};

template <class F, typename XT>
__global__ __launch_bounds__(kThreads) void gguf_gemv_lds_kernel(const uint8_t* __restrict__ W,
                                                                 int R, int C,
                                                                 const XT* __restrict__ x,
                                                                 float* __restrict__ y,
                                                                 int aligned4) {
    extern __shared__ uint8_t srow[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x * (kThreads / 64) + wave;
    const int rowbytes = (C / F::BE) * F::BB, stride = (rowbytes + 3) & ~3;
    uint8_t* my = srow + (size_t)wave * stride;
    if (r < R) {
        const uint8_t* rowp = W + (size_t)r * rowbytes;
        if (aligned4) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp);
            uint32_t* dst = reinterpret_cast<uint32_t*>(my);
            for (int i = lane; i < rowbytes / 4; i += 64) dst[i] = src[i];
        } else {
            for (int i = lane; i < rowbytes; i += 64) my[i] = rowp[i];
        }
    }
    __syncthreads();
    if (r >= R) return;  // (no barriers below)
    float acc = 0.0f;
    const int nit = (C + 63) >> 6;
#pragma unroll 4
    for (int it = 0; it < nit; ++it) {
        const int e = min(it * 64 + lane, C - 1);
        const int b = e / F::BE;
        const float w = F::at(my + (size_t)b * F::BB, e - b * F::BE);
        const float xv = csdr::to_f32(x[e]);
        if (it * 64 + lane < C) acc = fmaf(w, xv, acc);
    }
    acc = csdr::wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

// ---- format table: name, id, and the launchers of each format
struct Launch {
    int (*linear)(const uint8_t*, int, int, const void*, int, int, float*, hipStream_t);
    int (*dequant)(const uint8_t*, size_t, float*, hipStream_t);
};

template <class F>
int linear_of(const uint8_t* w, int R, int C, const void* x, int x_dtype, int M, float* y,
              hipStream_t st) {
    if (M == 1) {
        const int grid = (R + kThreads / 64 - 1) / (kThreads / 64);
        const size_t rowbytes = (size_t)(C / F::BE) * F::BB;
        const size_t lds = (kThreads / 64) * ((rowbytes + 3) & ~(size_t)3);
        if (StageRow<F>::value && lds <= kGemvLdsMax) {
            const int a4 = (rowbytes % 4 == 0 && reinterpret_cast<uintptr_t>(w) % 4 == 0);
            if (x_dtype == CSDR_F16)
                gguf_gemv_lds_kernel<F, _Float16><<<grid, kThreads, lds, st>>>(
                    w, R, C, static_cast<const _Float16*>(x), y, a4);
            else
                gguf_gemv_lds_kernel<F, float><<<grid, kThreads, lds, st>>>(
                    w, R, C, static_cast<const float*>(x), y, a4);
        } else if (x_dtype == CSDR_F16)
            gguf_gemv_kernel<F, _Float16><<<grid, kThreads, 0, st>>>(
                w, R, C, static_cast<const _Float16*>(x), y);
        else
            gguf_gemv_kernel<F, float><<<grid, kThreads, 0, st>>>(
                w, R, C, static_cast<const float*>(x), y);
    } else {
        if (x_dtype != CSDR_F16)
            return set_error(CSDR_E_UNSUPPORTED, "gguf_linear: M > 1 takes fp16 x");
        if (reinterpret_cast<uintptr_t>(x) % 8)
            return set_error(CSDR_E_INVALID, "gguf_linear: x must be 8-byte aligned");
        dim3 grid((R + 15) / 16, (M + 16 * kMaxNT - 1) / (16 * kMaxNT));
        gguf_mfma_kernel<F><<<grid, kThreads, 0, st>>>(w, R, C, static_cast<const _Float16*>(x),
                                                      M, y);
    }
    CSDR_LAUNCH_CHECK("gguf_linear");
    return CSDR_OK;
}

template <class F>
int dequant_of(const uint8_t* w, size_t nblocks, float* out, hipStream_t st) {
    const size_t total = nblocks * F::BE;
    const int grid = (int)std::min<size_t>((total + kThreads - 1) / kThreads, 65536);
    gguf_dequant_kernel<F><<<grid, kThreads, 0, st>>>(w, nblocks, out);
    CSDR_LAUNCH_CHECK("gguf_dequant");
    return CSDR_OK;
}

struct Format {
    const char* name;
    int id, block_bytes, block_elems;
    Launch fn;
};

template <class F>
constexpr Format fmt(const char* name, int id) {
    return Format{name, id, F::BB, F::BE, Launch{&linear_of<F>, &dequant_of<F>}};
}

// (the reference's names and block sizes, ggufBlockBytesForFormat :181-209)
const Format kFormats[] = {
    fmt<Q4_0>("q4_0", CSDR_GGUF_Q4_0),
    fmt<Q4_1>("q4_1", CSDR_GGUF_Q4_1),
    fmt<Q5<false>>("q5_0", CSDR_GGUF_Q5_0),
    fmt<Q5<true>>("q5_1", CSDR_GGUF_Q5_1),
    fmt<Q8_0>("q8_0", CSDR_GGUF_Q8_0),
    fmt<Q8_1>("q8_1", CSDR_GGUF_Q8_1),
    fmt<Packed<84, 256, 2>>("q2_k", CSDR_GGUF_Q2_K),
    fmt<Packed<110, 256, 3>>("q3_k", CSDR_GGUF_Q3_K),
    fmt<Q4_K>("q4_k", CSDR_GGUF_Q4_K),
    fmt<Packed<176, 256, 5>>("q5_k", CSDR_GGUF_Q5_K),
    fmt<Q6_K>("q6_k", CSDR_GGUF_Q6_K),
    fmt<Q8_K>("q8_k", CSDR_GGUF_Q8_K),
    fmt<Packed<66, 256, 2>>("iq2_xxs", CSDR_GGUF_IQ2_XXS),
    fmt<Packed<74, 256, 2>>("iq2_xs", CSDR_GGUF_IQ2_XS),
    fmt<Packed<98, 256, 3>>("iq3_xxs", CSDR_GGUF_IQ3_XXS),
    fmt<Packed<50, 256, 1>>("iq1_s", CSDR_GGUF_IQ1_S),
    fmt<Packed<18, 32, 4>>("iq4_nl", CSDR_GGUF_IQ4_NL),
    fmt<Packed<110, 256, 3>>("iq3_s", CSDR_GGUF_IQ3_S),
    fmt<Packed<82, 256, 2>>("iq2_s", CSDR_GGUF_IQ2_S),
    fmt<Packed<136, 256, 4>>("iq4_xs", CSDR_GGUF_IQ4_XS),
    fmt<Packed<56, 256, 1>>("iq1_m", CSDR_GGUF_IQ1_M),
    fmt<Packed<72, 128, 4>>("q4_0_4_4", CSDR_GGUF_Q4_0_4_4),
    fmt<Packed<144, 256, 4>>("q4_0_4_8", CSDR_GGUF_Q4_0_4_8),
    fmt<Packed<144, 256, 4>>("q4_0_8_8", CSDR_GGUF_Q4_0_8_8),
    fmt<Packed<54, 256, 1>>("tq1_0", CSDR_GGUF_TQ1_0),
    fmt<Packed<66, 256, 2>>("tq2_0", CSDR_GGUF_TQ2_0),
};

const Format* find(int id) {
    for (const Format& f : kFormats)
        if (f.id == id) return &f;
    return nullptr;
}

}  // namespace

extern "C" {

CSDR_API int csdr_gguf_format(const char* name) {
    if (!name) return -1;
    std::string s(name);
    for (char& ch : s) ch = (char)std::tolower((unsigned char)ch);
    for (const Format& f : kFormats)
        if (s == f.name) return f.id;
    return -1;
}

CSDR_API int csdr_gguf_block(int format, int* block_bytes, int* block_elems) {
    const Format* f = find(format);
    if (!f) return set_error(CSDR_E_INVALID, "gguf: unknown format");
    if (block_bytes) *block_bytes = f->block_bytes;
    if (block_elems) *block_elems = f->block_elems;
    return CSDR_OK;
}

CSDR_API int csdr_gguf_linear(const void* w, int format, int R, int C, const void* x,
                              int x_dtype, int M, float* y, void* hip_stream) {
    const Format* f = find(format);
    if (!f) return set_error(CSDR_E_INVALID, "gguf_linear: unknown format");
    if (!w || !x || !y || R <= 0 || C <= 0 || M <= 0)
        return set_error(CSDR_E_INVALID, "gguf_linear: bad argument");
    if (C % f->block_elems || (M > 1 && C % 16))
        return set_error(CSDR_E_INVALID, std::string("gguf_linear: C must be a multiple of ") +
                                             std::to_string(f->block_elems) + " for " + f->name);
    if (x_dtype != CSDR_F32 && x_dtype != CSDR_F16)
        return set_error(CSDR_E_INVALID, "gguf_linear: x_dtype must be CSDR_F32 or CSDR_F16");
    return f->fn.linear(static_cast<const uint8_t*>(w), R, C, x, x_dtype, M, y,
                        static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_gguf_dequant(const void* w, int format, size_t n_blocks, float* out,
                               void* hip_stream) {
    const Format* f = find(format);
    if (!f) return set_error(CSDR_E_INVALID, "gguf_dequant: unknown format");
    if (!w || !out) return set_error(CSDR_E_INVALID, "gguf_dequant: null argument");
    if (n_blocks == 0) return CSDR_OK;
    return f->fn.dequant(static_cast<const uint8_t*>(w), n_blocks, out,
                         static_cast<hipStream_t>(hip_stream));
}

}  // extern "C"
