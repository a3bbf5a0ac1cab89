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
//   gguf_gemv_lds_kernel (M == 1): one wave per row; the row's bytes staged in LDS with
//     16-byte loads all in flight at once. Formats with a dword-wide decode (Units: q4_0,
//     q4_1, q6_k, the q8 family and the generic rule) give lane l units u = l, l + 64, ... of
//     16 values read as dwords at any byte alignment; with fp16 x the quants become exact fp16
//     subnormal pairs for v_dot2_f32_f16 (scaled into the widest exact range: at 2^-24 the
//     dot's products lose precision). The others take values 8 g .. 8 g + 7 per lane (Dec8:
//     the block's header read once for the 8) in fp32. gguf_gemv_kernel is the element-wise
//     form from memory, for rows longer than the LDS budget. gguf_gemv_pipe_kernel (q8_0
//     and q5_k rows of 8192 values and more): x staged once per workgroup in LDS, a wave's
//     rows cut into 2 KiB items of whole blocks with two items' loads in flight while it
//     decodes a third from LDS.
//   gguf_mm_kernel (M > 1, fp16 X): split-K over 256-element steps of the row, 16 RT rows per
//     workgroup, the 4 waves taking every 4th step. A wave stages its rows' bytes of a step in
//     LDS with dword loads issued one step ahead (a row's step need not start 4-byte aligned),
//     then per 32-wide k step each lane decodes 8 consecutive values of its row (Dec8), rounds
//     them to fp16 once and issues one v_mfma_f32_16x16x32_f16 per 16 output columns (fp32
//     accumulate; the single rounding of W puts the product ~3e-4 relative L2 from fp32). The
//     waves' tiles meet in LDS and each split adds every output into Y (zeroed first) once,
//     16 neighbouring rows per 16 neighbouring threads; the splits of a row tile run on
//     different XCDs, each XCD fetching its share of X.
//   gguf_dequant_kernel: one thread per element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>

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

// The dword at byte offset o of LDS (any alignment): two aligned reads and a byte shift.
__device__ __forceinline__ uint32_t lds32(const uint32_t* s32, int o) {
    return __builtin_amdgcn_alignbyte(s32[(o >> 2) + 1], s32[o >> 2], (uint32_t)(o & 3));
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

// ---- 8 consecutive values e0 .. e0 + 7 of a block (e0 % 8 == 0): the same arithmetic as
// at(), with the block header, scale and quant bytes read once for the 8 (the default reads
// them per value)
template <class F>
struct Dec8 {
    __device__ static void run(const uint8_t* p, int e0, float* o) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = F::at(p, e0 + i);
    }
};
template <>
struct Dec8<Q4_0> {
    __device__ static void run(const uint8_t* p, int e0, float* o) {
        const float d = h16(p);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint8_t b = p[2 + (e0 >> 1) + k];
            o[2 * k] = ((float)(b & 0x0Fu) - 8.0f) * d;
            o[2 * k + 1] = ((float)(b >> 4) - 8.0f) * d;
        }
    }
};
template <>
struct Dec8<Q8_0> {
    __device__ static void run(const uint8_t* p, int e0, float* o) {
        const float d = h16(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (float)(int8_t)p[2 + e0 + i] * d;
    }
};
template <>
struct Dec8<Q6_K> {
    __device__ static void run(const uint8_t* p, int e0, float* o) {
        const int half = e0 >> 7, r = e0 & 127, t = r >> 5, l0 = r & 31;
        const uint8_t* ql = p + half * 64 + l0 + ((t & 1) ? 32 : 0);
        const uint8_t* qh = p + 128 + half * 32 + l0;
        const int sc = (int)(int8_t)p[192 + half * 8 + 2 * t];
        const float d = h16(p + 208);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint8_t lb = ql[i];
            const int lo = (t < 2) ? (lb & 0x0F) : (lb >> 4);
            const int q = (lo | (((qh[i] >> (2 * t)) & 3) << 4)) - 32;
            o[i] = d * (float)(sc * q);
        }
    }
};
template <int BB_, int BE_, int BITS>
struct Dec8<Packed<BB_, BE_, BITS>> {
    __device__ static void run(const uint8_t* p, int e0, float* o) {
        using F = Packed<BB_, BE_, BITS>;
        float d = h16(p);
        if (!isfinite(d) || fabsf(d) < 1e-12f) d = 1.0f;
        // 8 values x BITS bits = BITS whole bytes from bit e0 * BITS (byte aligned)
        const uint8_t* q = p + F::kData + (e0 * BITS >> 3);
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < BITS; ++k) v |= (uint64_t)q[k] << (8 * k);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int qi = (int)((v >> (i * BITS)) & ((1u << BITS) - 1u)) - (1 << (BITS - 1));
            o[i] = (float)qi * d;
        }
    }
};

// x[e0 .. e0 + 7] in fp32 (e0 % 8 == 0): one or two 16-byte loads when x is 16-byte aligned
template <typename XT>
__device__ __forceinline__ void x8(const XT* __restrict__ x, int e0, bool vec, float* o) {
    if (vec) {
        if constexpr (sizeof(XT) == 2) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 v = *reinterpret_cast<const h8*>(x + e0);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = (float)v[i];
        } else {
            const floatx4 a = *reinterpret_cast<const floatx4*>(x + e0);
            const floatx4 b = *reinterpret_cast<const floatx4*>(x + e0 + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = a[i];
                o[4 + i] = b[i];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = csdr::to_f32(x[e0 + i]);
    }
}

// ---- kernels
template <class F, typename XT>
__global__ __launch_bounds__(kThreads) void gguf_gemv_kernel(const uint8_t* __restrict__ W,
                                                             int R, int C,
                                                             const XT* __restrict__ x,
                                                             float* __restrict__ y, int xvec) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x * (kThreads / 64) + wave;
    if (r >= R) return;  // (no barriers below)
    const uint8_t* rowp = W + (size_t)r * (C / F::BE) * F::BB;
    float acc = 0.0f;
    // lane l takes values 8 g .. 8 g + 7 for g = l, l + 64, ... (C is a multiple of 32)
#pragma unroll 2
    for (int g = lane; g < (C >> 3); g += 64) {
        const int e0 = g << 3, b = e0 / F::BE;
        float w8[8], xv[8];
        Dec8<F>::run(rowp + (size_t)b * F::BB, e0 - b * F::BE, w8);
        x8(x, e0, xvec, xv);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(w8[i], xv[i], acc);
    }
    acc = csdr::wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

// Bytes of one 256-element step of a row (256 / BE whole blocks; BE is 32, 128 or 256) and
// the dwords of its staging slot (room for a start that is not 4-byte aligned).
template <class F>
struct Step {
    static_assert(256 % F::BE == 0, "block length must divide 256");
    static constexpr int kBytes = 256 / F::BE * F::BB;
    static constexpr int kDwords = (kBytes + 3 + 3) / 4;
};

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads)
        y[i] = 0.0f;
}

// ---- 8 consecutive values e0 .. e0 + 7 (e0 % 8 == 0) of the block at LDS byte offset bo, as
// the reference's fp32 values (the same single rounding) converted to fp16, from dword reads
// at any byte alignment (Dec8W<F>::value: a word-wide decode exists; else Dec8 byte reads,
// which q8_0 keeps: its word-wide form measured slower, 4096 x 14336 at M = 32 37 -> 57 us)
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
template <class F>
struct Dec8W {
    static constexpr bool value = false;
};
template <>
struct Dec8W<Q6_K> {  // d * (float)(sc * (q - 32)); sc * q - 32 sc is exact in fp32
    static constexpr bool value = true;
    __device__ static half8v run(const uint32_t* s32, int bo, int e0) {
        const int half = e0 >> 7, r = e0 & 127, t = r >> 5, l0 = r & 31;
        const int qlo = bo + half * 64 + l0 + ((t & 1) ? 32 : 0);
        const int qho = bo + 128 + half * 32 + l0;
        const float sc = (float)(int8_t)(lds32(s32, bo + 192 + half * 8 + 2 * t) & 0xFFu);
        const float d = csdr::h2f(lds32(s32, bo + 208) & 0xFFFFu);
        const float c = -32.0f * sc;
        half8v o;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t l = lds32(s32, qlo + 4 * k), h = lds32(s32, qho + 4 * k);
            const uint32_t lo = (t < 2) ? (l & 0x0F0F0F0Fu) : ((l >> 4) & 0x0F0F0F0Fu);
            const uint32_t q = lo | (((h >> (2 * t)) & 0x03030303u) << 4);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[4 * k + i] = (_Float16)(d * fmaf((float)((q >> (8 * i)) & 0xFFu), sc, c));
        }
        return o;
    }
};
template <>
struct Dec8W<Q4_0> {  // (n - 8) * d = fma(n, d, -8 d) with one rounding
    static constexpr bool value = true;
    __device__ static half8v run(const uint32_t* s32, int bo, int e0) {
        const float d = csdr::h2f(lds32(s32, bo) & 0xFFFFu), c = -8.0f * d;
        const uint32_t w = lds32(s32, bo + 2 + (e0 >> 1));
        const uint32_t L = w & 0x0F0F0F0Fu, H = (w >> 4) & 0x0F0F0F0Fu;
        half8v o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[2 * k] = (_Float16)fmaf((float)((L >> (8 * k)) & 0xFFu), d, c);
            o[2 * k + 1] = (_Float16)fmaf((float)((H >> (8 * k)) & 0xFFu), d, c);
        }
        return o;
    }
};
template <int BB_, int BE_, int BITS>
struct Dec8W<Packed<BB_, BE_, BITS>> {  // (q - 2^(BITS-1)) * d = fma(q, d, -2^(BITS-1) d)
    static constexpr bool value = true;
    __device__ static half8v run(const uint32_t* s32, int bo, int e0) {
        using F = Packed<BB_, BE_, BITS>;
        float d = csdr::h2f(lds32(s32, bo) & 0xFFFFu);
        if (!isfinite(d) || fabsf(d) < 1e-12f) d = 1.0f;
        const float c = -(float)(1 << (BITS - 1)) * d;
        const int qo = bo + F::kData + (e0 * BITS >> 3);
        const uint32_t lo = lds32(s32, qo), hi = lds32(s32, qo + 4);
        constexpr uint32_t kMask = (1u << BITS) - 1u;
        half8v o;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int sh = i * BITS;
            const uint32_t q = (sh < 32 ? __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh)
                                        : hi >> (sh - 32)) & kMask;
            o[i] = (_Float16)fmaf((float)q, d, c);
        }
        return o;
    }
};

// gguf_mm_kernel's placement: nrt row tiles (padded to nrt_p, a multiple of 8 / S), S splits of
// KB 256-element steps, column groups outer. Workgroup i runs on XCD i % 8, and split h of
// every row tile goes to the XCDs with xcd % S == h, so an XCD fetches 1/S of X into its L2.
struct MmGrid {
    int nrt, nrt_p, S, KB;
};

// Two waves per SIMD: the decode and the step prefetch want registers more than occupancy
// (measured at M = 32 against the default budget: q6_k 4096 x 14336 52.8 -> 42.5 us).
template <class F, int NT, int RT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void gguf_mm_kernel(const uint8_t* __restrict__ W, int R,
                                                           int C, const _Float16* __restrict__ X,
                                                           int M, float* __restrict__ Y, MmGrid gr) {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    constexpr int ND = Step<F>::kDwords;
    constexpr int ROWS = 16 * RT;
    constexpr int NW = kThreads / 64;
    // the waves' stages (+ 1: Dec8W's dword pairs end inside); after the steps, the waves'
    // tiles for the reduction
    constexpr int kStage = ROWS * ND + 1;
    constexpr int kRed = NW * RT * NT * 64 * 4;
    __shared__ __attribute__((aligned(16))) uint32_t smem[NW * kStage > kRed ? NW * kStage : kRed];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane & 15, j = lane >> 4;
    // the workgroup's tile from its number (number % 8 is the XCD it runs on)
    const int per_z = gr.nrt_p * gr.S;
    const int z = (int)blockIdx.x / per_z, rest = (int)blockIdx.x - z * per_z;
    const int xcd = rest & 7;
    const int t = (rest >> 3) * (8 / gr.S) + xcd / gr.S;
    const int nsteps = (C + 255) / 256;
    const int s0 = (xcd % gr.S) * gr.KB, s1 = min(nsteps, s0 + gr.KB);
    if (t >= gr.nrt || s0 >= s1) return;  // padding or an empty split (the whole workgroup)
    const int r0 = t * ROWS;
    const int n0 = z * 16 * NT;
    const size_t rowbytes = (size_t)(C / F::BE) * F::BB;
    const size_t total = (size_t)R * rowbytes;
    floatx4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const _Float16* xr[NT];
    bool xl[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int n = n0 + nt * 16 + rl;
        xl[nt] = n < M;
        xr[nt] = X + (size_t)min(n, M - 1) * C + 8 * j;
    }
    uint32_t* sw = smem + wave * kStage;
    // A step's staging: the wave's rows' bytes of the step, ROWS x ND dwords (row rr's bytes
    // start at byte (its start & 3) of its slot), PF per lane, loaded into registers one step
    // ahead of its use. Every load is issued unconditionally: a dword past W's last byte reads
    // the dword that holds that byte instead (W is 4-byte aligned, so an aligned dword holding
    // a byte of W lies in W's page), and such dwords are never decoded. (A branch per load, for
    // those few dwords, made every load wait for the one before it.)
    constexpr int PF = (ROWS * ND + 63) / 64;
    uint32_t pf[PF];
    const size_t last_dword = (total - 1) & ~(size_t)3;
    auto fetch = [&](int s) {
        const size_t soff = (size_t)s * Step<F>::kBytes;
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            const int i = min(lane + 64 * k, ROWS * ND - 1);
            const int rr = i / ND, q = i - rr * ND;
            const size_t start = (size_t)min(r0 + rr, R - 1) * rowbytes + soff;
            const size_t a = min((start & ~(size_t)3) + 4 * (size_t)q, last_dword);
            pf[k] = *reinterpret_cast<const uint32_t*>(W + a);
        }
    };
    // X of 32-wide k step t (this lane's 8 values of each column tile)
    auto xload = [&](int e0, int t, half8 (&bv)[NT]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const half8 v = *reinterpret_cast<const half8*>(xr[nt] + e0 + 32 * t);
            bv[nt] = xl[nt] ? v : half8{};
        }
    };
    // 32-wide k step t of step s from the staged bytes, with X already in bv
    auto kstep_x = [&](const uint8_t* const* rowsb, const int* rowso, int t,
                       const half8 (&bv)[NT]) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int e = 32 * t + 8 * j, b = e / F::BE;
            half8 a;
            if constexpr (Dec8W<F>::value) {
                a = Dec8W<F>::run(sw, rowso[rt] + b * F::BB, e - b * F::BE);
            } else {
                float w8[8];
                Dec8<F>::run(rowsb[rt] + b * F::BB, e - b * F::BE, w8);
#pragma unroll
                for (int i = 0; i < 8; ++i) a[i] = (_Float16)w8[i];
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv[nt], acc[rt][nt], 0, 0, 0);
        }
    };
    int s = s0 + wave;
    if (s < s1) fetch(s);
    for (; s < s1; s += NW) {
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            const int i = lane + 64 * k;
            if (i < ROWS * ND) sw[i] = pf[k];
        }
        // this wave's writes before its reads (LDS keeps a wave's operations in order; the
        // fence keeps the compiler from moving the reads up)
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (s + NW < s1) fetch(s + NW);  // the next step's bytes in flight during this one
        const int e0 = s * 256;
        const size_t soff = (size_t)s * Step<F>::kBytes;
        const uint8_t* rowsb[RT];
        int rowso[RT];  // the same as byte offsets in the wave's stage
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int rr = rt * 16 + rl;
            const size_t start = (size_t)min(r0 + rr, R - 1) * rowbytes + soff;
            rowso[rt] = rr * ND * 4 + (int)(start & 3);
            rowsb[rt] = reinterpret_cast<const uint8_t*>(sw) + rowso[rt];
        }
        const int nsub = min(256, C - e0) / 32;  // 32-wide k steps (C is a multiple of BE >= 32)
        if (nsub == 8) {
            // X one k step ahead: its loads in flight during the step before
            half8 xb[2][NT];
            xload(e0, 0, xb[0]);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (t + 1 < 8) xload(e0, t + 1, xb[(t + 1) & 1]);
                kstep_x(rowsb, rowso, t, xb[t & 1]);
            }
        } else {
            for (int t = 0; t < nsub; ++t) {
                half8 bv[NT];
                xload(e0, t, bv);
                kstep_x(rowsb, rowso, t, bv);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    // the 4 waves' tiles meet in LDS (once every wave is past its steps) and the workgroup
    // adds each output into Y once: output (row r, column c) of a tile is element r % 4 of lane
    // c + 16 (r / 4), and 16 neighbouring threads take 16 neighbouring rows (one 64-byte run of
    // Y per 16 atomics, where a lane's own 16 columns were 16 lines)
    __syncthreads();
    floatx4* red = reinterpret_cast<floatx4*>(smem);  // [wave][RT][NT][64]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) red[((wave * RT + rt) * NT + nt) * 64 + lane] = acc[rt][nt];
    __syncthreads();
    const float* redf = reinterpret_cast<const float*>(smem);
    for (int o = threadIdx.x; o < RT * NT * 256; o += kThreads) {
        const int r = o & 15, c = (o >> 4) & 15, tile = o >> 8;  // tile = rt * NT + nt
        const int at = (tile * 64 + c + 16 * (r >> 2)) * 4 + (r & 3);
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += redf[w * RT * NT * 256 + at];
        const int row = r0 + 16 * (tile / NT) + r, col = n0 + 16 * (tile % NT) + c;
        if (row < R && col < M)
            __hip_atomic_fetch_add(Y + (size_t)col * R + row, v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
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

// M == 1 with the row staged in LDS. A workgroup's 4 waves take a row each; a wave copies its
// row's bytes with 16-byte loads from the 16-byte boundary at or below the row's start, all of
// them issued before the first is waited for. Lane l then decodes values 8 g .. 8 g + 7 for
// g = l, l + 64, ... from its block in LDS (Dec8: the block's header read once for the 8) and
// multiplies them by x in fp32 (x read through the caches: staging it in LDS per workgroup
// of 4 rows measured slower, 4096 x 14336 q4_0 19.2 us against 17.9).
constexpr int kRowLoads = 16;  // 16-byte row loads per lane in flight (16 KiB per wave)

// Every format's M == 1 product stages its rows in LDS (rows longer than the LDS budget read
// from memory, gguf_gemv_kernel).
template <class F>
struct StageRow {
    static constexpr bool value = true;
};

// LDS bytes of one wave's row slot (the row plus the up to 15 bytes before it, and 16 more
// for dword reads that end past the row)
template <class F>
size_t gv_row_slot(int C) {
    return ((size_t)(C / F::BE) * F::BB + 15 + 15 + 16) & ~(size_t)15;
}

// v_dot2_f32_f16 on two fp16 pairs held as dwords
__device__ __forceinline__ float fdot2u(uint32_t a, uint32_t b, float c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
}


// x[e .. e + 3] in fp32 (e % 4 == 0): one load when x is 16-byte aligned
template <typename XT>
__device__ __forceinline__ void x4(const XT* __restrict__ x, int e, bool vec, float* o) {
    if (vec) {
        if constexpr (sizeof(XT) == 2) {
            const half4 v = *reinterpret_cast<const half4*>(x + e);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (float)v[i];
        } else {
            const floatx4 v = *reinterpret_cast<const floatx4*>(x + e);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = v[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = csdr::to_f32(x[e + i]);
    }
}

// Formats whose staged row is read in dword-wide units rather than 8 values at a time (Dec8):
// kPerBlock units per block, dot() = the unit's values times x.
template <class F>
struct Units {
    static constexpr bool value = false;
    static constexpr bool kUnitSums = false;
};
// x[e .. e + 7] in fp16 as four dwords of value pairs (16-byte aligned x)
template <typename XT>
__device__ __forceinline__ void xh8(const XT* __restrict__ x, int e, uint32_t* o) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + e);
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
}

constexpr uint32_t kOnesH2 = 0x3C003C00u;  // fp16 (1.0, 1.0)

// q4_0 / q4_1 (:398-417): unit u = half u % 2 of block u / 2, 16 values from 8 quant bytes,
// element i from byte i / 2 (low nibble for even i). With fp16 x each value pair (2k, 2k + 1)
// of a quant dword becomes one exact fp16 subnormal pair q 2^-18 by a byte permute of its low
// and high nibbles and a shift. q4_0: d * (sum q x - 8 sum x); q4_1: d * sum q x + m * sum x.
template <bool HAS_M>
struct UnitsQ4 {
    static constexpr bool value = true;
    static constexpr bool kUnitSums = true;  // x sum over values 16 u .. 16 u + 15 (dotx)
    static constexpr int kPerBlock = 2;
    static constexpr int BB = HAS_M ? 20 : 18, kQs = HAS_M ? 4 : 2;
    template <typename XT>
    __device__ static float dot(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                bool xvec) {
        return dotx<false>(s32, ro, u, x, xvec, nullptr);
    }
    // US: fp16 x in LDS with the unit's x sum given (us[u], formed once for all rows by
    // unit_xsum in the same order as below)
    template <bool US, typename XT>
    __device__ static float dotx(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                 bool xvec, const float* us) {
        const int blk = u >> 1, hf = u & 1;
        const int bo = ro + blk * BB;
        const uint32_t hd = lds32(s32, bo);
        const float d = csdr::h2f(hd & 0xFFFFu);
        const int xb = blk * 32 + hf * 16;
        float a = 0.0f, sx = 0.0f;
        if (sizeof(XT) == 2 && xvec) {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const uint32_t w = lds32(s32, bo + kQs + hf * 8 + 4 * g);
                const uint32_t L = w & 0x0F0F0F0Fu, H = (w >> 4) & 0x0F0F0F0Fu;
                uint32_t xw[4];
                xh8(x, xb + 8 * g, xw);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t pk = __builtin_amdgcn_perm(H, L, 0x0C040C00u + 0x00010001u * k)
                                        << 6;
                    a = fdot2u(pk, xw[k], a);
                    if constexpr (!US) sx = fdot2u(xw[k], kOnesH2, sx);
                }
            }
            if constexpr (US) sx = us[u];
            a *= 0x1p18f;
        } else {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const uint32_t w = lds32(s32, bo + kQs + hf * 8 + 4 * g);
                float xv[8];
                x8(x, xb + 8 * g, xvec, xv);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t b = (w >> (8 * k)) & 0xFFu;
                    a = fmaf((float)(b & 0x0Fu), xv[2 * k], a);
                    a = fmaf((float)(b >> 4), xv[2 * k + 1], a);
                    sx += xv[2 * k] + xv[2 * k + 1];
                }
            }
        }
        if constexpr (HAS_M) return fmaf(d, a, csdr::h2f(hd >> 16) * sx);
        else return d * fmaf(-8.0f, sx, a);
    }
};
template <>
struct Units<Q4_0> : UnitsQ4<false> {};
template <>
struct Units<Q4_1> : UnitsQ4<true> {};

// q8_0 / q8_1 / q8_k (:310-326, :387-395): unit u = values 16 j .. 16 j + 15 of block
// u / (BE / 16), four quant dwords of signed bytes. With fp16 x the bytes are offset to
// unsigned (b + 128, exact) and taken as fp16 subnormal pairs (b + 128) 2^-22:
// d * (sum (b + 128) x - 128 sum x).
template <int BB_, int BE_, int QOFF, bool SCALE_F32>
struct UnitsQ8 {
    static constexpr bool value = true;
    static constexpr bool kUnitSums = true;
    static constexpr int kPerBlock = BE_ / 16;
    template <typename XT>
    __device__ static float dot(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                bool xvec) {
        return dotx<false>(s32, ro, u, x, xvec, nullptr);
    }
    template <bool US, typename XT>
    __device__ static float dotx(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                 bool xvec, const float* us) {
        const int blk = u / kPerBlock, j = u - blk * kPerBlock;
        const int bo = ro + blk * BB_;
        const uint32_t hd = lds32(s32, bo);
        const float d = SCALE_F32 ? __builtin_bit_cast(float, hd) : csdr::h2f(hd & 0xFFFFu);
        const int qo = bo + QOFF + 16 * j;
        const int xb = blk * BE_ + 16 * j;
        float a = 0.0f, sx = 0.0f;
        if (sizeof(XT) == 2 && xvec) {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                uint32_t xw[4];
                xh8(x, xb + 8 * g, xw);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t w = lds32(s32, qo + 8 * g + 4 * h) ^ 0x80808080u;
                    const uint32_t p01 = __builtin_amdgcn_perm(0u, w, 0x0C010C00u) << 2;
                    const uint32_t p23 = __builtin_amdgcn_perm(0u, w, 0x0C030C02u) << 2;
                    a = fdot2u(p01, xw[2 * h], a);
                    a = fdot2u(p23, xw[2 * h + 1], a);
                    if constexpr (!US) {
                        sx = fdot2u(xw[2 * h], kOnesH2, sx);
                        sx = fdot2u(xw[2 * h + 1], kOnesH2, sx);
                    }
                }
            }
            if constexpr (US) sx = us[u];
            return d * fmaf(-128.0f, sx, a * 0x1p22f);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float xv[8];
            x8(x, xb + 8 * g, xvec, xv);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t w = lds32(s32, qo + 8 * g + 4 * h);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    a = fmaf((float)(int8_t)((w >> (8 * i)) & 0xFFu), xv[4 * h + i], a);
            }
        }
        return d * a;
    }
};
template <>
struct Units<Q8_0> : UnitsQ8<34, 32, 2, false> {};
template <>
struct Units<Q8_1> : UnitsQ8<40, 32, 8, true> {};
template <>
struct Units<Q8_K> : UnitsQ8<292, 256, 4, false> {};

// the generic rule (:439-465): unit u = values 16 j .. 16 j + 15 of block u / (BE / 16), two
// groups of 8 values x BITS bits = BITS bytes each (byte aligned), read as two dwords and
// split by funnel shifts; q - 2^(BITS-1) times the block's scale.
template <int BB_, int BE_, int BITS>
struct Units<Packed<BB_, BE_, BITS>> {
    using F = Packed<BB_, BE_, BITS>;
    static constexpr bool value = true;
    static constexpr bool kUnitSums = true;
    static constexpr int kPerBlock = BE_ / 16;
    template <typename XT>
    __device__ static float dot(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                bool xvec) {
        return dotx<false>(s32, ro, u, x, xvec, nullptr);
    }
    template <bool US, typename XT>
    __device__ static float dotx(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                 bool xvec, const float* us) {
        const int blk = u / kPerBlock, j = u - blk * kPerBlock;
        const int bo = ro + blk * BB_;
        float d = csdr::h2f(lds32(s32, bo) & 0xFFFFu);
        if (!isfinite(d) || fabsf(d) < 1e-12f) d = 1.0f;
        constexpr uint32_t kMask = (1u << BITS) - 1u;
        constexpr int kUp = 10 - BITS;  // fp16 x: q 2^(kUp - 24), the widest exact subnormal
        const int qo = bo + F::kData + j * 2 * BITS;
        const int xb = blk * BE_ + j * 16;
        float a = 0.0f, sx = 0.0f;
        const bool h16x = sizeof(XT) == 2 && xvec;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t lo = lds32(s32, qo + g * BITS), hi = lds32(s32, qo + g * BITS + 4);
            uint32_t qv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int sh = i * BITS;
                qv[i] = (sh < 32 ? __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh)
                                 : hi >> (sh - 32)) & kMask;
            }
            if (h16x) {
                uint32_t xw[4];
                xh8(x, xb + 8 * g, xw);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    a = fdot2u((qv[2 * k] | (qv[2 * k + 1] << 16)) << kUp, xw[k], a);
                    if constexpr (!US) sx = fdot2u(xw[k], kOnesH2, sx);
                }
            } else {
                float xv[8];
                x8(x, xb + 8 * g, xvec, xv);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    a = fmaf((float)qv[i], xv[i], a);
                    sx += xv[i];
                }
            }
        }
        if constexpr (US) sx = us[u];
        if (h16x) a *= (float)(1u << (24 - kUp));
        return d * fmaf(-(float)(1 << (BITS - 1)), sx, a);
    }
};

// q6_k (:329-359): unit u of a block = (half h, quad q): values h*128 + 32 t + 4 q + i of the
// four quarters t (scale bytes 192 + 8 h + 2 t) and i = 0..3. The quarters' 6-bit quants come
// from three dwords, ql[h*64 + 4q] (t = 0 low nibbles, t = 2 high), ql[h*64 + 32 + 4q] (t = 1,
// 3) and qh[h*32 + 4q] (bit pair t of each byte), four per dword op. Per quarter
// sum (q - 32) x = sum q x - 32 sum x, then d * sum_t sc_t * that.
template <>
struct Units<Q6_K> {
    static constexpr bool value = true;
    static constexpr bool kUnitSums = false;  // (units of four 4-value groups 32 apart)
    static constexpr int kPerBlock = 16;
    template <typename XT>
    __device__ static float dot(const uint32_t* s32, int ro, int u, const XT* __restrict__ x,
                                bool xvec) {
        const int blk = u >> 4, h = (u >> 3) & 1, q = u & 7;
        const int bo = ro + blk * Q6_K::BB;
        const uint32_t qa = lds32(s32, bo + h * 64 + 4 * q);
        const uint32_t qb = lds32(s32, bo + h * 64 + 32 + 4 * q);
        const uint32_t qh = lds32(s32, bo + 128 + h * 32 + 4 * q);
        const uint32_t s0 = lds32(s32, bo + 192 + h * 8), s1 = lds32(s32, bo + 196 + h * 8);
        const float d = csdr::h2f(lds32(s32, bo + 208) & 0xFFFFu);
        const uint32_t qt[4] = {(qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u),
                                (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u),
                                ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u),
                                ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u)};
        const float sc[4] = {(float)(int8_t)(s0 & 0xFFu), (float)(int8_t)((s0 >> 16) & 0xFFu),
                             (float)(int8_t)(s1 & 0xFFu), (float)(int8_t)((s1 >> 16) & 0xFFu)};
        const int xb = blk * 256 + h * 128 + 4 * q;
        float tot = 0.0f;
        if constexpr (sizeof(XT) == 2) {
            if (xvec) {
                // fp16 x: the quants as fp16 subnormal pairs q 2^-20 (exact), one
                // v_dot2_f32_f16 per two products and per two values of the x sum
                typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                constexpr uint32_t kOnes = 0x3C003C00u;  // (1.0, 1.0)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u32x2 xw = *reinterpret_cast<const u32x2*>(x + xb + 32 * t);
                    const uint32_t x01 = xw.x, x23 = xw.y;
                    const uint32_t p01 = __builtin_amdgcn_perm(0u, qt[t], 0x0C010C00u) << 4;
                    const uint32_t p23 = __builtin_amdgcn_perm(0u, qt[t], 0x0C030C02u) << 4;
                    float a = fdot2u(p01, x01, 0.0f);
                    a = fdot2u(p23, x23, a);
                    float sx = fdot2u(x01, kOnes, 0.0f);
                    sx = fdot2u(x23, kOnes, sx);
                    tot = fmaf(sc[t], fmaf(-0x1p-15f, sx, a), tot);
                }
                return d * 0x1p20f * tot;
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float xv[4];
            x4(x, xb + 32 * t, xvec, xv);
            float a = 0.0f, sx = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a = fmaf((float)((qt[t] >> (8 * i)) & 0xFFu), xv[i], a);
                sx += xv[i];
            }
            tot = fmaf(sc[t], fmaf(-32.0f, sx, a), tot);
        }
        return d * tot;
    }
};

template <class F, typename XT>
__global__ __launch_bounds__(kThreads) void gguf_gemv_lds_kernel(const uint8_t* __restrict__ W,
                                                                 int R, int C,
                                                                 const XT* __restrict__ x,
                                                                 float* __restrict__ y,
                                                                 int slot, int xvec) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = blockIdx.x * (kThreads / 64) + wave;
    const size_t rowbytes = (size_t)(C / F::BE) * F::BB;
    // The row from the 16-byte boundary (of the address) at or below its start, in 16-byte
    // pieces up to the boundary at or above its end. A 16-byte aligned piece never crosses a
    // page, so the bytes it holds outside W share a page with bytes of W.
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
    const uintptr_t start = wa + (size_t)min(r, R - 1) * rowbytes, a0 = start & ~(uintptr_t)15;
    const uintptr_t wend = (wa + (size_t)R * rowbytes + 15) & ~(uintptr_t)15;
    const int lead = (int)(start - a0), npiece = (int)((lead + rowbytes + 15) >> 4);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(a0), (short)0, (int)min(wend - a0, (uintptr_t)0x7FFFFFF0),
        0x00020000);
    uint8_t* my = gsm + (size_t)wave * slot;
    u32x4* myv = reinterpret_cast<u32x4*>(my);
    u32x4 v[kRowLoads];
    const bool has_row = r < R;
    const int np = has_row ? npiece : 0;
    auto load = [&](int p) {  // piece p of the row, or zeros past its end
        return __builtin_amdgcn_raw_buffer_load_b128(  // streaming (nontemporal) policy
            rs, p < np ? (uint32_t)p * 16 : 0x80000000u, 0, 2);
    };
    // the row in batches of kRowLoads pieces per lane
#pragma unroll
    for (int i = 0; i < kRowLoads; ++i)
        if (i * 64 < np) v[i] = load(i * 64 + lane);
#pragma unroll
    for (int i = 0; i < kRowLoads; ++i)
        if (i * 64 + lane < np) myv[i * 64 + lane] = v[i];
    for (int p0 = kRowLoads * 64; p0 < np; p0 += kRowLoads * 64) {
#pragma unroll
        for (int i = 0; i < kRowLoads; ++i)
            if (p0 + i * 64 < np) v[i] = load(p0 + i * 64 + lane);
#pragma unroll
        for (int i = 0; i < kRowLoads; ++i)
            if (p0 + i * 64 + lane < np) myv[p0 + i * 64 + lane] = v[i];
    }
    if (!has_row) return;
    // the row slot is this wave's own: its copy needs only a wave-level ordering
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float acc = 0.0f;
    if constexpr (Units<F>::value) {
        const uint32_t* s32 = reinterpret_cast<const uint32_t*>(gsm);
        const int ro = wave * slot + lead;
        const int nu = (C / F::BE) * Units<F>::kPerBlock;
#pragma unroll 2
        for (int u = lane; u < nu; u += 64) acc += Units<F>::dot(s32, ro, u, x, xvec);
    } else {
        const uint8_t* row = my + lead;
#pragma unroll 2
        for (int g = lane; g < (C >> 3); g += 64) {
            const int e0 = g << 3, b = e0 / F::BE;
            float w8[8], xv[8];
            Dec8<F>::run(row + (size_t)b * F::BB, e0 - b * F::BE, w8);
            x8(x, e0, xvec, xv);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc = fmaf(w8[i], xv[i], acc);
        }
    }
    acc = csdr::wave_sum(acc);
    if (lane == 0) y[r] = acc;
}


// ---- M == 1, pipelined: x staged once per workgroup in LDS, so a wave's only global loads are
// its weight bytes and it can keep two items of them in flight while it decodes a third. The
// workgroup's rows are cut into items of whole blocks (at most kPipeChunk bytes from the
// 16-byte boundary at or below the item's first byte), flattened row-major and split into
// one contiguous run per wave. Per item: the loads of item i + 2 are issued, item i is
// decoded from its LDS slot (x from LDS), and item i + 1 is copied from registers to the
// other slot. A wave's partial row sums meet in LDS (a row's items can fall to two waves).
constexpr int kPipeWaves = 8;
constexpr int kPipeThreads = kPipeWaves * 64;
constexpr int kPipeLpc = 2;                       // 16-byte pieces per lane per item
constexpr int kPipeChunk = 64 * kPipeLpc * 16;    // bytes per item, at most
constexpr int kPipeSlot = kPipeChunk + 16;        // + the dword a read at the end reaches
constexpr int kPipeMaxRows = 64;                  // rows per workgroup (LDS row sums)

template <class F>
constexpr int pipe_blocks() { return (kPipeChunk - 15) / F::BB; }  // blocks per item

// Formats the pipelined kernel serves, on rows of at least kPipeMinC values (measured, 4096
// rows, per call against the one-wave-per-row kernel: q8_0 x 14336 21.0 -> 18.1 us, q5_k
// 18.7 -> 17.0; q4_0 14.1 -> 14.0; q6_k 21.4 -> 24.2 and every 4096-value row 0.7-1.2 us
// slower, where a wave's run is two or three items: those keep the other kernel)
template <class F>
struct PipeM1 {
    static constexpr bool value = false;
};
template <>
struct PipeM1<Q8_0> {
    static constexpr bool value = true;
};
template <>
struct PipeM1<Packed<176, 256, 5>> {  // q5_k
    static constexpr bool value = true;
};
constexpr int kPipeMinC = 8192;

// LDS bytes of the pipelined kernel before the item slots: x, the row totals, the unit sums
// (16-byte multiples)
template <typename XT>
__host__ __device__ constexpr int pipe_fixed_bytes(int C) {
    return ((C * (int)sizeof(XT) + 15) & ~15) + kPipeMaxRows * 4 + (((C / 16) * 4 + 15) & ~15);
}

template <class F, typename XT>
__global__ __launch_bounds__(kPipeThreads) void gguf_gemv_pipe_kernel(
    const uint8_t* __restrict__ W, int R, int C, const XT* __restrict__ x, float* __restrict__ y,
    int rpg, int xvec) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    constexpr int BPC = pipe_blocks<F>();
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // LDS: x (C values), the row sums, the x sum of every 16-value unit (C / 16 floats: the
    // formats' offset terms, formed once here instead of per row), then two item slots per
    // wave
    XT* xs = reinterpret_cast<XT*>(gsm);
    const int xbytes = (C * (int)sizeof(XT) + 15) & ~15;
    float* rsum = reinterpret_cast<float*>(gsm + xbytes);
    float* usum = rsum + kPipeMaxRows;
    uint8_t* slots = gsm + pipe_fixed_bytes<XT>(C) + (size_t)wave * 2 * kPipeSlot;
    const int nbr = C / F::BE, nch = (nbr + BPC - 1) / BPC;
    const int rw0 = blockIdx.x * rpg, rw1 = min(R, rw0 + rpg);
    const int nitems = max(0, rw1 - rw0) * nch;
    const int per = (nitems + kPipeWaves - 1) / kPipeWaves;
    const int i0 = min(nitems, wave * per), i1 = min(nitems, i0 + per);
    // one buffer resource over W from the 16-byte boundary at or below it; a load at or past
    // the end returns zeros without a memory access
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W), wb = wa & ~(uintptr_t)15;
    const size_t rowbytes = (size_t)nbr * F::BB;
    const uint32_t wlen = (uint32_t)((wa - wb + (size_t)R * rowbytes + 15) & ~(size_t)15);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(wb), (short)0, (int)wlen, 0x00020000);
    auto span = [&](int it, int& row, int& cb0, int& nb, uint32_t& a0, int& lead) {
        row = rw0 + it / nch;
        cb0 = (it - (it / nch) * nch) * BPC;
        nb = min(BPC, nbr - cb0);
        const uint32_t off = (uint32_t)(wa - wb + (size_t)row * rowbytes + (size_t)cb0 * F::BB);
        a0 = off & ~15u;
        lead = (int)(off - a0);
    };
    auto issue = [&](int it, u32x4 (&v)[kPipeLpc]) {
        int row, cb0, nb, lead;
        uint32_t a0;
        span(min(it, max(i1 - 1, 0)), row, cb0, nb, a0, lead);
        const int np = it < i1 ? (lead + nb * F::BB + 15) >> 4 : 0;
#pragma unroll
        for (int j = 0; j < kPipeLpc; ++j) {
            const int pc = j * 64 + lane;
            v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, pc < np ? a0 + 16u * pc : 0x80000000u, 0, 2);
        }
    };
    auto put = [&](int slot, const u32x4 (&v)[kPipeLpc]) {
        u32x4* d = reinterpret_cast<u32x4*>(slots + slot * kPipeSlot);
#pragma unroll
        for (int j = 0; j < kPipeLpc; ++j) d[j * 64 + lane] = v[j];
        // the slot is this wave's own: a wave-level ordering suffices
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // x loads first (so that waiting for them does not wait for the weight loads), then the
    // first two items' loads, then x to LDS
    constexpr int kXv = 16 / sizeof(XT);  // values per 16-byte piece
    const int nxv = C / kXv;
    constexpr int kXPer = 4;
    u32x4 xr[kXPer];
    if (xvec) {
#pragma unroll
        for (int j = 0; j < kXPer; ++j)
            xr[j] = *reinterpret_cast<const u32x4*>(x + (size_t)min(j * kPipeThreads + tid, nxv - 1) * kXv);
    }
    u32x4 ring[3][kPipeLpc];
    issue(i0, ring[0]);
    issue(i0 + 1, ring[1]);
    if (xvec) {
#pragma unroll
        for (int j = 0; j < kXPer; ++j)
            if (j * kPipeThreads + tid < nxv)
                reinterpret_cast<u32x4*>(xs)[j * kPipeThreads + tid] = xr[j];
        for (int i = kXPer * kPipeThreads + tid; i < nxv; i += kPipeThreads)
            reinterpret_cast<u32x4*>(xs)[i] = *reinterpret_cast<const u32x4*>(x + (size_t)i * kXv);
    } else {
        for (int i = tid; i < C; i += kPipeThreads) xs[i] = x[i];
    }
    for (int i = tid; i < kPipeMaxRows; i += kPipeThreads) rsum[i] = 0.0f;
    __syncthreads();
    if constexpr (Units<F>::kUnitSums && sizeof(XT) == 2) {
        // each unit's x sum in the order the decoders accumulate it (bit-identical results)
        const uint32_t* xw = reinterpret_cast<const uint32_t*>(xs);
        for (int v = tid; v < C / 16; v += kPipeThreads) {
            float sx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) sx = fdot2u(xw[v * 8 + k], kOnesH2, sx);
            usum[v] = sx;
        }
        __syncthreads();
    }
    put(0, ring[0]);
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(gsm);
    float acc = 0.0f;
    auto step = [&](int it, auto rb) {  // rb: ring index of item it (compile-time)
        constexpr int kR = decltype(rb)::value;
        issue(it + 2, ring[(kR + 2) % 3]);
        if (it < i1) {
            int row, cb0, nb, lead;
            uint32_t a0;
            span(it, row, cb0, nb, a0, lead);
            const int sl = (it - i0) & 1;
            const XT* xp = xs + (size_t)cb0 * F::BE;
            if constexpr (Units<F>::value) {
                const int ro = (int)(slots - gsm) + sl * kPipeSlot + lead;
                const int nu = nb * Units<F>::kPerBlock;
                if constexpr (Units<F>::kUnitSums && sizeof(XT) == 2) {
                    const float* up = usum + cb0 * (F::BE / 16);
                    for (int u = lane; u < nu; u += 64)
                        acc += Units<F>::template dotx<true>(s32, ro, u, xp, true, up);
                } else {
                    for (int u = lane; u < nu; u += 64) acc += Units<F>::dot(s32, ro, u, xp, true);
                }
            } else {
                const uint8_t* rowp = slots + sl * kPipeSlot + lead;
                const int ng = nb * (F::BE / 8);
                for (int g = lane; g < ng; g += 64) {
                    const int e0 = g << 3, b = e0 / F::BE;
                    float w8[8], xv[8];
                    Dec8<F>::run(rowp + (size_t)b * F::BB, e0 - b * F::BE, w8);
                    x8(xp, e0, true, xv);
#pragma unroll
                    for (int k = 0; k < 8; ++k) acc = fmaf(w8[k], xv[k], acc);
                }
            }
            // the row's last item in this wave's run: its sum into the row's LDS total
            const int nrow = rw0 + (it + 1) / nch;
            if (it + 1 == i1 || nrow != row) {
                const float t = csdr::wave_sum(acc);
                if (lane == 0) atomicAdd(&rsum[row - rw0], t);
                acc = 0.0f;
            }
        }
        if (it + 1 < i1) put((it + 1 - i0) & 1, ring[(kR + 1) % 3]);
    };
    for (int it = i0; it < i1; it += 3) {
        step(it, std::integral_constant<int, 0>{});
        step(it + 1, std::integral_constant<int, 1>{});
        step(it + 2, std::integral_constant<int, 2>{});
    }
    __syncthreads();
    for (int i = tid; i < rw1 - rw0; i += kPipeThreads) y[rw0 + i] = rsum[i];
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
        const int xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0;
        // the pipelined kernel: x and the item slots in LDS, W within a 32-bit buffer range
        const size_t lds_p = (size_t)(x_dtype == CSDR_F16 ? pipe_fixed_bytes<_Float16>(C)
                                                          : pipe_fixed_bytes<float>(C)) +
                             (size_t)kPipeWaves * 2 * kPipeSlot;
        const size_t wbytes = (size_t)R * (C / F::BE) * F::BB + 16;
        const char* ev = std::getenv("CSDR_GGUF_PIPE");
        const bool pipe_on = !(ev && *ev && std::atoi(ev) == 0);
        if (PipeM1<F>::value && C >= kPipeMinC && pipe_on && pipe_blocks<F>() >= 1 &&
            lds_p <= 160 * 1024 && wbytes < 0x7FFFFFF0u) {
            int dev = 0, ncu = 256;
            if (hipGetDevice(&dev) == hipSuccess) {
                int v = 0;
                if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                        hipSuccess && v > 0)
                    ncu = v;
            }
            // about two workgroups per CU (each LDS holds x), rows split evenly
            int rpg = (R + 2 * ncu - 1) / (2 * ncu);
            rpg = std::max(1, std::min(rpg, kPipeMaxRows));
            const int g = (R + rpg - 1) / rpg;
            auto go = [&](auto kern, const auto* xp) {
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_p);
                kern<<<g, kPipeThreads, lds_p, st>>>(w, R, C, xp, y, rpg, xvec);
            };
            if (x_dtype == CSDR_F16)
                go(gguf_gemv_pipe_kernel<F, _Float16>, static_cast<const _Float16*>(x));
            else
                go(gguf_gemv_pipe_kernel<F, float>, static_cast<const float*>(x));
            CSDR_LAUNCH_CHECK("gguf_linear");
            return CSDR_OK;
        }
        const size_t slot = gv_row_slot<F>(C);
        const size_t lds = (kThreads / 64) * slot;
        if (StageRow<F>::value && lds <= 160 * 1024) {
            auto go = [&](auto kern, const auto* xp) {
                if (lds > 64 * 1024)
                    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                kern<<<grid, kThreads, lds, st>>>(w, R, C, xp, y, (int)slot, xvec);
            };
            if (x_dtype == CSDR_F16)
                go(gguf_gemv_lds_kernel<F, _Float16>, static_cast<const _Float16*>(x));
            else
                go(gguf_gemv_lds_kernel<F, float>, static_cast<const float*>(x));
        } else if (x_dtype == CSDR_F16)
            gguf_gemv_kernel<F, _Float16><<<grid, kThreads, 0, st>>>(
                w, R, C, static_cast<const _Float16*>(x), y, xvec);
        else
            gguf_gemv_kernel<F, float><<<grid, kThreads, 0, st>>>(
                w, R, C, static_cast<const float*>(x), y, xvec);
    } else {
        if (x_dtype != CSDR_F16)
            return set_error(CSDR_E_UNSUPPORTED, "gguf_linear: M > 1 takes fp16 x");
        if (reinterpret_cast<uintptr_t>(x) % 16)
            return set_error(CSDR_E_INVALID, "gguf_linear: x must be 16-byte aligned");
        if (reinterpret_cast<uintptr_t>(w) % 4)
            return set_error(CSDR_E_INVALID, "gguf_linear: W must be 4-byte aligned at M > 1");
        // Y = 0, then the split-K tiles add into it
        const size_t ny = (size_t)M * R;
        fill_zero_kernel<<<(unsigned)std::min<size_t>((ny + kThreads - 1) / kThreads, 4096),
                           kThreads, 0, st>>>(y, ny);
        // two row tiles per wave; 256-element steps per workgroup: four per wave on long rows
        // (the prefetch covers three of them; 4096 x 14336 at M = 32: q8_0 41.3 us against 8
        // steps' 48.6 at the default register budget), one on short ones; the split count
        // rounded up to a power of two (at most 8) for the XCD placement
        constexpr int RT = 2;
        const int NT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        const int nsteps = (C + 255) / 256;
        const int ks0 = nsteps >= 32 ? 16 : 4;
        MmGrid g;
        g.nrt = (R + 16 * RT - 1) / (16 * RT);
        g.S = 1;
        while (g.S < 8 && g.S * ks0 < nsteps) g.S *= 2;
        g.KB = (nsteps + g.S - 1) / g.S;
        const int pad = 8 / g.S;
        g.nrt_p = (g.nrt + pad - 1) / pad * pad;
        const int gz = (M + 16 * NT - 1) / (16 * NT);
        const long long nwg = (long long)g.nrt_p * g.S * gz;
        if (nwg > 0x7fffffffLL)
            return set_error(CSDR_E_UNSUPPORTED, "gguf_linear: too many output tiles");
        const auto* xp = static_cast<const _Float16*>(x);
        const unsigned grid = (unsigned)nwg;
        if (NT == 1) gguf_mm_kernel<F, 1, RT><<<grid, kThreads, 0, st>>>(w, R, C, xp, M, y, g);
        else if (NT == 2) gguf_mm_kernel<F, 2, RT><<<grid, kThreads, 0, st>>>(w, R, C, xp, M, y, g);
        else gguf_mm_kernel<F, 4, RT><<<grid, kThreads, 0, st>>>(w, R, C, xp, M, y, g);
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
