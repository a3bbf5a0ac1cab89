// q4k.hip — GGUF Q4_K dequant-matmul on gfx950, never materialising an fp32 W.
//
// Reference path (cortexSDR tree): SparseInferenceEngine.cpp decodeSupportedGGUFQuantized
// (q4_k at :362-384, scale/min unpack ggufGetScaleMinQ4K at :266-274) dequantises the whole
// tensor to fp32 at layer load, then Kernels::linear_forward (kernels/blas_kernels.cpp:264-293)
// computes out (M x R) = in (M x C) . W^T. The HSDR compress side reads the same blocks in
// the interleaved element order (HierarchicalSDRStrategy.cpp:836-845); both orders are served.
//
// Super-block (144 bytes, 256 values): f16 d, f16 dmin, 12 bytes of packed 6-bit scales and
// mins for 8 sub-blocks of 32, 128 bytes of 4-bit quants. value = d*sc*q - dmin*m.
//   ggml order:        32-byte group g holds sub-block 2g in its low nibbles, 2g+1 in its
//                      high nibbles (byte j of group g -> elements 64g+j and 64g+32+j).
//   interleaved order: element i of the super-block is byte i/2, low nibble when i is even.
//
// Kernels
//   q4k_gemv_kernel (M == 1): 16 waves per workgroup, a wave per row at a time; a lane takes
//     one 32-byte quant group of a super-block plus the block header, so a wave step covers
//     16 blocks, and a wave keeps up to 2 steps in flight. x is staged once per workgroup in a
//     lane-major LDS layout with the sub-block sums of x. Per group:
//     y += d*sc*(sum q*x) - dmin*m*(sum x), the products exact and summed in fp32.
//   q4k_mm_kernel (M > 1): 8 waves own 128 rows and a range of super-blocks (split K). Per
//     super-block a lane forms q * sc for 8 values of each sub-block of its row as exact fp16
//     subnormals, and v_mfma_f32_16x16x32_f16 multiplies them with fp16 X (staged in LDS in
//     the matching k order) into an fp32 tile scaled by d per super-block; the dmin * m term
//     is a second small product with the sub-block sums of X. No rounding of W: the product
//     is within about 1e-6 (relative L2) of fp32. Workgroups of one row range add into Y.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
constexpr int kBlockBytes = 144;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t byte_of(const u32x4& v, int k) {
    const uint32_t w = k < 4 ? v.y : (k < 8 ? v.z : v.w);  // header bytes 4..15 = scales
    return (w >> (8 * (k & 3))) & 0xFFu;
}

// 6-bit scale and min of sub-block j from the 12 scale bytes (header words y, z, w):
// j < 4: low 6 bits of bytes j / j+4; j >= 4: low nibble / high nibble of byte j+4 plus
// the top two bits of bytes j-4 / j.
__device__ __forceinline__ void scale_min(const u32x4& hdr, int j, float& sc, float& mn) {
    if (j < 4) {
        sc = (float)(byte_of(hdr, j) & 63u);
        mn = (float)(byte_of(hdr, j + 4) & 63u);
    } else {
        const uint32_t bj4 = byte_of(hdr, j + 4);
        sc = (float)((bj4 & 0xFu) | ((byte_of(hdr, j - 4) >> 6) << 4));
        mn = (float)((bj4 >> 4) | ((byte_of(hdr, j) >> 6) << 4));
    }
}

__device__ __forceinline__ float hdr_d(const u32x4& h) { return csdr::h2f(h.x & 0xFFFFu); }
__device__ __forceinline__ float hdr_dmin(const u32x4& h) { return csdr::h2f(h.x >> 16); }

// ---------------------------------------------------------------- M == 1
//
// A workgroup of 16 waves owns 16 rpw rows (rpw consecutive rows per wave). A wave step covers
// 16 super-blocks of one row: lane l takes block l / 4 of the step and its 32-byte quant group
// g = l % 4 (64 values, sub-blocks 2g and 2g+1 in both element orders), loading the block
// header and the group with three 16-byte loads. Each wave keeps RING steps in flight,
// issuing step t + RING as soon as step t is multiplied, and runs straight on from one of
// its rows into the next.
//
// x is staged once per workgroup in a lane-major layout, so each lane reads its values with
// 16-byte LDS reads that no two lanes of a wave share a bank for: chunk k (k = 0..7) of lane
// l holds the x values of quant bytes 4k .. 4k+3 of its group, ordered to match how a quant
// dword splits into value pairs. With fp16 x two nibbles masked in place (w & 0x000F000F,
// w & 0x00F000F0) are two fp16 subnormals, q * 2^-24 or q * 2^-20, so one v_dot2_f32_f16
// takes two exact products into an fp32 sum; the powers of two go into d. With fp32 x the
// nibbles are converted with v_cvt_f32_ubyteN and multiplied in fp32. The per-sub-block sums
// of x for the dmin * m term are formed once, at staging.
constexpr int kGvWaves = 16;
constexpr int kRawBufferDword3 = 0x00020000;  // raw buffer resource word 3 (bounds-checked)
constexpr int kGvThreads = 64 * kGvWaves;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// 16-byte LDS chunks per lane per 16-block step: 8 with fp16 x, 16 with fp32 (lo and hi halves)
template <typename XT>
constexpr int gv_chunks() {
    return sizeof(XT) == 2 ? 8 : 16;
}

// LDS bytes of the staged x and sub-block sums for nblk super-blocks
template <typename XT>
size_t gv_lds_bytes(int nblk) {
    const size_t ng = (size_t)(nblk + 15) / 16;
    return ng * gv_chunks<XT>() * 64 * 16 + ng * 16 * 8 * sizeof(float);
}

// One quant dword (bytes b0..b3) of a lane's group against its staged x chunk, into a
// low-nibble sum sl and a high-nibble sum sh.
// fp16 chunk: pairs (b0.lo, b2.lo) (b0.hi, b2.hi) (b1.lo, b3.lo) (b1.hi, b3.hi). A nibble
// masked in place is an fp16 subnormal: a low nibble at bits 0-3 is q * 2^-24, a high one at
// bits 4-7 is q * 2^-20, so sl gathers sum q x * 2^-24 and sh sum q x * 2^-20 exactly.
__device__ __forceinline__ void gv_dot_h(uint32_t w, const u32x4& xc, float& sl, float& sh) {
    const uint32_t w8 = w >> 8;
    const half2v p0 = __builtin_bit_cast(half2v, w & 0x000F000Fu);
    const half2v p1 = __builtin_bit_cast(half2v, w & 0x00F000F0u);
    const half2v p2 = __builtin_bit_cast(half2v, w8 & 0x000F000Fu);
    const half2v p3 = __builtin_bit_cast(half2v, w8 & 0x00F000F0u);
    // (the x dwords go through named copies: a bit cast of a vector element expression
    // reads element 0 with this compiler)
    const uint32_t x0 = xc.x, x1 = xc.y, x2 = xc.z, x3 = xc.w;
    sl = __builtin_amdgcn_fdot2(p0, __builtin_bit_cast(half2v, x0), sl, false);
    sh = __builtin_amdgcn_fdot2(p1, __builtin_bit_cast(half2v, x1), sh, false);
    sl = __builtin_amdgcn_fdot2(p2, __builtin_bit_cast(half2v, x2), sl, false);
    sh = __builtin_amdgcn_fdot2(p3, __builtin_bit_cast(half2v, x3), sh, false);
}
// byte I of w as a float (one v_cvt_f32_ubyteI)
template <int I>
__device__ __forceinline__ float ub(uint32_t w) {
    return (float)((w >> (8 * I)) & 0xFFu);
}
// fp32 chunks: lo = x of the low nibbles of b0..b3, hi = of the high nibbles
__device__ __forceinline__ void gv_dot_f(uint32_t w, const floatx4& lo, const floatx4& hi,
                                         float& s0, float& s1) {
    const uint32_t a = w & 0x0F0F0F0Fu, b = (w >> 4) & 0x0F0F0F0Fu;
    s0 = fmaf(ub<0>(a), lo.x, s0);
    s0 = fmaf(ub<1>(a), lo.y, s0);
    s0 = fmaf(ub<2>(a), lo.z, s0);
    s0 = fmaf(ub<3>(a), lo.w, s0);
    s1 = fmaf(ub<0>(b), hi.x, s1);
    s1 = fmaf(ub<1>(b), hi.y, s1);
    s1 = fmaf(ub<2>(b), hi.z, s1);
    s1 = fmaf(ub<3>(b), hi.w, s1);
}

// Scales and mins of sub-blocks j = 2g and 2g + 1 (the same unpacking as scale_min, for a pair)
__device__ __forceinline__ void scale_min_pair(const u32x4& hdr, int g, float& sc0, float& m0,
                                               float& sc1, float& m1) {
    const int sh = (g & 1) * 16;  // byte (2g) & 3 of the scale words
    const uint32_t Y = hdr.y >> sh, Z = hdr.z >> sh, Wd = hdr.w >> sh;
    // sub-blocks 0-3 keep 6 bits in one byte, 4-7 split them over two; both forms are formed
    // and one selected (a lane's g never changes, and a branch would split the wave)
    const uint32_t la0 = Y & 63u, la1 = (Y >> 8) & 63u, lb0 = Z & 63u, lb1 = (Z >> 8) & 63u;
    const uint32_t ha0 = (Wd & 15u) | ((Y >> 2) & 48u);
    const uint32_t ha1 = ((Wd >> 8) & 15u) | ((Y >> 10) & 48u);
    const uint32_t hb0 = ((Wd >> 4) & 15u) | ((Z >> 2) & 48u);
    const uint32_t hb1 = ((Wd >> 12) & 15u) | ((Z >> 10) & 48u);
    const bool low = g < 2;
    sc0 = (float)(low ? la0 : ha0);
    sc1 = (float)(low ? la1 : ha1);
    m0 = (float)(low ? lb0 : hb0);
    m1 = (float)(low ? lb1 : hb1);
}

// x -> LDS in the lane-major chunk layout, and the 32-value sub-block sums of x. An item is
// (block, group g, chunk k), 32 per block, k fastest so that the 8 items of a (block, g) sit
// in 8 neighbouring lanes and their partial sums meet by lane exchange. Chunk index
// ((G * CH + k) * 64 + l) for 16-block group G and lane l = 4 (block % 16) + g; with fp32 x
// chunk k is two LDS chunks, 2k (low-nibble values) and 2k + 1 (high).
constexpr int kStageItems = 2;  // items per thread per staging batch

struct GvStageRaw {
    u32x4 a, b;
};

template <int ORDER, typename XT>
__device__ __forceinline__ void gv_stage_load(const XT* __restrict__ x, int nblk, int batch,
                                              GvStageRaw (&raw)[kStageItems]) {
#pragma unroll
    for (int j = 0; j < kStageItems; ++j) {
        const int it = (batch * kStageItems + j) * kGvThreads + threadIdx.x;
        const int blk = min(it >> 5, nblk - 1), g = (it >> 3) & 3, k = it & 7;
        const XT* xb = x + (size_t)blk * 256 + 64 * g;
        if constexpr (sizeof(XT) == 2) {
            if (ORDER == 0) {
                const uint2 lo = *reinterpret_cast<const uint2*>(xb + 4 * k);
                const uint2 hi = *reinterpret_cast<const uint2*>(xb + 32 + 4 * k);
                raw[j].a = u32x4{lo.x, lo.y, hi.x, hi.y};
            } else {
                raw[j].a = *reinterpret_cast<const u32x4*>(xb + 8 * k);
            }
        } else {
            const int o0 = ORDER == 0 ? 4 * k : 8 * k, o1 = ORDER == 0 ? 32 + 4 * k : 8 * k + 4;
            raw[j].a = *reinterpret_cast<const u32x4*>(xb + o0);
            raw[j].b = *reinterpret_cast<const u32x4*>(xb + o1);
        }
    }
}

template <int ORDER, typename XT>
__device__ __forceinline__ void gv_stage_store(int nblk, int batch,
                                               const GvStageRaw (&raw)[kStageItems], u32x4* xs,
                                               float* sums) {
    constexpr int CH = gv_chunks<XT>();
#pragma unroll
    for (int j = 0; j < kStageItems; ++j) {
        const int it = (batch * kStageItems + j) * kGvThreads + threadIdx.x;
        const int blk = it >> 5, g = (it >> 3) & 3, k = it & 7;
        const bool valid = blk < nblk;
        const int G = blk >> 4, l = (blk & 15) * 4 + g;
        float s0, s1;  // ggml: low- and high-nibble values; interleaved: all 8 (s0)
        if constexpr (sizeof(XT) == 2) {
            const u32x4 e = raw[j].a;
            u32x4 out;
            if (ORDER == 0) {  // e = lo0 lo1 lo2 lo3 hi0 hi1 hi2 hi3
                out.x = __builtin_amdgcn_perm(e.y, e.x, 0x05040100u);
                out.y = __builtin_amdgcn_perm(e.w, e.z, 0x05040100u);
                out.z = __builtin_amdgcn_perm(e.y, e.x, 0x07060302u);
                out.w = __builtin_amdgcn_perm(e.w, e.z, 0x07060302u);
            } else {  // e = 8 consecutive values: lo t = value 2t, hi t = value 2t + 1
                out.x = __builtin_amdgcn_perm(e.z, e.x, 0x05040100u);
                out.y = __builtin_amdgcn_perm(e.z, e.x, 0x07060302u);
                out.z = __builtin_amdgcn_perm(e.w, e.y, 0x05040100u);
                out.w = __builtin_amdgcn_perm(e.w, e.y, 0x07060302u);
            }
            if (valid) xs[(G * CH + k) * 64 + l] = out;
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 v = __builtin_bit_cast(h8, e);
            const float a = ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
            const float b = ((float)v[4] + (float)v[5]) + ((float)v[6] + (float)v[7]);
            s0 = ORDER == 0 ? a : a + b;
            s1 = b;
        } else {
            const floatx4 a = __builtin_bit_cast(floatx4, raw[j].a);
            const floatx4 b = __builtin_bit_cast(floatx4, raw[j].b);
            floatx4 lo, hi;
            if (ORDER == 0) {
                lo = a;
                hi = b;
            } else {
                lo = floatx4{a.x, a.z, b.x, b.z};
                hi = floatx4{a.y, a.w, b.y, b.w};
            }
            if (valid) {
                xs[(G * CH + 2 * k) * 64 + l] = __builtin_bit_cast(u32x4, lo);
                xs[(G * CH + 2 * k + 1) * 64 + l] = __builtin_bit_cast(u32x4, hi);
            }
            const float sl = (lo.x + lo.y) + (lo.z + lo.w), sh = (hi.x + hi.y) + (hi.z + hi.w);
            s0 = ORDER == 0 ? sl : sl + sh;
            s1 = sh;
        }
        // sub-block sums: ggml sums s0 / s1 over the 8 chunks of (block, g) into sub-blocks
        // 2g / 2g + 1; interleaved sums s0 over chunks 0-3 (sub-block 2g) and 4-7 (2g + 1)
        s0 += __shfl_xor(s0, 1);
        s0 += __shfl_xor(s0, 2);
        if (ORDER == 0) {
            s1 += __shfl_xor(s1, 1);
            s1 += __shfl_xor(s1, 2);
            s0 += __shfl_xor(s0, 4);
            s1 += __shfl_xor(s1, 4);
            if (valid && k == 0) reinterpret_cast<float2*>(sums)[blk * 4 + g] = float2{s0, s1};
        } else {
            if (valid && (k & 3) == 0) sums[blk * 8 + 2 * g + (k >> 2)] = s0;
        }
    }
}

struct GvSlot {
    u32x4 h, q0, q1;
};

template <int ORDER, typename XT, int RING>
__global__ __launch_bounds__(kGvThreads) void q4k_gemv_kernel(const uint8_t* __restrict__ W, int R,
                                                              int nblk, const XT* __restrict__ x,
                                                              float* __restrict__ y, int rpw) {
    constexpr int CH = gv_chunks<XT>();
    extern __shared__ __attribute__((aligned(16))) unsigned char gv_smem[];
    const int spr = (nblk + 15) >> 4;  // wave steps per row (at least RING)
    u32x4* xs = reinterpret_cast<u32x4*>(gv_smem);
    float* sums = reinterpret_cast<float*>(gv_smem + (size_t)spr * CH * 64 * 16);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int bl = lane >> 2, g = lane & 3;
    const int row0 = (blockIdx.x * kGvWaves + wave) * rpw;
    const int nrows = max(0, min(rpw, R - row0));
    const int T = nrows * spr;  // this wave's steps: none, or at least RING
    // The wave's rows are read through a raw buffer resource bounded to them, so that a lane
    // past a row's last block loads without a branch (and gets zeros without touching
    // memory). A wave with rows has at least RING steps, so the first RING loads, and those
    // of the steady-state loop below, are unconditional: the compiler then waits for exactly
    // the step being multiplied. (A wave without rows loads zeros only.)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W + (size_t)min(row0, R - 1) * nblk * kBlockBytes), (short)0,
        nrows * nblk * kBlockBytes, kRawBufferDword3);
    int lr = 0, ls = 0;  // row and step of the next load
    auto load = [&](GvSlot& sl) {
        const int blk = ls * 16 + bl;
        const uint32_t off = blk < nblk ? (uint32_t)(lr * nblk + blk) * kBlockBytes : 0x80000000u;
        sl.h = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        sl.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 + 32 * g, 0, 0);
        sl.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32 + 32 * g, 0, 0);
        if (++ls == spr) {
            ls = 0;
            ++lr;
        }
    };
    int cr = 0, cs = 0;  // row and step being multiplied
    float acc = 0.0f;
    auto step = [&](const GvSlot& sl) {
        const int blk = cs * 16 + bl;
        // per-nibble sums: ggml puts low nibbles in sub-block 2g (a0, a1) and high ones in
        // 2g + 1 (b0, b1); interleaved puts dwords 0-3 in 2g (low a0, high a1) and 4-7 in
        // 2g + 1 (b0, b1)
        float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
        const uint32_t qd[8] = {sl.q0.x, sl.q0.y, sl.q0.z, sl.q0.w,
                                sl.q1.x, sl.q1.y, sl.q1.z, sl.q1.w};
        const u32x4* xc = xs + (size_t)cs * CH * 64 + lane;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float& u0 = ORDER == 0 ? ((c & 1) ? a1 : a0) : (c < 4 ? a0 : b0);
            float& u1 = ORDER == 0 ? ((c & 1) ? b1 : b0) : (c < 4 ? a1 : b1);
            if constexpr (sizeof(XT) == 2) {
                gv_dot_h(qd[c], xc[c * 64], u0, u1);
            } else {
                const floatx4 lo = __builtin_bit_cast(floatx4, xc[(2 * c) * 64]);
                const floatx4 hi = __builtin_bit_cast(floatx4, xc[(2 * c + 1) * 64]);
                gv_dot_f(qd[c], lo, hi, u0, u1);
            }
        }
        // sub-block sums of q x (fp16 x: high-nibble sums carry 2^-20 where low ones 2^-24)
        constexpr float kH = sizeof(XT) == 2 ? 0.0625f : 1.0f;
        const float A = ORDER == 0 ? a0 + a1 : a0 + kH * a1;
        const float B = ORDER == 0 ? kH * (b0 + b1) : b0 + kH * b1;
        float sc0, m0, sc1, m1;
        scale_min_pair(sl.h, g, sc0, m0, sc1, m1);
        const float d = hdr_d(sl.h) * (sizeof(XT) == 2 ? 16777216.0f : 1.0f);
        const float dm = hdr_dmin(sl.h);
        const float2 sx = reinterpret_cast<const float2*>(sums)[min(blk, nblk - 1) * 4 + g];
        const float part =
            ((d * sc0) * A - (dm * m0) * sx.x) + ((d * sc1) * B - (dm * m1) * sx.y);
        acc += blk < nblk ? part : 0.0f;
        if (++cs == spr) {
            acc = csdr::wave_sum(acc);
            if (lane == 0) y[row0 + cr] = acc;
            acc = 0.0f;
            cs = 0;
            ++cr;
        }
    };
    // x's first staging batch goes out first, then the weight steps, so that staging waits
    // only for its own loads
    GvStageRaw raw[kStageItems];
    gv_stage_load<ORDER, XT>(x, nblk, 0, raw);
    // Only the first step goes out before the barrier: every wave's first step is then
    // ahead of any wave's second in the memory pipeline
    GvSlot ring[RING];
    load(ring[0]);
    gv_stage_store<ORDER, XT>(nblk, 0, raw, xs, sums);
    const int nbatch = (nblk * 32 + kGvThreads * kStageItems - 1) / (kGvThreads * kStageItems);
    for (int b = 1; b < nbatch; ++b) {
        gv_stage_load<ORDER, XT>(x, nblk, b, raw);
        gv_stage_store<ORDER, XT>(nblk, b, raw, xs, sums);
    }
    __syncthreads();
    if (T == 0) return;  // (no barriers below)
#pragma unroll
    for (int k = 1; k < RING; ++k) load(ring[k]);
    int t0 = 0;
    for (; t0 + 2 * RING <= T; t0 += RING) {  // every step's follow-up load is in range
#pragma unroll
        for (int k = 0; k < RING; ++k) {
            step(ring[k]);
            load(ring[k]);
        }
    }
    for (; t0 < T; t0 += RING) {  // the last steps: loads only up to step T - 1
#pragma unroll
        for (int k = 0; k < RING; ++k) {
            if (t0 + k < T) step(ring[k]);
            if (t0 + k + RING < T) load(ring[k]);
        }
    }
}

template <typename T>
struct TypeTag {
    using type = T;
};

// Steps a wave keeps in flight for rows of spr steps: at most spr, so that a wave with rows
// has at least that many. Measured at 4096 x 14336, fp16 x (4 steps per row): 9.9 us with
// two, 10.1 with one, 10.8 with four (a wave's steps queue ahead of other waves' first ones).
int gv_ring_for(int spr) { return spr >= 2 ? 2 : 1; }

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads)
        y[i] = 0.0f;
}

// ---------------------------------------------------------------- M > 1, exact quants
//
// A workgroup of 8 waves owns 128 rows (a 16-row tile per wave), the range of super-blocks
// blockIdx.y covers (split K) and 16 NT columns. Per super-block every wave multiplies its
// tile on v_mfma_f32_16x16x32_f16 with W as the B operand (k x rows) and X as A (columns x k),
// so each output element a lane holds belongs to the lane's own W row:
//   * a lane (row rl = l % 16, k-slice j = l / 16) takes the 8 values 8j .. 8j + 7 of each
//     32-element sub-block s of its row; q * sc (at most 15 * 63 = 945) is formed as a pair of
//     16-bit integers with one v_pk_mul_lo_u16 and read as two fp16 subnormals q * sc * 2^-24,
//     exact, so the 8 sub-blocks of a super-block accumulate in one fp32 D tile;
//   * the min term sum_s m_s * (sum of x over s) is one more product, of the sub-block sums
//     of X (split into fp16 hi + lo parts, two steps) with m_s (6-bit, exact in fp16);
//   * per super-block: acc += (d * 2^24) * D - dmin * Dm in fp32.
// The k order inside a lane's 8 values follows how a quant dword splits into value pairs; X
// is staged in LDS in the same order, one super-block ahead (two buffers), with the
// sub-block sums. Workgroups of one row range add their partial sums into Y (zeroed first).
constexpr int kMmWaves = 8;
constexpr int kMmThreads = 64 * kMmWaves;
constexpr int kMmRows = 16 * kMmWaves;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// 16-byte LDS chunks of one super-block buffer: per column tile 8 X tiles and 2 sum tiles
template <int NT>
constexpr int mm_buf_chunks() {
    return NT * 10 * 64;
}

// x values e0..e7 (dwords d = (e0,e1) (e2,e3) (e4,e5) (e6,e7)) in the order the quant pairs
// take them: ggml (e0,e2) (e1,e3) (e4,e6) (e5,e7), interleaved (e0,e4) (e1,e5) (e2,e6) (e3,e7)
template <int ORDER>
__device__ __forceinline__ u32x4 mm_x_order(const u32x4& d) {
    u32x4 o;
    if (ORDER == 0) {
        o.x = __builtin_amdgcn_perm(d.y, d.x, 0x05040100u);
        o.y = __builtin_amdgcn_perm(d.y, d.x, 0x07060302u);
        o.z = __builtin_amdgcn_perm(d.w, d.z, 0x05040100u);
        o.w = __builtin_amdgcn_perm(d.w, d.z, 0x07060302u);
    } else {
        o.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
        o.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
        o.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
        o.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
    }
    return o;
}

// one nibble pair (bits 0-3 and 16-19 of v) times the sub-block scale, as two fp16 subnormals
__device__ __forceinline__ uint32_t mm_qs(uint32_t v, uint32_t sc2) {
    const u16x2 q = __builtin_bit_cast(u16x2, v & 0x000F000Fu);
    return __builtin_bit_cast(uint32_t, q * __builtin_bit_cast(u16x2, sc2));
}

template <int ORDER, int NT>
__global__ __launch_bounds__(kMmThreads) void q4k_mm_kernel(const uint8_t* __restrict__ W, int R,
                                                            int nblk, const _Float16* __restrict__ X,
                                                            int M, float* __restrict__ Y, int KB) {
    extern __shared__ __attribute__((aligned(16))) unsigned char mm_smem[];
    u32x4* xl = reinterpret_cast<u32x4*>(mm_smem);  // [2][mm_buf_chunks<NT>()]
    constexpr int kBuf = mm_buf_chunks<NT>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int rl = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * kMmRows + wave * 16;
    const int b0 = blockIdx.y * KB, b1 = min(nblk, b0 + KB);
    const int n0 = blockIdx.z * 16 * NT;
    const int C = nblk * 256;
    // the sum tiles hold values at k < 8 only (lanes 0-15): zero the rest once
    for (int i = threadIdx.x; i < 2 * NT * 2 * 48; i += kMmThreads) {
        const int l = 16 + i % 48, t = i / 48;  // t: buffer * 2 NT + nt * 2 + hi/lo
        const int buf = t / (2 * NT), nt = (t / 2) % NT, hl = t & 1;
        xl[buf * kBuf + (nt * 10 + 8 + hl) * 64 + l] = u32x4{0u, 0u, 0u, 0u};
    }
    // X staging: piece p = (column, sub-block, k-slice), 16 NT * 32 per super-block, NT per
    // thread
    auto stage_load = [&](int b, u32x4 (&xr)[NT]) {
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int p = i * kMmThreads + threadIdx.x;
            const int col = n0 + (p >> 5), s = (p >> 2) & 7, jj = p & 3;
            const u32x4 v = *reinterpret_cast<const u32x4*>(X + (size_t)min(col, M - 1) * C +
                                                            (size_t)b * 256 + 32 * s + 8 * jj);
            xr[i] = col < M ? v : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto stage_store = [&](int buf, const u32x4 (&xr)[NT]) {
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int p = i * kMmThreads + threadIdx.x;
            const int c = p >> 5, s = (p >> 2) & 7, jj = p & 3;
            const int nt = c >> 4, l = (c & 15) + 16 * jj;
            xl[buf * kBuf + (nt * 10 + s) * 64 + l] = mm_x_order<ORDER>(xr[i]);
            // the sub-block sum of this column: 4 neighbouring threads hold its 4 slices
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 v = __builtin_bit_cast(h8, xr[i]);
            float sm = (((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3])) +
                       (((float)v[4] + (float)v[5]) + ((float)v[6] + (float)v[7]));
            sm += __shfl_xor(sm, 1);
            sm += __shfl_xor(sm, 2);
            if (jj == 0) {
                const _Float16 hi = (_Float16)sm;
                const _Float16 lo = (_Float16)(sm - (float)hi);
                _Float16* th = reinterpret_cast<_Float16*>(xl + buf * kBuf + (nt * 10 + 8) * 64);
                _Float16* tl = reinterpret_cast<_Float16*>(xl + buf * kBuf + (nt * 10 + 9) * 64);
                th[(c & 15) * 8 + s] = hi;
                tl[(c & 15) * 8 + s] = lo;
            }
        }
    };
    // this lane's bytes of a super-block of its row: header, and per sub-block pair (ggml) or
    // sub-block (interleaved) the 8 or 4 bytes of its k-slice
    struct Blk {
        u32x4 hdr;
        uint32_t q[8];
    };
    const uint8_t* wrow = W + (size_t)min(r0 + rl, R - 1) * nblk * kBlockBytes;
    auto load_blk = [&](int b, Blk& o) {
        const uint8_t* bp = wrow + (size_t)b * kBlockBytes;
        o.hdr = *reinterpret_cast<const u32x4*>(bp);
        if (ORDER == 0) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint2 v = *reinterpret_cast<const uint2*>(bp + 16 + 32 * g + 8 * j);
                o.q[2 * g] = v.x;
                o.q[2 * g + 1] = v.y;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 8; ++s)
                o.q[s] = *reinterpret_cast<const uint32_t*>(bp + 16 + 16 * s + 4 * j);
        }
    };
    floatx4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const Blk& cb) {
        // B operands: q * sc per sub-block, and m at k = s for the min product
        half8 bq[8];
        float scf[8], mnf[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) scale_min(cb.hdr, s, scf[s], mnf[s]);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t sc = (uint32_t)scf[s], sc2 = sc | (sc << 16);
            uint32_t w0, w1;  // this lane's 8 (ggml) or 4 (interleaved) bytes of sub-block s
            if (ORDER == 0) {
                const int sh = (s & 1) * 4;  // odd sub-blocks: high nibbles
                w0 = cb.q[2 * (s >> 1)] >> sh;
                w1 = cb.q[2 * (s >> 1) + 1] >> sh;
                bq[s] = __builtin_bit_cast(
                    half8, u32x4{mm_qs(w0, sc2), mm_qs(w0 >> 8, sc2), mm_qs(w1, sc2),
                                 mm_qs(w1 >> 8, sc2)});
            } else {
                w0 = cb.q[s];
                bq[s] = __builtin_bit_cast(
                    half8, u32x4{mm_qs(w0, sc2), mm_qs(w0 >> 4, sc2), mm_qs(w0 >> 8, sc2),
                                 mm_qs(w0 >> 12, sc2)});
            }
        }
        half8 bm;
#pragma unroll
        for (int s = 0; s < 8; ++s) bm[s] = j == 0 ? (_Float16)mnf[s] : (_Float16)0.0f;
        const float d24 = hdr_d(cb.hdr) * 16777216.0f, dm = hdr_dmin(cb.hdr);
        const u32x4* xb = xl + buf * kBuf + lane;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            floatx4 D = {0.f, 0.f, 0.f, 0.f}, Dm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8 a = __builtin_bit_cast(half8, xb[(nt * 10 + s) * 64]);
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[s], D, 0, 0, 0);
            }
            const half8 ah = __builtin_bit_cast(half8, xb[(nt * 10 + 8) * 64]);
            const half8 al = __builtin_bit_cast(half8, xb[(nt * 10 + 9) * 64]);
            Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bm, Dm, 0, 0, 0);
            Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bm, Dm, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][i] += d24 * D[i] - dm * Dm[i];
        }
    };
    // the range's super-blocks, two at a time (named buffers keep both in registers); X and
    // W of the next super-block are loaded while this one is multiplied
    Blk ba, bb;
    u32x4 xa[NT], xb2[NT];
    if (b0 < b1) {
        stage_load(b0, xa);
        load_blk(b0, ba);
        stage_store(0, xa);
    }
    __syncthreads();
    for (int b = b0; b < b1; b += 2) {
        if (b + 1 < b1) {
            stage_load(b + 1, xb2);
            load_blk(b + 1, bb);
        }
        compute(0, ba);
        if (b + 1 < b1) stage_store(1, xb2);
        __syncthreads();
        if (b + 1 >= b1) break;
        if (b + 2 < b1) {
            stage_load(b + 2, xa);
            load_blk(b + 2, ba);
        }
        compute(1, bb);
        if (b + 2 < b1) stage_store(0, xa);
        __syncthreads();
    }
    // D tile: this lane holds columns 4 j + i of its row rl
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int r = r0 + rl;
        if (r >= R) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + nt * 16 + 4 * j + i;
            if (n < M)
                __hip_atomic_fetch_add(Y + (size_t)n * R + r, acc[nt][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------- dequant to fp32

template <int ORDER>
__global__ __launch_bounds__(kThreads) void q4k_dequant_kernel(const uint8_t* __restrict__ W,
                                                               size_t nblocks,
                                                               float* __restrict__ out) {
    const size_t total = nblocks * 256;
    for (size_t g = (size_t)blockIdx.x * kThreads + threadIdx.x; g < total;
         g += (size_t)gridDim.x * kThreads) {
        const size_t blk = g >> 8;
        const int e = (int)(g & 255);
        const uint8_t* bp = W + blk * kBlockBytes;
        const u32x4 hdr = *reinterpret_cast<const u32x4*>(bp);
        const int sb = e >> 5;
        float sc, m;
        scale_min(hdr, sb, sc, m);
        uint32_t q;
        if (ORDER == 0) {
            const uint8_t byte = bp[16 + (sb >> 1) * 32 + (e & 31)];
            q = (sb & 1) ? (byte >> 4) : (byte & 0xFu);
        } else {
            const uint8_t byte = bp[16 + e / 2];
            q = (e & 1) ? (byte >> 4) : (byte & 0xFu);
        }
        // same expression order as the reference: (d*sc)*q - (dmin*m)
        out[g] = (hdr_d(hdr) * sc) * (float)q - hdr_dmin(hdr) * m;
    }
}

int check_w(const void* w, int R, int C, int order) {
    if (!w || R <= 0 || C <= 0) return set_error(CSDR_E_INVALID, "q4k: bad W argument");
    if (C % 256) return set_error(CSDR_E_INVALID, "q4k: C must be a multiple of 256");
    if (order != CSDR_Q4K_GGML && order != CSDR_Q4K_INTERLEAVED)
        return set_error(CSDR_E_INVALID, "q4k: unknown element order");
    if (reinterpret_cast<uintptr_t>(w) % 16)
        return set_error(CSDR_E_INVALID, "q4k: W must be 16-byte aligned");
    return CSDR_OK;
}

}  // namespace

extern "C" {

CSDR_API int csdr_q4k_linear(const void* w, int R, int C, int order, const void* x, int x_dtype,
                             int M, float* y, void* hip_stream) {
    int rc = check_w(w, R, C, order);
    if (rc) return rc;
    if (!x || !y || M <= 0) return set_error(CSDR_E_INVALID, "q4k_linear: bad x/y/M");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const int nblk = C / 256;
    if (M == 1) {
        // rows per wave: one round of at most 256 workgroups (one per CU) of 16 waves
        const int rpw = (R + 16 * 256 - 1) / (16 * 256);
        const int grid = (R + kGvWaves * rpw - 1) / (kGvWaves * rpw);
        if (reinterpret_cast<uintptr_t>(x) % 16)
            return set_error(CSDR_E_INVALID, "q4k_linear: x must be 16-byte aligned");
        // a wave's rows (and the steps it loads past them) are addressed with 32-bit offsets
        if ((size_t)(rpw + 4) * nblk * kBlockBytes >= ((size_t)1 << 31))
            return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: rows too long for M = 1");
        const auto* wp = static_cast<const uint8_t*>(w);
        auto go = [&](auto kern, size_t lds, const auto* xp) -> int {
            if (lds > 160 * 1024) return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: C too large");
            if (lds > 64 * 1024)
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            kern<<<grid, kGvThreads, lds, st>>>(wp, R, nblk, xp, y, rpw);
            return CSDR_OK;
        };
        const int ring = gv_ring_for((nblk + 15) / 16);
        auto pick = [&](auto ord, auto xt) -> int {
            constexpr int O = decltype(ord)::value;
            using XT = typename decltype(xt)::type;
            const auto* xp = static_cast<const XT*>(x);
            const size_t lds = gv_lds_bytes<XT>(nblk);
            return ring == 1 ? go(q4k_gemv_kernel<O, XT, 1>, lds, xp)
                             : go(q4k_gemv_kernel<O, XT, 2>, lds, xp);
        };
        using G = std::integral_constant<int, 0>;
        using I = std::integral_constant<int, 1>;
        if (x_dtype == CSDR_F16) {
            using H = TypeTag<_Float16>;
            rc = order == CSDR_Q4K_GGML ? pick(G{}, H{}) : pick(I{}, H{});
        } else if (x_dtype == CSDR_F32) {
            using F = TypeTag<float>;
            rc = order == CSDR_Q4K_GGML ? pick(G{}, F{}) : pick(I{}, F{});
        } else {
            return set_error(CSDR_E_INVALID, "q4k_linear: x_dtype must be CSDR_F32 or CSDR_F16");
        }
        if (rc) return rc;
    } else {
        if (x_dtype != CSDR_F16)
            return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: M > 1 takes fp16 x");
        if (reinterpret_cast<uintptr_t>(x) % 16 || C % 8)
            return set_error(CSDR_E_INVALID, "q4k_linear: x must be 16-byte aligned");
        // Y = 0, then the split-K tiles add into it
        const size_t ny = (size_t)M * R;
        fill_zero_kernel<<<(unsigned)std::min<size_t>((ny + kThreads - 1) / kThreads, 4096),
                           kThreads, 0, st>>>(y, ny);
        // 128-row workgroups, 16 NT columns each, and the super-blocks split so that the grid
        // holds about 256 workgroups
        const int NT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        const int gx = (R + kMmRows - 1) / kMmRows, gz = (M + 16 * NT - 1) / (16 * NT);
        const int pk = std::max(1, std::min(nblk, (256 + gx * gz - 1) / (gx * gz)));
        const int KB = (nblk + pk - 1) / pk;
        dim3 grid(gx, (nblk + KB - 1) / KB, gz);
        const size_t lds = (size_t)2 * 10 * 64 * 16 * NT;
        const auto* wp = static_cast<const uint8_t*>(w);
        const auto* xp = static_cast<const _Float16*>(x);
        auto go = [&](auto kern) {
            if (lds > 64 * 1024)
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            kern<<<grid, kMmThreads, lds, st>>>(wp, R, nblk, xp, M, y, KB);
        };
        auto pick = [&](auto ord) {
            constexpr int O = decltype(ord)::value;
            if (NT == 1) go(q4k_mm_kernel<O, 1>);
            else if (NT == 2) go(q4k_mm_kernel<O, 2>);
            else go(q4k_mm_kernel<O, 4>);
        };
        if (order == CSDR_Q4K_GGML) pick(std::integral_constant<int, 0>{});
        else pick(std::integral_constant<int, 1>{});
    }
    CSDR_LAUNCH_CHECK("q4k_linear");
    return CSDR_OK;
}

CSDR_API int csdr_q4k_dequant(const void* w, size_t n_blocks, int order, float* out,
                              void* hip_stream) {
    if (!w || !out) return set_error(CSDR_E_INVALID, "q4k_dequant: null argument");
    if (order != CSDR_Q4K_GGML && order != CSDR_Q4K_INTERLEAVED)
        return set_error(CSDR_E_INVALID, "q4k_dequant: unknown element order");
    if (reinterpret_cast<uintptr_t>(w) % 16)
        return set_error(CSDR_E_INVALID, "q4k_dequant: W must be 16-byte aligned");
    if (n_blocks == 0) return CSDR_OK;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const size_t total = n_blocks * 256;
    const int grid = (int)std::min<size_t>((total + kThreads - 1) / kThreads, 65536);
    if (order == CSDR_Q4K_GGML)
        q4k_dequant_kernel<0><<<grid, kThreads, 0, st>>>(static_cast<const uint8_t*>(w), n_blocks, out);
    else
        q4k_dequant_kernel<1><<<grid, kThreads, 0, st>>>(static_cast<const uint8_t*>(w), n_blocks, out);
    CSDR_LAUNCH_CHECK("q4k_dequant");
    return CSDR_OK;
}

}  // extern "C"
