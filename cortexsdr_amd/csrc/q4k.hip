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
//   q4k_mm_kernel (M > 1): 8 waves own 32 rows, up to 64 columns and a range of
//     super-blocks (split K in at most 8 parts, each on its own XCDs). Wave w takes quant
//     group w % 4 of every other super-block; per super-block a lane forms q * sc for 8 values
//     of each of its two sub-blocks as exact fp16 subnormals, and v_mfma_f32_16x16x32_f16
//     multiplies them with fp16 X (loaded straight into the A operands in the matching k
//     order) into an fp32 tile scaled by d; the dmin * m term is a second small product with
//     the sub-block sums of X. No rounding of W: the product is within about 1e-6 (relative
//     L2) of fp32. The waves' tiles meet in LDS and each output is written once per split.
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
// A workgroup of 8 waves owns 64 rows (four 16-row tiles), 16 NT columns and a range of
// super-blocks (split K in S parts, S in {1, 2, 4, 8}). Wave w takes row tile w / 2 and half
// w % 2 of every super-block (sub-blocks 4h .. 4h + 3) and multiplies on
// v_mfma_f32_16x16x32_f16 with W as the B operand (k x rows) and X as A (columns x k), so each
// output element a lane holds belongs to the lane's own W row:
//   * a lane (row rl = l % 16, k-slice j = l / 16) takes the 8 values 8j .. 8j + 7 of each of
//     its sub-blocks in element order: the nibbles are split with two masks and paired with
//     v_perm_b32, and q * sc (at most 15 * 63 = 945) is formed as a pair of 16-bit integers
//     with one v_pk_mul_lo_u16 and read as two fp16 subnormals q * sc * 2^-24, exact;
//   * the min term sum_s m_s * (sum of x over s) is a second product with m_s (6-bit) in every
//     k position, also as subnormals m_s * 2^-24, so no sums of X are formed;
//   * per super-block: acc += (d * 2^24) * D - (dmin * 2^24) * Dm in fp32.
// X moves through LDS in memory order (plain 16-byte copies into tiles laid out as the A
// operands are read), in a ring of two buffers fed from kMmXR register sets, so each copy has
// kMmXR super-blocks' time to land; W runs kMmWD super-blocks ahead in registers. One barrier
// per super-block. The halves' tiles meet in LDS at the end and each output is written once per
// split: stored when S = 1, else added into Y (zeroed first).
//
// Placement: workgroup i runs on XCD i % 8. Split h of every row tile goes to the XCDs with
// xcd % S == h, so an XCD fetches 1/S of X into its L2.
constexpr int kMmWaves = 8;
constexpr int kMmThreads = 64 * kMmWaves;
constexpr int kMmRows = 64;
// W super-blocks in flight per wave and X super-blocks per thread (register sets). Measured at
// 4096 x 14336, M = 32 (us): 24.4 here, 25.8 with 4 X sets, 26.5 with 6, 27.0 with 4 W; the
// split count the same way: 39.3 with S = 2, 30.4 with S = 8 against S = 4 here.
constexpr int kMmWD = 2;
constexpr int kMmXR = 2;
constexpr int kMmUnroll = 2;  // a multiple of 2 (buffers), kMmWD and kMmXR

// q4k_mm_kernel's placement: nrt row tiles (padded to nrt_p, a multiple of 8 / S), S splits of
// KB super-blocks, column groups of 16 NT outer
struct MmGrid {
    int nrt, nrt_p, S, KB;
};

// LDS bytes of one X buffer: NT column tiles x 8 sub-blocks x 64 lanes x 16 bytes
template <int NT>
constexpr int mm_xbuf_bytes() {
    return NT * 8 * 64 * 16;
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// four (value, value) nibble pairs p0..p3 (values at bits 0-3 and 16-19) times the sub-block
// scale: 8 fp16 subnormals q * sc * 2^-24
__device__ __forceinline__ half8 mm_scale(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3,
                                          uint32_t sc2) {
    const u16x2 s = __builtin_bit_cast(u16x2, sc2);
    const u32x4 v = {__builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p0) * s),
                     __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p1) * s),
                     __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p2) * s),
                     __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p3) * s)};
    return __builtin_bit_cast(half8, v);
}

// the 4 scales and 4 mins of sub-blocks 4h .. 4h + 3 (h uniform across the wave), one per
// byte, from the 12 scale bytes (header words y, z, w), as scale_min unpacks them one at a time
__device__ __forceinline__ void scale_min_quad(const u32x4& hdr, int h, uint32_t& sc4,
                                               uint32_t& mn4) {
    if (h == 0) {
        sc4 = hdr.y & 0x3F3F3F3Fu;
        mn4 = hdr.z & 0x3F3F3F3Fu;
    } else {
        sc4 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        mn4 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    }
}

template <int ORDER, int NT>
__global__ __launch_bounds__(kMmThreads) void q4k_mm_kernel(const uint8_t* __restrict__ W, int R,
                                                            int nblk, const _Float16* __restrict__ X,
                                                            int M, float* __restrict__ Y, MmGrid g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char mm_smem[];
    u32x4* xl = reinterpret_cast<u32x4*>(mm_smem);  // [2 buffers][NT * 8 tiles][64 lanes]
    constexpr int kBuf = NT * 8 * 64;               // u32x4 per buffer
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int rt = wave >> 1, half = wave & 1;
    const int rl = lane & 15, j = lane >> 4;
    // the workgroup's tile from its number (number % 8 is the XCD it runs on)
    const int per_z = g.nrt_p * g.S;
    const int z = (int)blockIdx.x / per_z, rest = (int)blockIdx.x - z * per_z;
    const int xcd = rest & 7;
    const int sp = xcd % g.S;
    const int t = (rest >> 3) * (8 / g.S) + xcd / g.S;
    const int b0 = sp * g.KB, b1 = min(nblk, b0 + g.KB);
    if (t >= g.nrt || b0 >= b1) return;  // padding or an empty split (the whole workgroup)
    const int nb = b1 - b0;
    const int r0 = t * kMmRows, n0 = z * 16 * NT;
    const int C = nblk * 256;
    const uint8_t* wrow = W + (size_t)min(r0 + 16 * rt + rl, R - 1) * nblk * kBlockBytes;
    // X staging: pieces q = i * kMmThreads + tid, i < NT: tile q / 64 = (column tile, sub-block),
    // lane q % 64 = (column c, k-slice j); 16 bytes each
    const _Float16* xsrc[NT];
    bool xlive[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int q = i * kMmThreads + (int)threadIdx.x;
        const int tile = q >> 6, ln = q & 63;
        const int n = n0 + 16 * (tile >> 3) + (ln & 15);
        xlive[i] = n < M;
        xsrc[i] = X + (size_t)min(n, M - 1) * C + 32 * (tile & 7) + 8 * (ln >> 4);
    }
    auto xload = [&](int k, u32x4 (&xr)[NT]) {
        const int b = b0 + min(k, nb - 1);
#pragma unroll
        for (int i = 0; i < NT; ++i) xr[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + (size_t)b * 256);
    };
    auto xstore = [&](int buf, const u32x4 (&xr)[NT]) {
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < NT; ++i) xl[buf * kBuf + i * kMmThreads + threadIdx.x] = xlive[i] ? xr[i] : zero;
    };
    // a super-block's W for this lane: the header and the quant bytes of its 4 sub-blocks
    struct Wq {
        u32x4 hdr;
        uint32_t q[4];
    };
    auto wload = [&](int k, Wq& o) {
        const uint8_t* bp = wrow + (size_t)(b0 + min(k, nb - 1)) * kBlockBytes;
        o.hdr = *reinterpret_cast<const u32x4*>(bp);
        if (ORDER == 0) {
            // groups 2h, 2h + 1: bytes 8j .. 8j + 7 of each (low nibbles: sub-block 2g, high: 2g+1)
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const uint2 v = *reinterpret_cast<const uint2*>(bp + 16 + 32 * (2 * half + gi) + 8 * j);
                o.q[2 * gi] = v.x;
                o.q[2 * gi + 1] = v.y;
            }
        } else {
            // sub-blocks 4h .. 4h + 3: bytes 4j .. 4j + 3 of each (two values per byte)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                o.q[u] = *reinterpret_cast<const uint32_t*>(bp + 16 + 16 * (4 * half + u) + 4 * j);
        }
    };
    floatx4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const Wq& w) {
        uint32_t sc4, mn4;
        scale_min_quad(w.hdr, half, sc4, mn4);
        floatx4 D[NT], Dm[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            D[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
            Dm[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // sub-block 4h + u: the scale and min of byte u in both 16-bit lanes
            const uint32_t sel = 0x0c000c00u + 0x00010001u * (uint32_t)u;
            const uint32_t sc2 = __builtin_amdgcn_perm(sc4, sc4, sel);
            const uint32_t m2 = __builtin_amdgcn_perm(mn4, mn4, sel);
            half8 bq;
            if (ORDER == 0) {
                // group 2h + u / 2, nibble u % 2 of its 8 bytes
                const int sh = 4 * (u & 1);
                const uint32_t ta = (w.q[2 * (u >> 1)] >> sh) & 0x0F0F0F0Fu;
                const uint32_t tb = (w.q[2 * (u >> 1) + 1] >> sh) & 0x0F0F0F0Fu;
                bq = mm_scale(__builtin_amdgcn_perm(ta, ta, 0x0c010c00u),
                              __builtin_amdgcn_perm(ta, ta, 0x0c030c02u),
                              __builtin_amdgcn_perm(tb, tb, 0x0c010c00u),
                              __builtin_amdgcn_perm(tb, tb, 0x0c030c02u), sc2);
            } else {
                // value 2i: low nibble of byte i; 2i + 1: its high nibble
                const uint32_t lo = w.q[u] & 0x0F0F0F0Fu, hi = (w.q[u] >> 4) & 0x0F0F0F0Fu;
                bq = mm_scale(__builtin_amdgcn_perm(hi, lo, 0x0c040c00u),
                              __builtin_amdgcn_perm(hi, lo, 0x0c050c01u),
                              __builtin_amdgcn_perm(hi, lo, 0x0c060c02u),
                              __builtin_amdgcn_perm(hi, lo, 0x0c070c03u), sc2);
            }
            const half8 bm = __builtin_bit_cast(half8, u32x4{m2, m2, m2, m2});
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const half8 a = __builtin_bit_cast(half8, xl[buf * kBuf + (nt * 8 + 4 * half + u) * 64 + lane]);
                D[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq, D[nt], 0, 0, 0);
                Dm[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bm, Dm[nt], 0, 0, 0);
            }
        }
        const float d24 = hdr_d(w.hdr) * 16777216.0f, dm24 = hdr_dmin(w.hdr) * 16777216.0f;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][i] += d24 * D[nt][i] - dm24 * Dm[nt][i];
    };
    // prologue: X of super-blocks 0 .. kMmXR - 1 in the register sets, 0 stored into buffer 0
    // and kMmXR loaded in its place; W 0 .. kMmWD - 1 (every load is issued, past the end as a
    // repeat of the last super-block, so that the compiler's wait counts stay exact)
    u32x4 xr[kMmXR][NT];
    Wq wr[kMmWD];
#pragma unroll
    for (int s = 0; s < kMmXR; ++s) xload(s, xr[s]);
#pragma unroll
    for (int k = 0; k < kMmWD; ++k) wload(k, wr[k]);
    xstore(0, xr[0]);
    xload(kMmXR, xr[0]);
    __syncthreads();
    // iteration k: multiply super-block k from buffer k % 2; store X(k + 1) from its register
    // set into the other buffer (last read in iteration k - 1, before its barrier) and load
    // X(k + 1 + kMmXR) into that set, so every X load has kMmXR iterations to land
    static_assert(kMmUnroll % 2 == 0 && kMmUnroll % kMmWD == 0 && kMmUnroll % kMmXR == 0, "");
    for (int k0 = 0; k0 < nb; k0 += kMmUnroll) {
#pragma unroll
        for (int u = 0; u < kMmUnroll; ++u) {
            const int k = k0 + u;
            if (k >= nb) break;
            compute(u & 1, wr[u % kMmWD]);
            wload(k + kMmWD, wr[u % kMmWD]);
            xstore((u + 1) & 1, xr[(u + 1) % kMmXR]);
            xload(k + 1 + kMmXR, xr[(u + 1) % kMmXR]);
            __syncthreads();
        }
    }
    // the halves' tiles: half 1 parks its tile in LDS (after the last barrier no wave reads X),
    // half 0 adds it and writes the outputs; lane (rl, j) holds row rl, columns 4j .. 4j + 3
    floatx4* red = reinterpret_cast<floatx4*>(mm_smem);  // [4 row tiles][NT][64 lanes]
    if (half == 1) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) red[(rt * NT + nt) * 64 + lane] = acc[nt];
    }
    __syncthreads();
    if (half == 0) {
        const int row = r0 + 16 * rt + rl;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const floatx4 v = acc[nt] + red[(rt * NT + nt) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int col = n0 + 16 * nt + 4 * j + i;
                if (row < R && col < M) {
                    float* yp = Y + (size_t)col * R + row;
                    if (g.S == 1)
                        *yp = v[i];
                    else
                        __hip_atomic_fetch_add(yp, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
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
        // 64-row tiles of up to 64 columns; the super-blocks split in S parts (S a power of
        // two up to 8) so that the grid holds at least 256 workgroups where the row tiles
        // alone do not
        const int NT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        const int gz = (M + 16 * NT - 1) / (16 * NT);
        MmGrid g;
        g.nrt = (R + kMmRows - 1) / kMmRows;
        g.S = 1;
        while (g.S < 8 && g.S < nblk && (long long)g.nrt * g.S * gz < 256) g.S *= 2;
        g.KB = (nblk + g.S - 1) / g.S;
        const int pad = 8 / g.S;
        g.nrt_p = (g.nrt + pad - 1) / pad * pad;
        const long long nwg = (long long)g.nrt_p * g.S * gz;
        if (nwg > 0x7fffffffLL)
            return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: too many output tiles");
        if (g.S > 1) {
            // Y = 0, then the splits add into it
            const size_t ny = (size_t)M * R;
            fill_zero_kernel<<<(unsigned)std::min<size_t>((ny + kThreads - 1) / kThreads, 4096),
                               kThreads, 0, st>>>(y, ny);
        }
        const auto* wp = static_cast<const uint8_t*>(w);
        const auto* xp = static_cast<const _Float16*>(x);
        auto go = [&](auto kern, size_t lds) {
            if (lds > 64 * 1024)
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            kern<<<(unsigned)nwg, kMmThreads, lds, st>>>(wp, R, nblk, xp, M, y, g);
        };
        auto pick = [&](auto ord) {
            constexpr int O = decltype(ord)::value;
            if (NT == 1) go(q4k_mm_kernel<O, 1>, 2 * mm_xbuf_bytes<1>());
            else if (NT == 2) go(q4k_mm_kernel<O, 2>, 2 * mm_xbuf_bytes<2>());
            else go(q4k_mm_kernel<O, 4>, 2 * mm_xbuf_bytes<4>());
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
