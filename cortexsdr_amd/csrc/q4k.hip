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
//   q4k_gemv_kernel (M == 1): one wave per row. Every lane takes one 16-byte piece of a
//     super-block's quants plus the block header (the 8 lanes of a block read the same 16
//     header bytes), so a wave load instruction covers 8 whole blocks. x is staged in LDS.
//     Per piece: y += d*sc*(sum q*x) - dmin*m*(sum x) in fp32 (q stays an exact integer).
//   q4k_mm_kernel (M > 1): a workgroup owns 16 RT rows and a range of super-blocks (split K);
//     each wave holds RT 16-row tiles and takes every 4th super-block of the range (the next
//     one's loads issued before the current one is multiplied). Per
//     32-element sub-block a lane dequantises its 8 values of each row tile in fp32
//     ((d*sc)*q - dmin*m, one fused multiply-add) and rounds them to fp16 once, and each
//     16-column tile of X (fp16, read straight into the B operand, 16 bytes per lane) takes
//     one v_mfma_f32_16x16x32_f16 (fp32 accumulate). The waves' tiles are summed through LDS
//     and added into Y (zeroed by a fill launch) with one atomic per output per workgroup.
//     The single fp16 rounding of W puts the product about 3e-4 (relative L2) from fp32.
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
constexpr int kUnroll = 4;  // 8-block steps per wave issued back to back (gemv)

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

// x (C elements, C % 256 == 0, 16-byte aligned) -> LDS in 16-byte pieces, up to 8 pieces
// per thread in flight per batch (one batch covers C <= 64K fp16 / 32K fp32 values).
template <typename XT>
__device__ __forceinline__ void stage_x(const XT* __restrict__ x, int C, XT* xs) {
    const u32x4* src = reinterpret_cast<const u32x4*>(x);
    u32x4* dst = reinterpret_cast<u32x4*>(xs);
    const int n16 = C * (int)sizeof(XT) / 16;
    for (int i0 = 0; i0 < n16; i0 += kThreads * 8) {
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[min(i0 + j * kThreads + (int)threadIdx.x, n16 - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * kThreads + threadIdx.x;
            if (i < n16) dst[i] = v[j];
        }
    }
}

// sum over 16 consecutive x values of q_i * x_i (q = nibble NIB of byte i of `q`) and of x_i
template <typename XT, int NIB>
__device__ __forceinline__ void dot16(const u32x4& q, const XT* xp, float& sq, float& sx) {
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float xv = csdr::to_f32(xp[wi * 4 + b]);
            const float qv = (float)((w4[wi] >> (8 * b + 4 * NIB)) & 0xFu);
            sq = fmaf(qv, xv, sq);
            sx += xv;
        }
}

// 32 interleaved values: byte i -> elements 2i (low nibble), 2i+1 (high nibble)
template <typename XT>
__device__ __forceinline__ void dot32i(const u32x4& q, const XT* xp, float& sq, float& sx) {
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int i = wi * 4 + b;
            const float x0 = csdr::to_f32(xp[2 * i]), x1 = csdr::to_f32(xp[2 * i + 1]);
            const uint32_t byte = (w4[wi] >> (8 * b)) & 0xFFu;
            sq = fmaf((float)(byte & 0xFu), x0, sq);
            sq = fmaf((float)(byte >> 4), x1, sq);
            sx += x0 + x1;
        }
}

template <int ORDER, typename XT>
__global__ __launch_bounds__(kThreads) void q4k_gemv_kernel(const uint8_t* __restrict__ W, int R,
                                                            int nblk, const XT* __restrict__ x,
                                                            float* __restrict__ y,
                                                            int rows_per_wave) {
    extern __shared__ unsigned char smem_raw[];
    XT* xs = reinterpret_cast<XT*>(smem_raw);
    const int C = nblk * 256;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int piece = lane & 7;  // which 16 bytes of the block's quants
    const int bl = lane >> 3;    // which of the 8 blocks of a step
    const int row0 = (blockIdx.x * (kThreads / 64) + wave) * rows_per_wave;
    auto load_step = [&](int r, int b0, u32x4 (&hdr)[kUnroll], u32x4 (&qs)[kUnroll]) {
        const uint8_t* rowp = W + (size_t)min(r, R - 1) * nblk * kBlockBytes;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int blk = min(b0 + u * 8 + bl, nblk - 1);
            const u32x4* bp = reinterpret_cast<const u32x4*>(rowp + (size_t)blk * kBlockBytes);
            hdr[u] = __builtin_nontemporal_load(bp);
            qs[u] = __builtin_nontemporal_load(bp + 1 + piece);
        }
    };
    // the first weight loads go out before x is staged (they overlap the staging latency)
    u32x4 hdr0[kUnroll], qs0[kUnroll];
    load_step(row0, 0, hdr0, qs0);
    stage_x(x, C, xs);
    __syncthreads();
    for (int rr = 0; rr < rows_per_wave; ++rr) {
        const int r = row0 + rr;
        if (r >= R) break;
        float acc = 0.0f;
        for (int b0 = 0; b0 < nblk; b0 += 8 * kUnroll) {
            u32x4 hdr[kUnroll], qs[kUnroll];
            if (rr == 0 && b0 == 0) {
#pragma unroll
                for (int u = 0; u < kUnroll; ++u) {
                    hdr[u] = hdr0[u];
                    qs[u] = qs0[u];
                }
            } else {
                load_step(r, b0, hdr, qs);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int blk = b0 + u * 8 + bl;
                if (blk >= nblk) continue;
                const float d = hdr_d(hdr[u]), dmin = hdr_dmin(hdr[u]);
                const XT* xb = xs + (size_t)blk * 256;
                if (ORDER == 0) {
                    const int g = piece >> 1, h = piece & 1;
                    float sc0, m0, sc1, m1;
                    scale_min(hdr[u], 2 * g, sc0, m0);
                    scale_min(hdr[u], 2 * g + 1, sc1, m1);
                    float sq0 = 0.f, sx0 = 0.f, sq1 = 0.f, sx1 = 0.f;
                    dot16<XT, 0>(qs[u], xb + 64 * g + 16 * h, sq0, sx0);
                    dot16<XT, 1>(qs[u], xb + 64 * g + 32 + 16 * h, sq1, sx1);
                    acc += (d * sc0) * sq0 - (dmin * m0) * sx0;
                    acc += (d * sc1) * sq1 - (dmin * m1) * sx1;
                } else {
                    float sc, m;
                    scale_min(hdr[u], piece, sc, m);
                    float sq = 0.f, sx = 0.f;
                    dot32i<XT>(qs[u], xb + 32 * piece, sq, sx);
                    acc += (d * sc) * sq - (dmin * m) * sx;
                }
            }
        }
        acc = csdr::wave_sum(acc);
        if (lane == 0) y[r] = acc;
    }
}

// ---------------------------------------------------------------- M > 1, split-K MFMA

// Launch shape of q4k_mm_kernel: RT 16-row tiles per wave (16 RT rows per workgroup) and KB
// super-blocks per workgroup for NT 16-column tiles. Measured on cfg3 (4096 x 4096 and
// 4096 x 14336, M = 16 / 32 / 64, including the fill launch): up to 32 columns two row tiles
// and 8 super-blocks (16 past 32 super-blocks per row): 13.5 / 32.4 us at M = 32 against
// 16.4 / 39.8 for four tiles and 4. At 64 columns four tiles and 16 super-blocks halve the
// partial-sum atomics (43.0 us at 4096 x 14336 against 57.6) while that still gives 256
// workgroups; below that (4096 x 4096: 64 workgroups, 33.3 us) two tiles and 8 (20.8 us).
void q4k_mm_shape(int R, int nblk, int NT, int& RT, int& KB) {
    RT = 2;
    KB = nblk > 32 ? 16 : 8;
    if (NT >= 4 && (size_t)((R + 63) / 64) * (size_t)((nblk + 15) / 16) >= 256) {
        RT = 4;
        KB = 16;
    }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads)
        y[i] = 0.0f;
}

// 8 quant values of sub-block s for this lane (k = 8 j .. 8 j + 7 of the sub-block, j = lane
// group) as bytes, from the block's quants (ggml: the 8-byte piece of group s / 2, low nibbles
// for even s; interleaved: the 4-byte piece of sub-block s, nibbles low / high alternating).
template <int ORDER>
__device__ __forceinline__ void quant8(const uint32_t* q, int s, uint32_t& w0, uint32_t& w1) {
    if (ORDER == 0) {
        const int sh = (s & 1) * 4;
        w0 = (q[2 * (s >> 1)] >> sh) & 0x0F0F0F0Fu;
        w1 = (q[2 * (s >> 1) + 1] >> sh) & 0x0F0F0F0Fu;
    } else {
        const uint32_t v = q[s];
        const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
        // element order lo.b0 hi.b0 lo.b1 hi.b1 | lo.b2 hi.b2 lo.b3 hi.b3 as bytes
        w0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        w1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    }
}

template <int ORDER, int NT, int RT>
__global__ __launch_bounds__(kThreads) void q4k_mm_kernel(const uint8_t* __restrict__ W, int R,
                                                          int nblk, const _Float16* __restrict__ X,
                                                          int M, float* __restrict__ Y, int KB) {
    __shared__ floatx4 red[3][RT][NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rl = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * (16 * RT);
    const int b0 = blockIdx.y * KB, b1 = min(nblk, b0 + KB);
    const int n0 = blockIdx.z * 16 * NT;
    const int C = nblk * 256;
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
    const uint8_t* wr[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        wr[rt] = W + (size_t)min(r0 + rt * 16 + rl, R - 1) * nblk * kBlockBytes;
    // a block's header and this lane's quants of every row tile
    struct Blk {
        u32x4 hdr[RT];
        uint32_t q[RT][8];
    };
    auto load_blk = [&](int blk, Blk& o) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint8_t* bp = wr[rt] + (size_t)blk * kBlockBytes;
            o.hdr[rt] = *reinterpret_cast<const u32x4*>(bp);
            if (ORDER == 0) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint2 v = *reinterpret_cast<const uint2*>(bp + 16 + 32 * g + 8 * j);
                    o.q[rt][2 * g] = v.x;
                    o.q[rt][2 * g + 1] = v.y;
                }
            } else {
#pragma unroll
                for (int sb = 0; sb < 8; ++sb)
                    o.q[rt][sb] = *reinterpret_cast<const uint32_t*>(bp + 16 + 16 * sb + 4 * j);
            }
        }
    };
    auto compute_blk = [&](int blk, const Blk& cb) {
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) {
            half8 bv[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const half8 v = *reinterpret_cast<const half8*>(xr[nt] + (size_t)blk * 256 + 32 * sb);
                bv[nt] = xl[nt] ? v : half8{};
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                float sc, mn;
                scale_min(cb.hdr[rt], sb, sc, mn);
                const float ds = hdr_d(cb.hdr[rt]) * sc, dm = hdr_dmin(cb.hdr[rt]) * mn;
                uint32_t w0, w1;
                quant8<ORDER>(cb.q[rt], sb, w0, w1);
                half8 a;
                a[0] = (_Float16)fmaf(ds, (float)((w0 >> 0) & 0xFFu), -dm);
                a[1] = (_Float16)fmaf(ds, (float)((w0 >> 8) & 0xFFu), -dm);
                a[2] = (_Float16)fmaf(ds, (float)((w0 >> 16) & 0xFFu), -dm);
                a[3] = (_Float16)fmaf(ds, (float)((w0 >> 24) & 0xFFu), -dm);
                a[4] = (_Float16)fmaf(ds, (float)((w1 >> 0) & 0xFFu), -dm);
                a[5] = (_Float16)fmaf(ds, (float)((w1 >> 8) & 0xFFu), -dm);
                a[6] = (_Float16)fmaf(ds, (float)((w1 >> 16) & 0xFFu), -dm);
                a[7] = (_Float16)fmaf(ds, (float)((w1 >> 24) & 0xFFu), -dm);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bv[nt], acc[rt][nt], 0, 0, 0);
            }
        }
    };
    // every 4th block of the range; the next block's loads go out before this one is
    // multiplied (two buffers, named, so that both stay in registers)
    int blk = b0 + wave;
    if (blk < b1) {
        Blk ba, bb;
        load_blk(blk, ba);
        for (;;) {
            const int nb1 = blk + kThreads / 64;
            if (nb1 < b1) load_blk(nb1, bb);
            compute_blk(blk, ba);
            if (nb1 >= b1) break;
            const int nb2 = nb1 + kThreads / 64;
            if (nb2 < b1) load_blk(nb2, ba);
            compute_blk(nb1, bb);
            if (nb2 >= b1) break;
            blk = nb2;
        }
    }
    // the 4 waves' tiles: waves 1..3 park theirs in LDS, wave 0 sums and adds into Y
    if (wave > 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) red[wave - 1][rt][nt][lane] = acc[rt][nt];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                floatx4 v = acc[rt][nt];
#pragma unroll
                for (int w = 0; w < 3; ++w) v += red[w][rt][nt][lane];
                // D tile: this lane holds rows 4 j + i, column rl
                const int n = n0 + nt * 16 + rl;
                if (n >= M) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = r0 + rt * 16 + 4 * j + i;
                    if (r < R)
                        __hip_atomic_fetch_add(Y + (size_t)n * R + r, v[i], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
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
        const int rpw = R >= 8192 ? 2 : 1;
        const int grid = (R + (kThreads / 64) * rpw - 1) / ((kThreads / 64) * rpw);
        if (reinterpret_cast<uintptr_t>(x) % 16)
            return set_error(CSDR_E_INVALID, "q4k_linear: x must be 16-byte aligned");
        if (x_dtype == CSDR_F16) {
            const size_t lds = (size_t)C * 2;
            if (lds > 160 * 1024) return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: C too large");
            if (order == CSDR_Q4K_GGML)
                q4k_gemv_kernel<0, _Float16><<<grid, kThreads, lds, st>>>(
                    static_cast<const uint8_t*>(w), R, nblk, static_cast<const _Float16*>(x), y, rpw);
            else
                q4k_gemv_kernel<1, _Float16><<<grid, kThreads, lds, st>>>(
                    static_cast<const uint8_t*>(w), R, nblk, static_cast<const _Float16*>(x), y, rpw);
        } else if (x_dtype == CSDR_F32) {
            const size_t lds = (size_t)C * 4;
            if (lds > 160 * 1024) return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: C too large");
            if (order == CSDR_Q4K_GGML)
                q4k_gemv_kernel<0, float><<<grid, kThreads, lds, st>>>(
                    static_cast<const uint8_t*>(w), R, nblk, static_cast<const float*>(x), y, rpw);
            else
                q4k_gemv_kernel<1, float><<<grid, kThreads, lds, st>>>(
                    static_cast<const uint8_t*>(w), R, nblk, static_cast<const float*>(x), y, rpw);
        } else {
            return set_error(CSDR_E_INVALID, "q4k_linear: x_dtype must be CSDR_F32 or CSDR_F16");
        }
    } else {
        if (x_dtype != CSDR_F16)
            return set_error(CSDR_E_UNSUPPORTED, "q4k_linear: M > 1 takes fp16 x");
        if (reinterpret_cast<uintptr_t>(x) % 16 || C % 8)
            return set_error(CSDR_E_INVALID, "q4k_linear: x must be 16-byte aligned");
        // Y = 0, then the split-K tiles add into it
        const size_t ny = (size_t)M * R;
        fill_zero_kernel<<<(unsigned)std::min<size_t>((ny + kThreads - 1) / kThreads, 4096),
                           kThreads, 0, st>>>(y, ny);
        // launch shape: row tiles per wave (RT) and super-blocks per workgroup (KB)
        const int NT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        int RT = 2, KB = 8;
        q4k_mm_shape(R, nblk, NT, RT, KB);
        dim3 grid((R + 16 * RT - 1) / (16 * RT), (nblk + KB - 1) / KB, (M + 16 * NT - 1) / (16 * NT));
        const auto* wp = static_cast<const uint8_t*>(w);
        const auto* xp = static_cast<const _Float16*>(x);
        auto go = [&](auto kern) { kern<<<grid, kThreads, 0, st>>>(wp, R, nblk, xp, M, y, KB); };
        auto pick = [&](auto ord) {
            constexpr int O = decltype(ord)::value;
            if (RT == 4) {
                if (NT == 1) go(q4k_mm_kernel<O, 1, 4>);
                else if (NT == 2) go(q4k_mm_kernel<O, 2, 4>);
                else go(q4k_mm_kernel<O, 4, 4>);
            } else {
                if (NT == 1) go(q4k_mm_kernel<O, 1, 2>);
                else if (NT == 2) go(q4k_mm_kernel<O, 2, 2>);
                else go(q4k_mm_kernel<O, 4, 2>);
            }
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
