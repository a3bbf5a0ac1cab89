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
//   q4k_mfma_kernel (M > 1): 16 rows per workgroup, the 4 waves split the super-blocks; each
//     16-wide k step dequantises 4 values per lane in fp32, splits them into fp16 hi + lo and
//     issues two v_mfma_f32_16x16x16f16 per 16 output columns (fp32 accumulate), then the
//     waves' partial tiles are summed through LDS.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
constexpr int kBlockBytes = 144;
constexpr int kUnroll = 4;  // 8-block steps per wave issued back to back (gemv)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
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

// ---------------------------------------------------------------- M > 1 (MFMA)

constexpr int kMaxNT = 4;  // up to 64 output columns per launch slice (grid.y covers more)

template <int ORDER>
__global__ __launch_bounds__(kThreads) void q4k_mfma_kernel(const uint8_t* __restrict__ W, int R,
                                                            int nblk,
                                                            const _Float16* __restrict__ X,
                                                            int M, float* __restrict__ Y) {
    __shared__ floatx4 red[3][kMaxNT][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 16;
    const int n0 = blockIdx.y * 16 * kMaxNT;
    const int C = nblk * 256;
    const int arow = min(r0 + (lane & 15), R - 1);  // A operand row of this lane
    const int kq = lane >> 4;                        // 4-value k quad within a 16-k step
    const uint8_t* rowp = W + (size_t)arow * nblk * kBlockBytes;
    floatx4 acc[kMaxNT];
#pragma unroll
    for (int t = 0; t < kMaxNT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    int nt_live = min(kMaxNT, (M - n0 + 15) / 16);

    for (int blk = wave; blk < nblk; blk += kThreads / 64) {
        const uint8_t* bp = rowp + (size_t)blk * kBlockBytes;
        const u32x4 hdr = *reinterpret_cast<const u32x4*>(bp);
        const float d = hdr_d(hdr), dmin = hdr_dmin(hdr);
        for (int sb = 0; sb < 8; ++sb) {
            float sc, m;
            scale_min(hdr, sb, sc, m);
            const float ds = d * sc, dm = dmin * m;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int e0 = sb * 32 + kk * 16 + kq * 4;  // element index in the block
                float q[4];
                if (ORDER == 0) {
                    const uint32_t v =
                        *reinterpret_cast<const uint32_t*>(bp + 16 + (sb >> 1) * 32 + (e0 & 31));
                    const int sh = (sb & 1) * 4;
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = (float)((v >> (8 * i + sh)) & 0xFu);
                } else {
                    const uint16_t v = *reinterpret_cast<const uint16_t*>(bp + 16 + e0 / 2);
                    q[0] = (float)(v & 0xFu);
                    q[1] = (float)((v >> 4) & 0xFu);
                    q[2] = (float)((v >> 8) & 0xFu);
                    q[3] = (float)((v >> 12) & 0xFu);
                }
                half4 ahi, alo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float wv = fmaf(ds, q[i], -dm);
                    const _Float16 h = (_Float16)wv;
                    ahi[i] = h;
                    alo[i] = (_Float16)(wv - (float)h);
                }
                const int kcol = blk * 256 + e0;
                for (int t = 0; t < nt_live; ++t) {
                    const int n = n0 + t * 16 + (lane & 15);
                    half4 bv = half4{0, 0, 0, 0};
                    if (n < M) bv = *reinterpret_cast<const half4*>(X + (size_t)n * C + kcol);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ahi, bv, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(alo, bv, acc[t], 0, 0, 0);
                }
            }
        }
    }
    // sum the 4 waves' tiles: waves 1..3 park theirs in LDS, wave 0 adds and stores
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
        if (reinterpret_cast<uintptr_t>(x) % 8)
            return set_error(CSDR_E_INVALID, "q4k_linear: x must be 8-byte aligned");
        dim3 grid((R + 15) / 16, (M + 16 * kMaxNT - 1) / (16 * kMaxNT));
        if (order == CSDR_Q4K_GGML)
            q4k_mfma_kernel<0><<<grid, kThreads, 0, st>>>(static_cast<const uint8_t*>(w), R, nblk,
                                                         static_cast<const _Float16*>(x), M, y);
        else
            q4k_mfma_kernel<1><<<grid, kThreads, 0, st>>>(static_cast<const uint8_t*>(w), R, nblk,
                                                         static_cast<const _Float16*>(x), M, y);
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
