// gemm_f32.hip — dense fp32 Y = X . W^T (+ bias, + Y) on the gfx950 matrix cores.
//
// The compute-bound form of a product: once many token rows share one weight matrix (the
// decoder's batched prefill, every projection over the prompt's M rows) the weight is decoded
// once to dense fp32 (csdr_hsdb_decompress) and multiplied here, in fp32 throughout
// (v_mfma_f32_16x16x4_f32, fp32 accumulation), so the prompt's K/V cache and hidden states
// stay within fp32 rounding of the one-token-at-a-time path. Reference layout: the dense
// fallback Kernels::linear_forward (kernels/blas_kernels.cpp:264-293), y (M x R) = x (M x C)
// . W^T, W row-major R x C.
//
// Tiling. A workgroup of 2 x 2 waves owns a (32 WR rows of W) x (32 WM token rows) tile of Y;
// each wave a (16 WR) x (16 WM) block of 16 x 16 MFMA tiles. The contraction runs in 32-deep
// stages: the W and X slices of the next stage are loaded into registers (16-byte loads, 8
// lanes per 128-byte row piece) while the current stage's are multiplied out of LDS.
// MFMA 16x16x4 f32: lane l supplies A[l % 16][k = l / 16] and B[k = l / 16][l % 16] and holds
// D[4 (l / 16) + v][l % 16]. Within a stage the k order is permuted: step s of the eight takes
// k = 8 (l / 16) + s for lane group l / 16, so each lane reads its eight A (and B) values as
// one contiguous 32-byte run; LDS rows are padded to 36 floats, which puts the 16 rows a
// 16-lane group reads on distinct banks.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
constexpr int kBK = 32;       // contraction depth per stage
constexpr int kLd = kBK + 4;  // LDS row stride (floats)

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int WR, int WM>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const float* __restrict__ W, int R,
                                                            int C, const float* __restrict__ X,
                                                            int M, float* __restrict__ Y,
                                                            const float* __restrict__ bias,
                                                            int accumulate) {
    constexpr int BR = 32 * WR, BM = 32 * WM;
    constexpr int NA = BR * (kBK / 4) / kThreads;  // 16-byte pieces per thread per stage
    constexpr int NB = BM * (kBK / 4) / kThreads;
    __shared__ __attribute__((aligned(16))) float As[BR * kLd];
    __shared__ __attribute__((aligned(16))) float Bs[BM * kLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * BR, m0 = blockIdx.y * BM;
    const int wr0 = (wave >> 1) * 16 * WR, wm0 = (wave & 1) * 16 * WM;

    floatx4 pa[NA], pb[NB];
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int e = tid + j * kThreads, row = e >> 3, k = k0 + (e & 7) * 4;
            const int r = r0 + row;
            pa[j] = (r < R && k < C) ? *reinterpret_cast<const floatx4*>(W + (size_t)r * C + k)
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int e = tid + j * kThreads, row = e >> 3, k = k0 + (e & 7) * 4;
            const int m = m0 + row;
            pb[j] = (m < M && k < C) ? *reinterpret_cast<const floatx4*>(X + (size_t)m * C + k)
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };

    floatx4 acc[WR][WM];
#pragma unroll
    for (int a = 0; a < WR; ++a)
#pragma unroll
        for (int b = 0; b < WM; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int nst = (C + kBK - 1) / kBK;
    load(0);
    for (int st = 0; st < nst; ++st) {
        __syncthreads();  // the previous stage's LDS reads are done
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int e = tid + j * kThreads;
            *reinterpret_cast<floatx4*>(As + (e >> 3) * kLd + (e & 7) * 4) = pa[j];
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int e = tid + j * kThreads;
            *reinterpret_cast<floatx4*>(Bs + (e >> 3) * kLd + (e & 7) * 4) = pb[j];
        }
        __syncthreads();
        if (st + 1 < nst) load((st + 1) * kBK);  // in flight during this stage's MFMAs
        floatx4 af[WR][2], bf[WM][2];
#pragma unroll
        for (int a = 0; a < WR; ++a) {
            const float* p = As + (wr0 + a * 16 + li) * kLd + lg * 8;
            af[a][0] = *reinterpret_cast<const floatx4*>(p);
            af[a][1] = *reinterpret_cast<const floatx4*>(p + 4);
        }
#pragma unroll
        for (int b = 0; b < WM; ++b) {
            const float* p = Bs + (wm0 + b * 16 + li) * kLd + lg * 8;
            bf[b][0] = *reinterpret_cast<const floatx4*>(p);
            bf[b][1] = *reinterpret_cast<const floatx4*>(p + 4);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int a = 0; a < WR; ++a)
#pragma unroll
                for (int b = 0; b < WM; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        af[a][s >> 2][s & 3], bf[b][s >> 2][s & 3], acc[a][b], 0, 0, 0);
    }

    // lane holds Y[m][r .. r + 3] (W rows along the MFMA's D rows)
#pragma unroll
    for (int b = 0; b < WM; ++b) {
        const int m = m0 + wm0 + b * 16 + li;
        if (m >= M) continue;
        float* yr = Y + (size_t)m * R;
#pragma unroll
        for (int a = 0; a < WR; ++a) {
            const int r = r0 + wr0 + a * 16 + 4 * lg;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (r + v >= R) continue;
                float val = acc[a][b][v];
                if (bias) val += bias[r + v];
                if (accumulate) val += yr[r + v];
                yr[r + v] = val;
            }
        }
    }
}

// Small-M form (and any shape the tiled kernel does not take): one wave per W row, lanes
// striding over the input features, fp32 sums reduced across the wave.
__global__ __launch_bounds__(kThreads) void dense_rows_kernel(const float* __restrict__ W, int R,
                                                              int C, const float* __restrict__ x,
                                                              int M, float* __restrict__ y,
                                                              const float* __restrict__ bias,
                                                              int accumulate) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (r >= R) return;
    const float* w = W + (size_t)r * C;
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (size_t)m * C;
        float acc = 0.0f;
        for (int c = lane; c < C; c += 64) acc = fmaf(w[c], xm[c], acc);
        acc = csdr::wave_sum(acc);
        if (lane == 0) {
            if (bias) acc += bias[r];
            if (accumulate) acc += y[(size_t)m * R + r];
            y[(size_t)m * R + r] = acc;
        }
    }
}

constexpr int kMinTiledM = 8;  // below this the row-per-wave kernel reads W once for all M

}  // namespace

extern "C" {

CSDR_API int csdr_dense_linear_ex(const float* w, int R, int C, const float* x, int M, float* y,
                                  const float* bias, int flags, void* hip_stream) {
    if (!w || !x || !y || R <= 0 || C <= 0 || M <= 0)
        return set_error(CSDR_E_INVALID, "dense_linear: bad argument");
    if (flags & ~CSDR_HSDB_ACCUMULATE)
        return set_error(CSDR_E_INVALID, "dense_linear: unknown flag");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const int acc = (flags & CSDR_HSDB_ACCUMULATE) ? 1 : 0;
    const bool tiled = M >= kMinTiledM && C % 4 == 0 &&
                       reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (tiled) {
        // 64 x 64 tiles when they still give every CU a workgroup, else 32 x 32
        const long long big = (long long)((R + 63) / 64) * ((M + 63) / 64);
        if (big >= 256) {
            dim3 grid((R + 63) / 64, (M + 63) / 64);
            gemm_f32_kernel<2, 2><<<grid, kThreads, 0, st>>>(w, R, C, x, M, y, bias, acc);
        } else {
            dim3 grid((R + 31) / 32, (M + 31) / 32);
            gemm_f32_kernel<1, 1><<<grid, kThreads, 0, st>>>(w, R, C, x, M, y, bias, acc);
        }
    } else {
        const int rows_per_block = kThreads / 64;
        dense_rows_kernel<<<(R + rows_per_block - 1) / rows_per_block, kThreads, 0, st>>>(
            w, R, C, x, M, y, bias, acc);
    }
    CSDR_LAUNCH_CHECK("dense_linear");
    return CSDR_OK;
}

CSDR_API int csdr_dense_linear(const float* w, int R, int C, const float* x, int M, float* y,
                               void* hip_stream) {
    return csdr_dense_linear_ex(w, R, C, x, M, y, nullptr, 0, hip_stream);
}

}  // extern "C"
