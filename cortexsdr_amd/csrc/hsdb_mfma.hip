// hsdb_mfma.hip — batched (M >= 2) block-coded product Y = W.X on gfx950 matrix cores.
//
// Path (cortexSDR tree): HierarchicalSDRStrategy::matmulRowMajor with batch > 1
// (strategies/HierarchicalSDRStrategy.cpp:1257-1338), block-coded as in research
// exp_c_kernel/benchmark.py:106-130. W is never stored: each 64-column tile of a 128-row
// strip is decoded into registers straight in the MFMA A-operand layout and multiplied
// against the matching 64 x M slice of X.
//
// Decode: W[r][k] = g0 * sum_j (c_j * g_j / g0) * D[idx_j][k] over the row's slots (g0 the
// largest stage gain), with the
// dictionary held in LDS as fp16 (K <= 1024 atoms: 128 KiB): packed fp16 fused multiply-adds
// (v_pk_fma_f16, two weights per lane instruction) accumulate each lane's 16 weights of a
// row straight in the A-operand registers of the matrix-core step (v_mfma_f32_16x16x32_f16,
// fp32 accumulation; gfx950 runs it at full rate), and g0 scales the fp32 result. X is fp16 as given, or split into fp16 hi + lo parts for fp32 input (two
// MFMAs). The fp16 dictionary and the fp16 accumulation over the slots keep the product
// within ~5e-4 relative L2 of the fp32 decode (the path's bar is 1e-3).
//
// Layout. Every 64-long k range (one block column) is stored permuted (kperm64), in both the
// LDS dictionary and the transposed X, so that lane l (q = l/16) reads 16 consecutive
// positions 16q .. 16q + 15 as one contiguous 32-byte run; the block's two 32-deep MFMA steps
// take positions 16q + 8c .. + 7 (c = 0, 1) as lane group q's 8 k values in both operands
// (any common bijection of k leaves the product unchanged). The result: lane l holds rows
// 4(l/16) + i (i = 0..3) of column l % 16.
//
// Launches: an init kernel (Y = bias (+ Y when accumulating) + the fp32 edge strip times X,
// and X transposed to fp16 [m][k] with the permutation, in the workspace), then one
// persistent kernel: workgroup = 8 or 16 waves x 16 rows; the (row strip, block column) units
// of all matrices are split in contiguous ranges over the workgroups, and each strip's
// partial sums are added into Y with device-scope float atomics. A unit's X slice is staged
// in LDS by the workgroup (two barriers per unit), or, for a single 16-column tile, each wave
// loads its X operands from the workspace one unit ahead and the waves run without barriers.
// At M <= 16 with fp16 X and 4 or 8 slots the persistent kernel is the dictionary route
// instead (qroute_kernel): no weight is decoded; each unit's Q_b = D . X_b is formed on the
// matrix cores and every row gathers its slots' rows of Q_b from LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "hsdb_impl.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;  // 4 waves
constexpr int kMaxAtoms = 1024;
constexpr int kMaxMTile = 256;
constexpr int kGroup = 8;
constexpr int kMfmaMinM = 2;  // smallest batch routed to this path (M = 1: the P-path GEMV)

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct MDesc {
    const uint32_t* codes;
    const _Float16* dict16p;  // K x 64 fp16, rows in kperm64 order
    const float* edge;
    const void* x;
    float* y;
    const float* bias;
    _Float16* xt;  // Mpad x C_full fp16 (hi), then Mpad x C_full (lo) for fp32 X
    int R, K, NB, NBc, slots, Ce, C_full;
    int u_base, u_count;  // units (row strip x block column) [u_base, u_base + u_count)
    float g0;             // the largest stage gain: scales the accumulated products
    uint32_t grel[16];    // slot j's gain relative to g0 as an fp16 pair (g_j / g0, same)
};

struct MParams {
    MDesc m[kGroup];
    int G, M, Mpad, x_f16, accumulate, total_units;
    int tm;  // token-major X (M x C) and Y (M x R)
    int m0;  // first column of this launch (the launch covers 16 * NT columns)
};

// X element (feature k, column m) in the call's layout.
__device__ __forceinline__ float xget(const MParams& p, const MDesc& d, int k, int m) {
    const size_t i = p.tm ? (size_t)m * (d.C_full + d.Ce) + k : (size_t)k * p.M + m;
    return p.x_f16 ? (float)static_cast<const _Float16*>(d.x)[i]
                   : static_cast<const float*>(d.x)[i];
}

// ---- init: Y start values, and X transposed to [m][k] fp16 in 16-byte granules of the
// permuted k order (threads run along m, so the X reads coalesce).
__global__ __launch_bounds__(kThreads) void mfma_init_kernel(MParams p) {
    const MDesc& d = p.m[blockIdx.y];
    const int M = p.M;
    const size_t ny = (size_t)d.R * M;
    const size_t ngr = (size_t)p.Mpad * d.NB * 8;
    const size_t nx = (size_t)p.Mpad * d.C_full;
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t t = (size_t)blockIdx.x * kThreads + threadIdx.x; t < ny + ngr; t += stride) {
        if (t < ny) {
            const int r = p.tm ? (int)(t % d.R) : (int)(t / M);
            const int m = p.tm ? (int)(t / d.R) : (int)(t - (size_t)r * M);
            float v = p.accumulate ? d.y[t] : 0.0f;
            if (d.bias) v += d.bias[r];
            if (d.Ce > 0) {
                const float* e = d.edge + (size_t)r * d.Ce;
                float s = 0.0f;
                for (int cc = 0; cc < d.Ce; ++cc)
                    s = fmaf(e[cc], xget(p, d, d.C_full + cc, m), s);
                v += s;
            }
            d.y[t] = v;
        } else {
            const size_t u = t - ny;
            const int m = (int)(u % p.Mpad);
            const size_t bg = u / p.Mpad;
            const int b = (int)(bg >> 3), g = (int)(bg & 7);
            _Float16 hi[8], lo[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int k = b * 64 + csdr::kperm64(g * 8 + j);
                const float xv = (m < M) ? xget(p, d, k, m) : 0.0f;
                hi[j] = (_Float16)xv;
                lo[j] = (_Float16)(xv - (float)hi[j]);
            }
            const size_t o = (size_t)m * d.C_full + (size_t)b * 64 + g * 8;
            *reinterpret_cast<u32x4*>(d.xt + o) = __builtin_bit_cast(u32x4, hi);
            if (!p.x_f16)
                *reinterpret_cast<u32x4*>(d.xt + nx + o) = __builtin_bit_cast(u32x4, lo);
        }
    }
}

__device__ __forceinline__ int find_matrix(const MParams& p, int u, int g) {
    if (g >= 0 && u >= p.m[g].u_base && u < p.m[g].u_base + p.m[g].u_count) return g;
    g = 0;
    while (g + 1 < p.G && u >= p.m[g + 1].u_base) ++g;
    return g;
}

// ---- main: persistent; NT = 16-column tiles of this launch, XS = fp32-X split, W waves of
// 32 rows (strip = 32 W rows). The codes and X slice of unit u + 1 are loaded into registers
// while unit u is decoded and multiplied. One workgroup per CU (the dictionary fills most of
// the LDS), so latency is hidden by the W waves of that workgroup.
// XR: each wave loads its X operands straight from the transposed X (global memory, L1/L2
// hits: the workgroup's waves all take the same unit sequence) one unit ahead, so the units
// need no X staging and no barriers; the waves run apart and one's LDS reads overlap
// another's arithmetic. Else the unit's X slice is staged in LDS by the whole workgroup.
// LB: slots whose dictionary reads are issued together before their multiply-adds.
template <int NT, bool XS, int W, int RT, int SLOTS, bool XR>
__global__ __launch_bounds__(W * 64) void mfma_kernel(MParams p) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    constexpr int CW = SLOTS / 4;  // 16-byte code pieces per tile
    constexpr int kThreads = W * 64;
    constexpr int kStripRows = W * 16 * RT;
    extern __shared__ __attribute__((aligned(16))) _Float16 smem16[];
    constexpr int MT = NT * 16;
    constexpr int NGR = MT * 8 * (XS ? 2 : 1);  // 16-byte X granules per unit
    constexpr int GPT = XR ? 1 : (NGR + kThreads - 1) / kThreads;
    constexpr int NP = XS ? 2 : 1;           // X parts (fp32 X: hi, lo)
    constexpr int LB = SLOTS < 4 ? SLOTS : 4;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int q = lane >> 4, rl = lane & 15;
    const int U = p.total_units;
    const int u0 = (int)((long long)U * blockIdx.x / gridDim.x);
    const int u1 = (int)((long long)U * (blockIdx.x + 1) / gridDim.x);
    if (u0 >= u1) return;
    // K x 64; 16-byte granule g of atom a at g ^ ((a >> 1) & 7): rows are 128 bytes, so
    // without it the 16 lanes of one k segment would meet in two bank groups
    _Float16* Ds = smem16;
    _Float16* Xs = smem16 + (size_t)kMaxAtoms * 64;  // MT x 64 (hi), then MT x 64 (lo)
    const int M = p.M;

    floatx4 acc[RT][NT];
    u32x4 xr[GPT];   // prefetched X granules of the next unit (staged X)
    u32x4 xb[XR ? NT : 1][NP][2];  // prefetched X operands of the next unit (XR)
    u32x4 cr[RT][CW];  // prefetched code words of the next unit (RT row tiles)
    int ng = -1, nstrip = 0, nb = 0;  // the prefetched unit

    auto prefetch = [&](int u) {
        ng = find_matrix(p, u, ng);
        const MDesc& d = p.m[ng];
        const int lu = u - d.u_base;
        nstrip = lu / d.NB;
        nb = lu - nstrip * d.NB;
        const size_t nxt = (size_t)p.Mpad * d.C_full;
        if constexpr (XR) {
            // lane (column n = 16 nt + rl, group q): granules 2q and 2q + 1 of the block
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int part = 0; part < NP; ++part)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        xb[nt][part][c] = *reinterpret_cast<const u32x4*>(
                            d.xt + part * nxt + (size_t)(p.m0 + nt * 16 + rl) * d.C_full +
                            (size_t)nb * 64 + (2 * q + c) * 8);
        }
#pragma unroll
        for (int i = 0; i < (XR ? 0 : GPT); ++i) {
            const int gi = min(tid + i * kThreads, NGR - 1);
            const int part = XS ? gi / (MT * 8) : 0;
            const int gg = gi - part * MT * 8;
            const int mrow = gg >> 3, gr = gg & 7;
            xr[i] = *reinterpret_cast<const u32x4*>(
                d.xt + part * nxt + (size_t)(p.m0 + mrow) * d.C_full + (size_t)nb * 64 + gr * 8);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int r = min(nstrip * kStripRows + wave * 16 * RT + rt * 16 + rl, d.R - 1);
            const uint32_t* cw =
                d.codes + csdr::tile_word_offset(r, nb, d.R, d.NB, d.NBc, d.slots);
#pragma unroll
            for (int j4 = 0; j4 < CW; ++j4) cr[rt][j4] = *reinterpret_cast<const u32x4*>(cw + j4 * 4);
        }
    };

    auto flush = [&](int g, int strip) {
        const MDesc& d = p.m[g];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int rbase = strip * kStripRows + wave * 16 * RT + rt * 16 + q * 4;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int m = p.m0 + nt * 16 + rl;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = rbase + i;
                    if (r < d.R && m < M)
                        __hip_atomic_fetch_add(d.y + (p.tm ? (size_t)m * d.R + r : (size_t)r * M + m),
                                               acc[rt][nt][i] * d.g0,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    };

    int cur_g = -1, cur_strip = -1;
    prefetch(u0);
    for (int u = u0; u < u1; ++u) {
        const int g = ng, strip = nstrip, b = nb;
        (void)b;
        const MDesc& d = p.m[g];
        if (g != cur_g || strip != cur_strip) {
            if (cur_strip >= 0) flush(cur_g, cur_strip);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[rt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (g != cur_g) {
                // the matrix's fp16 dictionary -> LDS (16-byte granules, 8 loads in flight)
                __syncthreads();
                const int n = d.K * 8;
                for (int i0 = 0; i0 < n; i0 += kThreads * 8) {
                    u32x4 v[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        v[j] = *reinterpret_cast<const u32x4*>(
                            d.dict16p + (size_t)min(i0 + j * kThreads + tid, n - 1) * 8);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int i = i0 + j * kThreads + tid;
                        const int a = i >> 3, gr = i & 7;
                        if (i < n)
                            *reinterpret_cast<u32x4*>(Ds + (size_t)a * 64 +
                                                      ((gr ^ ((a >> 1) & 7)) * 8)) = v[j];
                    }
                }
                if constexpr (XR) __syncthreads();
            }
            cur_g = g;
            cur_strip = strip;
        }
        u32x4 xc[XR ? NT : 1][NP][2];
        if constexpr (XR) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int part = 0; part < NP; ++part)
#pragma unroll
                    for (int c = 0; c < 2; ++c) xc[nt][part][c] = xb[nt][part][c];
        }
        // X slice -> LDS; granule index XOR (row & 7) against bank conflicts
        if constexpr (!XR) __syncthreads();
#pragma unroll
        for (int i = 0; i < (XR ? 0 : GPT); ++i) {
            const int gi = min(tid + i * kThreads, NGR - 1);
            const int part = XS ? gi / (MT * 8) : 0;
            const int gg = gi - part * MT * 8;
            const int mrow = gg >> 3, gr = gg & 7;
            *reinterpret_cast<u32x4*>(Xs + (size_t)part * MT * 64 + mrow * 64 +
                                      ((gr ^ (mrow & 7)) * 8)) = xr[i];
        }
        u32x4 cc[RT][CW];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int j4 = 0; j4 < CW; ++j4) cc[rt][j4] = cr[rt][j4];
        if constexpr (!XR) __syncthreads();
        if (u + 1 < u1) prefetch(u + 1);
        // decode this lane's 16 k values of each of its rows: per slot the coefficient as an
        // fp16 pair (times the slot's gain relative to slot 0) and 8 packed fp16 FMAs over the
        // atom's two 16-byte granules, accumulated in place as the two 8-value A operands
        half8 a[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            h2 w[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) w[t] = h2{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
            for (int j0 = 0; j0 < SLOTS; j0 += LB) {
                // the batch's LB atoms: both 16-byte granules of each read before any is used
                u32x4 lo[LB], hi[LB];
#pragma unroll
                for (int jj = 0; jj < LB; ++jj) {
                    const uint32_t word = cc[rt][(j0 + jj) >> 2][(j0 + jj) & 3];
                    const uint32_t at = word & 0x7FFFu;
                    const uint32_t sw = (at >> 1) & 7;
                    const _Float16* drow = Ds + at * 64;
                    lo[jj] = *reinterpret_cast<const u32x4*>(drow + (((2 * q) ^ sw) * 8));
                    hi[jj] = *reinterpret_cast<const u32x4*>(drow + (((2 * q + 1) ^ sw) * 8));
                }
#pragma unroll
                for (int jj = 0; jj < LB; ++jj) {
                    const int j = j0 + jj;
                    const uint32_t word = cc[rt][j >> 2][j & 3];
                    // (c, c): the word's high half in both halves
                    const h2 c2 =
                        __builtin_bit_cast(h2, __builtin_amdgcn_perm(word, word, 0x07060706u)) *
                        __builtin_bit_cast(h2, d.grel[j]);
                    // (vector elements go through a scalar: bit-casting a subscripted vector
                    // element directly reads element 0 whatever the subscript)
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t el = lo[jj][t], eh = hi[jj][t];
                        w[t] = __builtin_elementwise_fma(c2, __builtin_bit_cast(h2, el), w[t]);
                        w[4 + t] = __builtin_elementwise_fma(c2, __builtin_bit_cast(h2, eh), w[4 + t]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const u32x4 v = {__builtin_bit_cast(uint32_t, w[4 * c]),
                                 __builtin_bit_cast(uint32_t, w[4 * c + 1]),
                                 __builtin_bit_cast(uint32_t, w[4 * c + 2]),
                                 __builtin_bit_cast(uint32_t, w[4 * c + 3])};
                a[rt][c] = __builtin_bit_cast(half8, v);
            }
        }
        // two 32-deep steps over the block column: lane group q holds positions 16 q + 8 c ..
        // + 7 of the permuted k order in step c, in both operands
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = nt * 16 + rl;
            const int g0 = (2 * q) ^ (n & 7), g1 = (2 * q + 1) ^ (n & 7);
#pragma unroll
            for (int part = 0; part < (XS ? 2 : 1); ++part) {
                half8 bs[2];
                if constexpr (XR) {
                    bs[0] = __builtin_bit_cast(half8, xc[nt][part][0]);
                    bs[1] = __builtin_bit_cast(half8, xc[nt][part][1]);
                } else {
                    const _Float16* xrow = Xs + (size_t)part * MT * 64 + n * 64;
                    bs[0] = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4*>(xrow + g0 * 8));
                    bs[1] = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4*>(xrow + g1 * 8));
                }
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a[rt][c], bs[c], acc[rt][nt], 0, 0, 0);
            }
        }
    }
    if (cur_strip >= 0) flush(cur_g, cur_strip);
}

// ---- main, one 16-column tile (M <= 16): the dictionary route. Per unit (256-row strip,
// block column b) the workgroup forms Q_b = D . X_b (K atoms x 16 columns) on the matrix
// cores and each row then gathers its slots' rows of Q_b from LDS:
//   y[r][m] += g0 * sum_j (c_j * g_j / g0) * Q_b[idx_j][m],
// 32 bytes of LDS per (row, slot) where decoding the weights reads the atom's 128.
// - The dictionary lives in registers for the whole launch: 16 waves x 64 atoms, each wave's
//   atoms as the B operands of v_mfma_f32_16x16x32_f16 (8 x 16 bytes per lane), so LDS holds
//   only Q (two 32 KiB buffers: Q_{u+1} is formed while unit u is gathered, one barrier per
//   unit).
// - Q^T = X_b^T . D^T: lane (n = l % 16, q = l / 16) of a 16-atom tile ends with atom n's
//   columns 4q .. 4q + 3, one 8-byte LDS store. Q rows are 32 bytes of four 8-byte pieces,
//   piece q at q ^ 2 on atoms with bit 2 set, so that the gather's 16-byte halves stay whole
//   and its reads of random rows spread over all bank groups. Q is stored in fp16 (fp32
//   accumulation; |Q| <= ||x_b|| for unit-norm atoms).
// - Gather: lane (row l % 16 of the wave's 16, slot group q) takes slots q S/4 .. of its row
//   (S/4 code words, no lane loads another's) and all 16 columns (two 16-byte reads per slot,
//   fp16 x fp16 -> fp32 multiply-adds). When the strip ends the four slot groups of a row are
//   reduce-scattered by shuffles and the wave's 16 x 16 tile goes through LDS, so that each
//   device-scope atomic instruction into Y covers four whole rows.
// - Loads: each unit's code words and the X operands of the unit after it form one bundle,
//   issued two units ahead into a register ring (the wait for a bundle's X also covers every
//   earlier load, so both streams share one depth). Every load is unconditional (see below).
// A unit's position: strip, block column b, and the chunk holding b (first column b0,
// width nbc), advanced one unit at a time within one matrix whose geometry the caller keeps
// in registers (reading it from the kernel arguments inside the loop puts a scalar load and
// its wait, which also drains every LDS operation in flight, into every unit).
struct UnitCursor {
    int strip, b, b0, nbc;
};

struct SegGeom {
    int NB, NBc, R, nstrips, nfull;  // nfull: columns in full chunks
};

__device__ __forceinline__ void cursor_chunk(const SegGeom& s, UnitCursor& c) {
    if (c.b < s.nfull) {
        c.b0 = c.b & ~(s.NBc - 1);
        c.nbc = s.NBc;
        return;
    }
    uint32_t cc, b0, nbc;
    csdr::chunk_of((uint32_t)c.b, (uint32_t)s.NB, (uint32_t)s.NBc, cc, b0, nbc);
    c.b0 = (int)b0;
    c.nbc = (int)nbc;
}

// Next unit of the same matrix (wrapping past its last unit, so a cursor always names valid
// codes and X: the pipeline's loads past a range's end stay unconditional and in bounds).
__device__ __forceinline__ void cursor_next(const SegGeom& s, UnitCursor& c) {
    if (++c.b == s.NB) {
        c.b = 0;
        if (++c.strip == s.nstrips) c.strip = 0;
    }
    if (c.b == 0 || c.b >= c.b0 + c.nbc) cursor_chunk(s, c);
}

template <int SLOTS, bool XS>
__global__ __launch_bounds__(1024) void qroute_kernel(MParams p) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    constexpr int SPL = SLOTS / 4;   // slots per lane
    constexpr int NP = XS ? 2 : 1;   // X parts (fp32 X: hi, lo)
    constexpr int QB = kMaxAtoms * 16;  // fp16 per Q buffer
    typedef typename std::conditional<SPL == 4, u32x4,
            typename std::conditional<SPL == 2, uint2, uint32_t>::type>::type cword_t;
    extern __shared__ __attribute__((aligned(16))) _Float16 smem16[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int q = lane >> 4, rl = lane & 15;
    const int U = p.total_units;
    const int u0 = (int)((long long)U * blockIdx.x / gridDim.x);
    const int u1 = (int)((long long)U * (blockIdx.x + 1) / gridDim.x);
    if (u0 >= u1) return;
    const int M = p.M;

    // the units of one matrix at a time: its atoms in registers, then a pipeline over its units
    // in which every load is unconditional (a load under a branch makes the compiler's wait
    // counts assume the worst at the join, which drained the pipeline every unit)
    for (int s0 = u0; s0 < u1;) {
        const int g = find_matrix(p, s0, -1);
        const MDesc& d = p.m[g];
        const int s1 = min(u1, d.u_base + d.u_count);
        half8 dreg[4][2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int a = min(wave * 64 + t * 16 + rl, d.K - 1);
#pragma unroll
            for (int c = 0; c < 2; ++c)
                dreg[t][c] = __builtin_bit_cast(
                    half8, *reinterpret_cast<const u32x4*>(d.dict16p + (size_t)a * 64 + (2 * q + c) * 8));
        }
        // this lane's slots' gains relative to g0 (fp16), chosen from uniform loads
        _Float16 gl[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const uint32_t a0 = d.grel[j], a1 = d.grel[SPL + j], a2 = d.grel[2 * SPL + j],
                           a3 = d.grel[3 * SPL + j];
            const uint32_t w = q == 0 ? a0 : (q == 1 ? a1 : (q == 2 ? a2 : a3));
            gl[j] = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
        }
        const _Float16* xt0 = d.xt + (size_t)rl * d.C_full + q * 16;
        const size_t nxt = (size_t)p.Mpad * d.C_full;
        const int K = d.K;
        SegGeom sg;
        sg.NB = d.NB;
        sg.NBc = d.NBc;
        sg.R = d.R;
        sg.nstrips = (d.R + 255) >> 8;
        sg.nfull = d.NB & ~(d.NBc - 1);
        const uint32_t* codes = d.codes;
        float* y = d.y;
        const float g0 = d.g0;

        u32x4 xr[2][NP][2];
        cword_t cr[2];
        float ya[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) ya[e] = 0.0f;

        auto load_x = [&](const UnitCursor& c, u32x4 (&dst)[NP][2]) {
            const _Float16* src = xt0 + (size_t)c.b * 64;
#pragma unroll
            for (int part = 0; part < NP; ++part)
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
                    dst[part][cc] = *reinterpret_cast<const u32x4*>(src + part * nxt + cc * 8);
        };
        auto load_codes = [&](const UnitCursor& c, cword_t& dst) {
            const int r = min(c.strip * 256 + wave * 16 + rl, sg.R - 1);
            const size_t w =
                ((size_t)c.b0 * sg.R + (size_t)r * c.nbc + (c.b - c.b0)) * SLOTS + q * SPL;
            dst = *reinterpret_cast<const cword_t*>(codes + w);
        };
        // Q of a unit from its X operands xo, two atom tiles (t0, t0 + 1) at a time, each pair
        // then stored into buffer buf
        auto q_mfma = [&](const u32x4 (&xo)[NP][2], floatx4 (&acc)[2], int t0) {
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int part = 0; part < NP; ++part)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8, xo[part][cc]), dreg[t0 + t][cc], acc[t], 0, 0, 0);
        };
        auto q_store = [&](const floatx4 (&acc)[2], int buf, int t0) {
            _Float16* Qb = smem16 + (size_t)buf * QB;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int a = wave * 64 + (t0 + t) * 16 + rl;
                if (wave * 64 + (t0 + t) * 16 < K) {  // (uniform per wave)
                    const h2 lo = h2{(_Float16)acc[t][0], (_Float16)acc[t][1]};
                    const h2 hi = h2{(_Float16)acc[t][2], (_Float16)acc[t][3]};
                    const uint2 v = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
                    // 8-byte piece q of the 32-byte row at q ^ 2 (a bit 2): the two halves read
                    // by the gather stay 16-byte granules, spread over all bank groups
                    *reinterpret_cast<uint2*>(Qb + (size_t)a * 16 + ((q ^ ((a >> 1) & 2)) * 4)) = v;
                }
            }
        };
        auto words_of = [&](const cword_t& cw, uint32_t (&words)[SPL]) {
            if constexpr (SPL == 1) {
                words[0] = cw;
            } else if constexpr (SPL == 2) {
                words[0] = cw.x;
                words[1] = cw.y;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) words[j] = cw[j];
            }
        };
        auto g_read = [&](const uint32_t (&words)[SPL], int buf, u32x4 (&h)[SPL][2]) {
            const _Float16* Qb = smem16 + (size_t)buf * QB;
#pragma unroll
            for (int j = 0; j < SPL; ++j) {
                const uint32_t at = words[j] & 0x7FFFu;
                const uint32_t sw = (at >> 2) & 1;
                const _Float16* row = Qb + at * 16;
                h[j][0] = *reinterpret_cast<const u32x4*>(row + sw * 8);
                h[j][1] = *reinterpret_cast<const u32x4*>(row + (sw ^ 1) * 8);
            }
        };
        // the gather's multiply-adds of slot j
        auto g_acc = [&](const uint32_t (&words)[SPL], const u32x4 (&h)[SPL][2], int j) {
            const _Float16 cf = __builtin_bit_cast(_Float16, (uint16_t)(words[j] >> 16)) * gl[j];
            const float cfl = (float)cf;
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t dw = h[j][half][k];
                    const h2 pr = __builtin_bit_cast(h2, dw);
                    ya[half * 8 + 2 * k] = fmaf(cfl, (float)pr[0], ya[half * 8 + 2 * k]);
                    ya[half * 8 + 2 * k + 1] = fmaf(cfl, (float)pr[1], ya[half * 8 + 2 * k + 1]);
                }
        };
        // the strip's row sums: the four slot groups of a row summed by shuffles, then the
        // wave's 16 x 16 tile through LDS so that each atomic instruction covers four whole rows
        // of Y (token-major: four whole columns) instead of 16 scattered 16-byte pieces
        auto flush = [&](int strip) {
            float* T = reinterpret_cast<float*>(smem16 + 2 * (size_t)QB) + wave * 256;
            // reduce-scatter over the four slot groups (lanes l, l ^ 16, l ^ 32, l ^ 48): lane q
            // ends with columns 8 (q & 1) + 4 (q >> 1) .. + 3 of its row
            const bool b = q & 1, c = q >> 1;
            float t[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float keep = b ? ya[8 + k] : ya[k];
                const float send = b ? ya[k] : ya[8 + k];
                t[k] = keep + __shfl_xor(send, 16, 64);
            }
            float4 w;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float keep = c ? t[4 + k] : t[k];
                const float send = c ? t[k] : t[4 + k];
                w[k] = keep + __shfl_xor(send, 32, 64);
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) ya[e] = 0.0f;
            *reinterpret_cast<float4*>(T + rl * 16 + 8 * (q & 1) + 4 * (q >> 1)) = w;
            const int r0 = strip * 256 + wave * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // row-major: rows 4i + lane / 16, column lane % 16; token-major: rows lane % 16,
                // column 4i + lane / 16
                const int rr = p.tm ? rl : 4 * i + q;
                const int m = p.tm ? 4 * i + q : rl;
                const float v = T[rr * 16 + m];
                const int r = r0 + rr;
                if (r < sg.R && m < M)
                    __hip_atomic_fetch_add(y + (p.tm ? (size_t)m * sg.R + r : (size_t)r * M + m),
                                           v * g0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        };

        // cursors: gathered unit v, its successor (Q formed), the next bundle's codes (v + 2)
        // and X (v + 3); bundle w = (codes of w, X of w + 1), two in flight
        UnitCursor cg;
        {
            const int lu = s0 - d.u_base;
            cg.strip = lu / sg.NB;
            cg.b = lu - cg.strip * sg.NB;
            cursor_chunk(sg, cg);
        }
        UnitCursor cm = cg;
        cursor_next(sg, cm);
        UnitCursor cc = cg, cx = cm;
        {
            u32x4 x0[NP][2];
            load_x(cg, x0);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                load_x(cx, xr[i]);
                load_codes(cc, cr[i]);
                cursor_next(sg, cx);
                cursor_next(sg, cc);
            }
#pragma unroll
            for (int t0 = 0; t0 < 4; t0 += 2) {
                floatx4 acc[2];
                q_mfma(x0, acc, t0);
                q_store(acc, 0, t0);
            }
        }
        __syncthreads();
        // per unit: the gather's LDS reads of Q_v, the matrix-core steps of Q_{v+1} while they
        // are in flight, the gather's multiply-adds, then Q_{v+1} into the other buffer
        auto step = [&](int v, auto S) {
            constexpr int sl = decltype(S)::value;
            const bool more = v + 1 < s1;
            uint32_t words[SPL];
            words_of(cr[sl], words);
            u32x4 h[SPL][2];
            g_read(words, (v - s0) & 1, h);
            // tile pairs interleaved with the slots' multiply-adds
            constexpr int JP = SPL >= 2 ? SPL / 2 : 1;  // slots per tile pair
#pragma unroll
            for (int t0 = 0; t0 < 4; t0 += 2) {
                floatx4 acc[2];
                if (more) q_mfma(xr[sl], acc, t0);
#pragma unroll
                for (int jj = 0; jj < JP; ++jj) {
                    const int j = (t0 / 2) * JP + jj;
                    if (j < SPL) g_acc(words, h, j);
                }
                if (more) q_store(acc, (v + 1 - s0) & 1, t0);
            }
            load_x(cx, xr[sl]);
            load_codes(cc, cr[sl]);
            if (!more || cm.strip != cg.strip) flush(cg.strip);
            cg = cm;
            cursor_next(sg, cm);
            cursor_next(sg, cc);
            cursor_next(sg, cx);
            __syncthreads();
        };
        int v = s0;
        for (; v + 1 < s1; v += 2) {
            step(v, std::integral_constant<int, 0>{});
            step(v + 1, std::integral_constant<int, 1>{});
        }
        if (v < s1) step(v, std::integral_constant<int, 0>{});
        s0 = s1;
    }
}

// Columns of X the kernels see: M rounded up to a power of two >= 16 (<= 256), beyond 256 to
// a multiple of 256, so every launch covers a power-of-two tile of 16 NT columns.
int padded_m(int M) {
    if (M > kMaxMTile) return (M + kMaxMTile - 1) / kMaxMTile * kMaxMTile;
    int p = 16;
    while (p < M) p *= 2;
    return p;
}

size_t xt_bytes(const csdr_hsdb* s, int M) {
    const size_t mpad = (size_t)padded_m(M);
    return csdr::align_up(2 * mpad * s->C_full * sizeof(_Float16), 256);
}

// Waves per workgroup and 16-row tiles per wave for a column tile of 16 NT: more waves hide
// more load latency and let one wave's decode run beside another's matrix-core steps; the
// register budget (accumulators grow with NT and RT) caps them. Measured on cfg2 against two
// row tiles per wave (16 waves to 16 columns, 8 to 64, 4 beyond): one row tile, 16 waves to
// 64 columns and 8 beyond: M = 32 / 64 / 128 / 256 at 4096 x 11008: 47.1 -> 44.0, 58.6 ->
// 52.2, 78.2 -> 68.7, 105.5 -> 98.6 us (M = 16 unchanged).
constexpr int waves_for(int nt) { return nt <= 4 ? 16 : 8; }
// (two 16-row tiles per wave from 64 columns up, so that each X operand read from LDS feeds
// two matrix-core steps, measured slower: cfg2 M = 64 44.3 -> 56.6 us, M = 256 88.0 -> 104.8)
constexpr int rows_for(int) { return 1; }
// X operands from global memory (no X staging) for one 16-column tile: cfg2 4096 x 11008 at
// M = 16 36.2 -> 33.3 us per call; at two tiles (M = 32) slower, 40.4 -> 44.0; at four the
// prefetched operands spill
constexpr bool x_in_regs(int nt, bool) { return nt == 1; }

// The dictionary route for one 16-column tile (M <= 16); CSDR_HSDB_QROUTE=0 keeps the
// weight-decoding kernel there.
bool qroute_enabled() {
    const char* e = std::getenv("CSDR_HSDB_QROUTE");
    return !(e && *e && std::atoi(e) == 0);
}

template <int NT, bool XS, int SLOTS>
int launch_one(const MParams& p, int grid, size_t lds, hipStream_t st) {
    constexpr int W = waves_for(NT), RT = rows_for(NT);
    constexpr bool XR = x_in_regs(NT, XS);
    const void* fn = reinterpret_cast<const void*>(&mfma_kernel<NT, XS, W, RT, SLOTS, XR>);
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    mfma_kernel<NT, XS, W, RT, SLOTS, XR><<<grid, W * 64, lds, st>>>(p);
    CSDR_LAUNCH_CHECK("hsdb mfma");
    return CSDR_OK;
}

template <int NT, bool XS>
int launch_slots(const MParams& p, int slots, int grid, size_t lds, hipStream_t st) {
    switch (slots) {
        case 4: return launch_one<NT, XS, 4>(p, grid, lds, st);
        case 8: return launch_one<NT, XS, 8>(p, grid, lds, st);
        default: return launch_one<NT, XS, 16>(p, grid, lds, st);
    }
}

template <int NT>
int launch_main(const MParams& p, bool xs, int slots, int grid, size_t lds, hipStream_t st) {
    return xs ? launch_slots<NT, true>(p, slots, grid, lds, st)
              : launch_slots<NT, false>(p, slots, grid, lds, st);
}

}  // namespace

namespace csdr {

bool mfma_eligible(int n, const csdr_hsdb* const* segs, int M) {
    const char* e = std::getenv("CSDR_HSDB_MFMA");
    if (e && *e && std::atoi(e) == 0) return false;
    if (M < kMfmaMinM) return false;
    for (int i = 0; i < n; ++i) {
        const csdr_hsdb* s = segs[i];
        if (!s || s->tile_rows != 1 || s->tile_cols != 64 || s->K > (uint32_t)kMaxAtoms ||
            !s->d_dict16p ||
            s->NB == 0 || !(s->slots == 4 || s->slots == 8 || s->slots == 16) ||
            s->slots != segs[0]->slots)
            return false;
    }
    return true;
}

size_t mfma_workspace_bytes(int n, const csdr_hsdb* const* segs, int M) {
    size_t t = csdr::kWsHead;
    for (int i = 0; i < n; ++i) t += xt_bytes(segs[i], M);
    return t;
}

int mfma_matmul(int n, const csdr_hsdb* const* segs, const void* const* xs, int x_dtype, int M,
                float* const* ys, const float* const* bias, int accumulate, int token_major,
                void* workspace, size_t workspace_bytes, hipStream_t st) {
    const size_t need = mfma_workspace_bytes(n, segs, M);
    if (!workspace || workspace_bytes < need)
        return set_error(CSDR_E_WORKSPACE,
                         "hsdb_matmul: workspace needs " + std::to_string(need) + " bytes");
    MParams p{};
    p.G = n;
    p.M = M;
    p.Mpad = padded_m(M);
    p.x_f16 = (x_dtype == CSDR_F16);
    p.accumulate = accumulate;
    p.tm = token_major;
    char* ws = static_cast<char*>(workspace);
    size_t off = csdr::kWsHead;
    size_t max_elems = 0;
    for (int i = 0; i < n; ++i) {
        const csdr_hsdb* s = segs[i];
        MDesc& d = p.m[i];
        d.codes = s->d_codes;
        d.dict16p = s->d_dict16p;
        d.edge = s->d_edge;
        d.x = xs[i];
        d.y = ys[i];
        d.bias = bias ? bias[i] : nullptr;
        d.xt = reinterpret_cast<_Float16*>(ws + off);
        off += xt_bytes(s, M);
        d.R = (int)s->R;
        d.K = (int)s->K;
        d.NB = (int)s->NB;
        d.NBc = (int)s->NBc;
        d.slots = (int)s->slots;
        d.Ce = (int)s->Ce;
        d.C_full = (int)s->C_full;
        // the slots' gains relative to the largest: 1 for the usual single stage and powers of
        // two for gamma_l = 0.5^l (exact in fp16), never above 1 (no fp16 overflow)
        float gmax = 0.0f;
        for (uint32_t j = 0; j < s->slots && j < 16; ++j)
            gmax = std::max(gmax, std::fabs(s->h_slot_gamma[j]));
        d.g0 = gmax > 0.0f ? gmax : 1.0f;
        for (uint32_t j = 0; j < 16; ++j) {
            const float rel = j < s->slots ? s->h_slot_gamma[j] / d.g0 : 0.0f;
            const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)rel);
            d.grel[j] = h << 16 | h;
        }
        max_elems = std::max(max_elems, (size_t)d.R * M + (size_t)p.Mpad * d.NB * 8);
    }
    int dev = 0, ncu = 256, lds_max = 65536;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            v > 0)
            ncu = v;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) ==
                hipSuccess &&
            v > 0)
            lds_max = v;
    }
    {
        const int gx = (int)std::min<size_t>(2048, (max_elems + kThreads - 1) / kThreads);
        mfma_init_kernel<<<dim3(std::max(gx, 1), n), kThreads, 0, st>>>(p);
        CSDR_LAUNCH_CHECK("hsdb mfma init");
    }
    const bool xsplit = !p.x_f16;
    const size_t dict_lds = (size_t)kMaxAtoms * 64 * sizeof(_Float16);
    // widest power-of-two column tile whose X slice fits next to the dictionary
    int mt = std::min(p.Mpad, kMaxMTile);
    while (mt > 16 && dict_lds + (size_t)mt * 64 * 2 * (xsplit ? 2 : 1) > (size_t)lds_max)
        mt /= 2;
    const size_t lds = dict_lds + (size_t)mt * 64 * 2 * (xsplit ? 2 : 1);
    if (lds > (size_t)lds_max)
        return set_error(CSDR_E_UNSUPPORTED, "hsdb_matmul: LDS too small for the MFMA path");
    const int nt = mt / 16;
    int strip_rows = 16 * 2 * waves_for(1);
    switch (nt) {
        case 16: strip_rows = 16 * rows_for(16) * waves_for(16); break;
        case 8: strip_rows = 16 * rows_for(8) * waves_for(8); break;
        case 4: strip_rows = 16 * rows_for(4) * waves_for(4); break;
        case 2: strip_rows = 16 * rows_for(2) * waves_for(2); break;
        default: strip_rows = 16 * rows_for(1) * waves_for(1); break;
    }
    int units = 0;
    for (int i = 0; i < n; ++i) {
        MDesc& d = p.m[i];
        d.u_base = units;
        d.u_count = (d.R + strip_rows - 1) / strip_rows * d.NB;
        units += d.u_count;
    }
    p.total_units = units;
    const int grid = std::max(1, std::min(units, ncu));
    const int slots0 = (int)segs[0]->slots;
    if (nt == 1 && !xsplit && (slots0 == 4 || slots0 == 8) && qroute_enabled()) {
        // one 16-column tile of fp16 X: Q_b formed per unit on the matrix cores, rows gathered
        // from LDS (fp32 X and 16 slots keep the decoding kernel: their operand rings spill)
        // two Q buffers, then a 16 x 16 fp32 tile per wave for the strip flushes
        const size_t qlds = (size_t)2 * kMaxAtoms * 16 * sizeof(_Float16) + 16 * 256 * sizeof(float);
        auto go = [&](auto kern) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)qlds);
            kern<<<grid, 1024, qlds, st>>>(p);
        };
        if (slots0 == 4) go(qroute_kernel<4, false>);
        else go(qroute_kernel<8, false>);
        CSDR_LAUNCH_CHECK("hsdb qroute");
        return CSDR_OK;
    }
    for (int m0 = 0; m0 < p.Mpad; m0 += mt) {
        MParams q = p;
        q.m0 = m0;
        int rc;
        const int slots = (int)segs[0]->slots;
        switch (nt) {
            case 16: rc = launch_main<16>(q, xsplit, slots, grid, lds, st); break;
            case 8: rc = launch_main<8>(q, xsplit, slots, grid, lds, st); break;
            case 4: rc = launch_main<4>(q, xsplit, slots, grid, lds, st); break;
            case 2: rc = launch_main<2>(q, xsplit, slots, grid, lds, st); break;
            default: rc = launch_main<1>(q, xsplit, slots, grid, lds, st); break;
        }
        if (rc != CSDR_OK) return rc;
    }
    return CSDR_OK;
}

}  // namespace csdr
