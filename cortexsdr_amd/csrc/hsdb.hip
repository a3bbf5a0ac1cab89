// hsdb.hip — device-resident HSDR/HSDB segments and their kernels (gfx950).
//
// Path (cortexSDR tree): HierarchicalSDRStrategy::matmulRowMajor
// (strategies/HierarchicalSDRStrategy.cpp:1257-1338) and decompress (:1340-1440), with the
// block-coded "HSDB" generalisation of research exp_c_kernel/benchmark.py:106-130.
//
// Math. W is R x C; tile (r, b) covers W[r, b*B : b*B+B] (1-row tiles, B = tile_cols) and
// is sum_j c_j * D[idx_j] over its S*k coded slots, c_j = gamma_{j/k} * signed fp16 |c|
// (binary HSDR: |c| = 1). Y = W.X is computed without W:
//   kernel 1 (dx):     P[b][a][m] = D[a] . X[b*B : b*B+B, m]          (the reference's Dx)
//   kernel 2 (gather): Y[r][m] = sum_b sum_j c_j * P[b][idx_j][m] + edge strip . X
//
// Device code layout (built at load time; 4 bytes per slot, the stream's own byte count):
//   word = (signed fp16 coefficient bits << 16) | atom index (15 bits)
// ordered chunk-major: block columns are grouped in chunks of NBc; chunk c holds, for
// every row r, the NBc tiles (r, c*NBc .. c*NBc+NBc-1) back to back, so a workgroup that
// owns (chunk, row tile) streams one contiguous range. 2-D tiles (tile_rows > 1, decode
// only) keep the stream's tile-major order.
//
// Gather workgroup = (chunk, row tile). It stages the chunk's P slice (NBc*K floats per
// column) in LDS, streams its code words once (non-temporal vector loads), gathers from
// LDS, reduces per row, writes a per-chunk partial, and the last workgroup to finish a row
// tile (device-scope counter, self-resetting by wrap-around) sums the partials in chunk
// order and adds the fp32 edge strip. Workgroups are numbered so that all row tiles of a
// chunk land on one XCD (dispatch is round-robin over the 8 XCDs), which keeps that
// chunk's P slice in a single L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"

struct csdr_hsdb {
    uint32_t R = 0, C = 0, tile_rows = 1, tile_cols = 0, K = 0, S = 0, k = 0, slots = 0;
    uint32_t n_row_tiles = 0, NB = 0, n_tiles = 0, R_full = 0, C_full = 0, Ce = 0;
    uint32_t NBc = 1, nchunks = 1;
    int is_hsdb = 0;
    int device = 0;
    float* d_dict = nullptr;        // K x tile_dim fp32
    uint32_t* d_codes = nullptr;    // n_tiles * slots words
    float* d_slot_gamma = nullptr;  // slots floats: gamma[j / k]
    float* d_edge = nullptr;        // top-right strip (R_full x Ce) then bottom strip
    size_t edge_floats = 0;
    size_t device_bytes = 0;
};

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kDxBlocksPerWG = 16;
constexpr uint32_t kMaxChunkBlocks = 8;

// Row-tile height of the gather for a given column group width.
inline int gather_rows_per_wg(int MV) { return MV == 1 ? 256 : 64; }

// ------------------------------------------------------------------ dx kernels

// P[b][a][m] for block length 64: one thread per atom, D row held in registers, the
// x blocks of this workgroup staged in LDS. Summation order over t matches the CPU
// restatement (t ascending, fused multiply-add).
template <typename XT>
__global__ __launch_bounds__(kThreads) void dx_b64_kernel(const float* __restrict__ D,
                                                          const XT* __restrict__ x, int K,
                                                          int NB, int M,
                                                          float* __restrict__ P) {
    __shared__ float xs[kDxBlocksPerWG][64];
    const int a = blockIdx.x * kThreads + threadIdx.x;
    const int b0 = blockIdx.y * kDxBlocksPerWG;
    const int m = blockIdx.z;
    const int nb = min(kDxBlocksPerWG, NB - b0);
    for (int i = threadIdx.x; i < nb * 64; i += kThreads)
        xs[i >> 6][i & 63] = csdr::to_f32(x[(size_t)(b0 * 64 + i) * M + m]);
    __syncthreads();
    if (a >= K) return;
    float drow[64];
    const float4* dp = reinterpret_cast<const float4*>(D + (size_t)a * 64);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = dp[i];
        drow[4 * i + 0] = v.x;
        drow[4 * i + 1] = v.y;
        drow[4 * i + 2] = v.z;
        drow[4 * i + 3] = v.w;
    }
    for (int bb = 0; bb < nb; ++bb) {
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < 64; ++t) acc = fmaf(drow[t], xs[bb][t], acc);
        P[((size_t)(b0 + bb) * K + a) * M + m] = acc;
    }
}

// P[b][a][m] for any block length (1-row HSDR streams have B = C): one wave per
// (b, a, group of up to 8 columns); lanes stride over the block, then a wave reduction.
template <typename XT>
__global__ __launch_bounds__(kThreads) void dx_generic_kernel(const float* __restrict__ D,
                                                              const XT* __restrict__ x, int K,
                                                              int NB, int blen, int M,
                                                              float* __restrict__ P) {
    const int lane = threadIdx.x & 63;
    const long long wave = ((long long)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const int mg = (M + 7) / 8;
    if (wave >= (long long)NB * K * mg) return;
    const int g = (int)(wave % mg);
    const long long ba = wave / mg;
    const int b = (int)(ba / K), a = (int)(ba % K);
    const int m0 = g * 8, nm = min(8, M - m0);
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    const float* drow = D + (size_t)a * blen;
    const XT* xb = x + (size_t)b * blen * M + m0;
    for (int t = lane; t < blen; t += 64) {
        const float dv = drow[t];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < nm) acc[j] = fmaf(dv, csdr::to_f32(xb[(size_t)t * M + j]), acc[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = csdr::wave_sum(acc[j]);
    if (lane == 0)
        for (int j = 0; j < nm; ++j) P[((size_t)b * K + a) * M + m0 + j] = acc[j];
}

// ------------------------------------------------------------------ gather kernel

struct GatherParams {
    const uint32_t* codes;
    const float* P;
    const float* slot_gamma;
    const float* edge;
    const void* x;
    float* y;
    float* ypart;
    unsigned int* counters;
    int x_f16;
    int R, K, NB, NBc, nchunks, slots, Rt, nrt, M, MVz, Ce, C_full;
};

template <typename XT>
__device__ __forceinline__ float edge_dot(const GatherParams& p, int r, int m) {
    const XT* x = static_cast<const XT*>(p.x);
    const float* e = p.edge + (size_t)r * p.Ce;
    float s = 0.0f;
    for (int c = 0; c < p.Ce; ++c)
        s = fmaf(e[c], csdr::to_f32(x[(size_t)(p.C_full + c) * p.M + m]), s);
    return s;
}

// MV: output columns per pass (1 or 4); MAXIT: (row, block) pairs per thread;
// SLOTS: coded slots per tile when it is a multiple of 4 (vector loads), 0 = any.
template <int MV, int MAXIT, int SLOTS>
__global__ __launch_bounds__(kThreads) void gather_kernel(GatherParams p) {
    extern __shared__ float smem[];
    // ---- workgroup -> (chunk, row tile), all row tiles of a chunk on one XCD
    const int wg = blockIdx.x;
    const int xcd = wg & 7;
    const int j = wg >> 3;
    const int cl = j / p.nrt;
    const int rt = j - cl * p.nrt;
    const int c = cl * 8 + xcd;
    if (c >= p.nchunks) return;

    const int tid = threadIdx.x;
    const int b0 = c * p.NBc;
    const int nbc = min(p.NBc, p.NB - b0);
    const int r0 = rt * p.Rt;
    const int nr = min(p.Rt, p.R - r0);
    const int npairs = nr * nbc;
    const int slots = SLOTS > 0 ? SLOTS : p.slots;
    const uint32_t* cb =
        p.codes + (size_t)c * p.NBc * p.R * slots + (size_t)r0 * nbc * slots;

    float* Ps = smem;                                      // nbc * K * MV
    float* part = smem + (size_t)p.NBc * p.K * MV;         // Rt * NBc * MV

    // ---- 1. stream this workgroup's code words into registers (issued first)
    constexpr int NV = SLOTS > 0 ? SLOTS / 4 : 1;
    u32x4 wv[MAXIT][NV];
    if constexpr (SLOTS > 0) {
#pragma unroll
        for (int i = 0; i < MAXIT; ++i) {
            const int pi = tid + i * kThreads;
            if (pi < npairs) {
                const u32x4* src = reinterpret_cast<const u32x4*>(cb + (size_t)pi * SLOTS);
#pragma unroll
                for (int q = 0; q < NV; ++q) wv[i][q] = __builtin_nontemporal_load(src + q);
            }
        }
    }
    float sg[SLOTS > 0 ? SLOTS : 1];
    if constexpr (SLOTS > 0) {
#pragma unroll
        for (int q = 0; q < SLOTS; ++q) sg[q] = p.slot_gamma[q];
    }

    const bool direct = (p.nchunks == 1);
    for (int z = 0; z < p.MVz; ++z) {
        const int m0 = z * MV;
        // ---- 2. stage the chunk's P slice (columns m0 .. m0+MV) in LDS
        if (z > 0) __syncthreads();
        const int nP = nbc * p.K;
        const float* Pg = p.P + (size_t)b0 * p.K * p.M;
        if (MV == 1 && p.M == 1 && (p.K & 3) == 0) {
            const int n4 = nP >> 2;
            const float4* s4 = reinterpret_cast<const float4*>(Pg);
            float4* d4 = reinterpret_cast<float4*>(Ps);
            for (int i = tid; i < n4; i += kThreads) d4[i] = s4[i];
            for (int i = (n4 << 2) + tid; i < nP; i += kThreads) Ps[i] = Pg[i];
        } else {
            for (int i = tid; i < nP * MV; i += kThreads) {
                const int e = i / MV, mm = i - e * MV;
                const int m = m0 + mm;
                Ps[i] = (m < p.M) ? Pg[(size_t)e * p.M + m] : 0.0f;
            }
        }
        __syncthreads();

        // ---- 3. gather from LDS
        float acc[MAXIT][MV];
#pragma unroll
        for (int i = 0; i < MAXIT; ++i)
#pragma unroll
            for (int mm = 0; mm < MV; ++mm) acc[i][mm] = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXIT; ++i) {
            const int pi = tid + i * kThreads;
            if (pi < npairs) {
                const int bb = pi % nbc;
                const float* Pb = Ps + (size_t)bb * p.K * MV;
                if constexpr (SLOTS > 0) {
#pragma unroll
                    for (int q = 0; q < NV; ++q) {
                        const uint32_t w4[4] = {wv[i][q].x, wv[i][q].y, wv[i][q].z, wv[i][q].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t w = w4[e];
                            const float cf = sg[q * 4 + e] * csdr::h2f(w >> 16);
                            const float* pv = Pb + (size_t)(w & 0x7FFFu) * MV;
                            if constexpr (MV == 1) {
                                acc[i][0] = fmaf(cf, pv[0], acc[i][0]);
                            } else {
                                const float4 v = *reinterpret_cast<const float4*>(pv);
                                acc[i][0] = fmaf(cf, v.x, acc[i][0]);
                                acc[i][1] = fmaf(cf, v.y, acc[i][1]);
                                acc[i][2] = fmaf(cf, v.z, acc[i][2]);
                                acc[i][3] = fmaf(cf, v.w, acc[i][3]);
                            }
                        }
                    }
                } else {
                    const uint32_t* src = cb + (size_t)pi * slots;
                    for (int s = 0; s < slots; ++s) {
                        const uint32_t w = src[s];
                        const float cf = p.slot_gamma[s] * csdr::h2f(w >> 16);
                        const float* pv = Pb + (size_t)(w & 0x7FFFu) * MV;
#pragma unroll
                        for (int mm = 0; mm < MV; ++mm) acc[i][mm] = fmaf(cf, pv[mm], acc[i][mm]);
                    }
                }
            }
        }

        // ---- 4. per-row reduction over the chunk's blocks (block order)
#pragma unroll
        for (int i = 0; i < MAXIT; ++i) {
            const int pi = tid + i * kThreads;
            if (pi < npairs)
#pragma unroll
                for (int mm = 0; mm < MV; ++mm) part[pi * MV + mm] = acc[i][mm];
        }
        __syncthreads();
        for (int t = tid; t < nr * MV; t += kThreads) {
            const int rr = t / MV, mm = t - rr * MV;
            const int m = m0 + mm;
            if (m >= p.M) continue;
            float s = 0.0f;
            for (int bb = 0; bb < nbc; ++bb) s += part[(rr * nbc + bb) * MV + mm];
            const int r = r0 + rr;
            if (direct) {
                if (p.Ce > 0)
                    s += p.x_f16 ? edge_dot<_Float16>(p, r, m) : edge_dot<float>(p, r, m);
                p.y[(size_t)r * p.M + m] = s;
            } else {
                p.ypart[((size_t)c * p.R + r) * p.M + m] = s;
            }
        }
    }
    if (direct) return;

    // ---- 5. last workgroup of this row tile sums the chunk partials in chunk order
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned int old = atomicInc(&p.counters[rt], (unsigned int)(p.nchunks - 1));
        s_last = (old == (unsigned int)(p.nchunks - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int t = tid; t < nr * p.M; t += kThreads) {
        const int rr = t / p.M, m = t - rr * p.M;
        const int r = r0 + rr;
        float s = 0.0f;
        for (int cc = 0; cc < p.nchunks; ++cc)
            s += __builtin_nontemporal_load(&p.ypart[((size_t)cc * p.R + r) * p.M + m]);
        if (p.Ce > 0) s += p.x_f16 ? edge_dot<_Float16>(p, r, m) : edge_dot<float>(p, r, m);
        p.y[(size_t)r * p.M + m] = s;
    }
}

// ------------------------------------------------------------------ decode / export

__device__ __forceinline__ size_t code_offset(const csdr_hsdb& s, uint32_t t) {
    if (s.tile_rows != 1) return (size_t)t * s.slots;
    const uint32_t r = t / s.NB, b = t - r * s.NB;
    const uint32_t c = b / s.NBc, bb = b - c * s.NBc;
    const uint32_t nbc = min(s.NBc, s.NB - c * s.NBc);
    return ((size_t)c * s.NBc * s.R + (size_t)r * nbc + bb) * s.slots;
}

// Dense tiles: element e of tile t = sum over slots (stage-major) of coef * atom[e], one
// fused multiply-add per slot starting from 0 (decodeAllTiles order), then reassembled.
__global__ __launch_bounds__(kThreads) void decode_dense_kernel(csdr_hsdb s,
                                                                float* __restrict__ W) {
    const uint32_t tile_dim = s.tile_rows * s.tile_cols;
    const size_t total = (size_t)s.n_tiles * tile_dim;
    const uint32_t n_col_tiles = s.C_full / s.tile_cols;
    for (size_t g = (size_t)blockIdx.x * kThreads + threadIdx.x; g < total;
         g += (size_t)gridDim.x * kThreads) {
        const uint32_t t = (uint32_t)(g / tile_dim);
        const uint32_t e = (uint32_t)(g - (size_t)t * tile_dim);
        const uint32_t* w = s.d_codes + code_offset(s, t);
        float acc = 0.0f;
        for (uint32_t j = 0; j < s.slots; ++j) {
            const uint32_t wd = w[j];
            const float cf = s.d_slot_gamma[j] * csdr::h2f(wd >> 16);
            acc = fmaf(cf, s.d_dict[(size_t)(wd & 0x7FFFu) * tile_dim + e], acc);
        }
        const uint32_t br = t / n_col_tiles, bc = t - br * n_col_tiles;
        const uint32_t rr = e / s.tile_cols, cc = e - rr * s.tile_cols;
        W[(size_t)(br * s.tile_rows + rr) * s.C + bc * s.tile_cols + cc] = acc;
    }
}

// Edge strips back into W: top-right (rows < R_full, cols >= C_full), then bottom rows.
__global__ __launch_bounds__(kThreads) void decode_edge_kernel(csdr_hsdb s,
                                                               float* __restrict__ W) {
    const size_t tr = (size_t)s.R_full * s.Ce;
    for (size_t g = (size_t)blockIdx.x * kThreads + threadIdx.x; g < s.edge_floats;
         g += (size_t)gridDim.x * kThreads) {
        size_t dst;
        if (g < tr) {
            const size_t r = g / s.Ce, cc = g - r * s.Ce;
            dst = r * s.C + s.C_full + cc;
        } else {
            const size_t h = g - tr;
            dst = (size_t)s.R_full * s.C + h;
        }
        W[dst] = s.d_edge[g];
    }
}

__global__ __launch_bounds__(kThreads) void export_codes_kernel(csdr_hsdb s,
                                                                uint16_t* __restrict__ packed,
                                                                uint16_t* __restrict__ coef) {
    const size_t total = (size_t)s.n_tiles * s.slots;
    for (size_t g = (size_t)blockIdx.x * kThreads + threadIdx.x; g < total;
         g += (size_t)gridDim.x * kThreads) {
        const uint32_t t = (uint32_t)(g / s.slots);
        const uint32_t j = (uint32_t)(g - (size_t)t * s.slots);
        const uint32_t w = s.d_codes[code_offset(s, t) + j];
        packed[g] = (uint16_t)((w & 0x7FFFu) | ((w >> 16) & 0x8000u));
        if (coef) coef[g] = (uint16_t)((w >> 16) & 0x7FFFu);
    }
}

// ------------------------------------------------------------------ host side

uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

int grid_for(size_t work) {
    size_t g = (work + kThreads - 1) / kThreads;
    return (int)std::max<size_t>(1, std::min<size_t>(g, 65536));
}

// Stream parse with the reference's checks (HierarchicalSDRStrategy.cpp:1265-1290 and
// readBuffer's truncation check) plus index < n_atoms.
int parse_and_upload(const uint8_t* buf, size_t n, hipStream_t st, csdr_hsdb* s) {
    if (!buf) return set_error(CSDR_E_INVALID, "hsdb_load: null stream");
    if (n < 36) return set_error(CSDR_E_TRUNCATED, "hsdb_load: stream shorter than header");
    if (std::memcmp(buf, "HSDR", 4) == 0) {
        s->is_hsdb = 0;
        if (rd32(buf + 4) != 2) return set_error(CSDR_E_FORMAT, "HSDR: unsupported version");
    } else if (std::memcmp(buf, "HSDB", 4) == 0) {
        s->is_hsdb = 1;
        if (rd32(buf + 4) != 1) return set_error(CSDR_E_FORMAT, "HSDB: unsupported version");
    } else {
        return set_error(CSDR_E_FORMAT, "hsdb_load: bad magic - not an HSDR/HSDB stream");
    }
    s->R = rd32(buf + 8);
    s->C = rd32(buf + 12);
    s->n_tiles = rd32(buf + 16);
    s->tile_rows = rd16(buf + 20);
    s->tile_cols = rd16(buf + 22);
    s->K = rd16(buf + 24);
    s->S = buf[26];
    s->k = buf[27];
    const uint32_t edge_bytes = rd32(buf + 32);
    if (s->tile_rows == 0 || s->tile_cols == 0 || s->K == 0)
        return set_error(CSDR_E_FORMAT, "hsdb_load: zero tile geometry or dictionary");
    if (s->K > 32768) return set_error(CSDR_E_FORMAT, "hsdb_load: n_atoms exceeds 15-bit index");
    if (s->is_hsdb && s->tile_rows != 1)
        return set_error(CSDR_E_FORMAT, "HSDB: tile_rows must be 1");
    s->slots = s->S * s->k;
    s->R_full = (s->R / s->tile_rows) * s->tile_rows;
    s->C_full = (s->C / s->tile_cols) * s->tile_cols;
    s->n_row_tiles = s->R_full / s->tile_rows;
    s->NB = s->C_full / s->tile_cols;
    if ((uint64_t)s->n_row_tiles * s->NB != s->n_tiles)
        return set_error(CSDR_E_FORMAT, "hsdb_load: tile count does not match shape");
    s->Ce = s->C - s->C_full;
    const uint64_t expect_edge =
        ((uint64_t)s->R_full * s->Ce + (uint64_t)(s->R - s->R_full) * s->C) * 4u;
    if (expect_edge != edge_bytes)
        return set_error(CSDR_E_FORMAT, "hsdb_load: edge byte count does not match shape");
    s->edge_floats = edge_bytes / 4;
    const size_t tile_dim = (size_t)s->tile_rows * s->tile_cols;
    const size_t n_codes = (size_t)s->n_tiles * s->slots;
    const size_t off_gamma = 36;
    const size_t off_dict = off_gamma + 4u * s->S;
    const size_t off_packed = off_dict + 4u * (size_t)s->K * tile_dim;
    const size_t off_coef = off_packed + 2u * n_codes;
    const size_t off_edge = off_coef + (s->is_hsdb ? 2u * n_codes : 0);
    const size_t end = off_edge + edge_bytes;
    if (end > n) return set_error(CSDR_E_TRUNCATED, "hsdb_load: truncated stream");
    if (s->slots == 0 && s->n_tiles > 0)
        return set_error(CSDR_E_FORMAT, "hsdb_load: zero coded slots per tile");

    // chunking of block columns (1-row tiles): P slice of a chunk <= 16 KiB per column
    if (s->tile_rows == 1) {
        uint32_t nbc = kMaxChunkBlocks;
        while (nbc > 1 && (size_t)nbc * s->K * 4 > 16384) nbc >>= 1;
        while (nbc > 1 && nbc > s->NB) nbc >>= 1;
        s->NBc = nbc;
        s->nchunks = s->NB ? (s->NB + nbc - 1) / nbc : 0;
    }

    // build the device words
    std::vector<uint32_t> words(n_codes);
    for (size_t i = 0; i < n_codes; ++i) {
        const uint16_t pk = rd16(buf + off_packed + 2 * i);
        const uint32_t idx = pk & 0x7FFFu;
        if (idx >= s->K)
            return set_error(CSDR_E_FORMAT, "hsdb_load: atom index " + std::to_string(idx) +
                                                " >= n_atoms " + std::to_string(s->K));
        const uint32_t mag = s->is_hsdb ? (rd16(buf + off_coef + 2 * i) & 0x7FFFu) : 0x3C00u;
        const uint32_t h = mag | (pk & 0x8000u);
        size_t dst = i;
        if (s->tile_rows == 1) {
            const size_t t = i / s->slots, j = i - t * s->slots;
            const uint32_t r = (uint32_t)(t / s->NB), b = (uint32_t)(t - (size_t)r * s->NB);
            const uint32_t c = b / s->NBc, bb = b - c * s->NBc;
            const uint32_t nbc = std::min(s->NBc, s->NB - c * s->NBc);
            dst = ((size_t)c * s->NBc * s->R + (size_t)r * nbc + bb) * s->slots + j;
        }
        words[dst] = (h << 16) | idx;
    }
    std::vector<float> slot_gamma(std::max<uint32_t>(s->slots, 1), 0.0f);
    for (uint32_t j = 0; j < s->slots; ++j)
        std::memcpy(&slot_gamma[j], buf + off_gamma + 4u * (j / s->k), 4);

    const size_t b_dict = (size_t)s->K * tile_dim * 4;
    const size_t b_codes = n_codes * 4;
    const size_t b_gamma = slot_gamma.size() * 4;
    const size_t b_edge = edge_bytes;
    CSDR_HIP_CHECK(hipMalloc(&s->d_dict, std::max<size_t>(b_dict, 4)));
    CSDR_HIP_CHECK(hipMalloc(&s->d_codes, std::max<size_t>(b_codes, 4)));
    CSDR_HIP_CHECK(hipMalloc(&s->d_slot_gamma, b_gamma));
    CSDR_HIP_CHECK(hipMalloc(&s->d_edge, std::max<size_t>(b_edge, 4)));
    s->device_bytes = b_dict + b_codes + b_gamma + b_edge;
    CSDR_HIP_CHECK(hipMemcpyAsync(s->d_dict, buf + off_dict, b_dict, hipMemcpyHostToDevice, st));
    if (b_codes)
        CSDR_HIP_CHECK(
            hipMemcpyAsync(s->d_codes, words.data(), b_codes, hipMemcpyHostToDevice, st));
    CSDR_HIP_CHECK(
        hipMemcpyAsync(s->d_slot_gamma, slot_gamma.data(), b_gamma, hipMemcpyHostToDevice, st));
    if (b_edge)
        CSDR_HIP_CHECK(hipMemcpyAsync(s->d_edge, buf + off_edge, b_edge, hipMemcpyHostToDevice, st));
    // the host vectors die with this call: wait for the copies
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    return CSDR_OK;
}

void release(csdr_hsdb* s) {
    if (!s) return;
    if (s->d_dict) (void)hipFree(s->d_dict);
    if (s->d_codes) (void)hipFree(s->d_codes);
    if (s->d_slot_gamma) (void)hipFree(s->d_slot_gamma);
    if (s->d_edge) (void)hipFree(s->d_edge);
    delete s;
}

struct WsLayout {
    size_t counters, P, ypart, total;
};

WsLayout ws_layout(const csdr_hsdb* s, int M) {
    WsLayout w{};
    const size_t max_row_tiles = (s->R + 63) / 64;
    w.counters = 0;
    w.P = csdr::align_up(max_row_tiles * 4, 256);
    w.ypart = w.P + csdr::align_up((size_t)s->NB * s->K * M * 4, 256);
    w.total = w.ypart + csdr::align_up((size_t)s->nchunks * s->R * M * 4, 256);
    return w;
}

template <int MV, int MAXIT>
hipError_t launch_gather_mv(const GatherParams& p, int slots, int grid, size_t lds,
                            hipStream_t st) {
    switch (slots) {
        case 4:
            gather_kernel<MV, MAXIT, 4><<<grid, kThreads, lds, st>>>(p);
            break;
        case 8:
            gather_kernel<MV, MAXIT, 8><<<grid, kThreads, lds, st>>>(p);
            break;
        case 16:
            gather_kernel<MV, MAXIT, 16><<<grid, kThreads, lds, st>>>(p);
            break;
        case 24:
            gather_kernel<MV, MAXIT, 24><<<grid, kThreads, lds, st>>>(p);
            break;
        default:
            gather_kernel<MV, MAXIT, 0><<<grid, kThreads, lds, st>>>(p);
            break;
    }
    return hipGetLastError();
}

template <int MV>
hipError_t launch_gather(const GatherParams& p, int maxit, int slots, int grid, size_t lds,
                         hipStream_t st) {
    switch (maxit) {
        case 1:
            return launch_gather_mv<MV, 1>(p, slots, grid, lds, st);
        case 2:
            return launch_gather_mv<MV, 2>(p, slots, grid, lds, st);
        case 4:
            return launch_gather_mv<MV, 4>(p, slots, grid, lds, st);
        default:
            return launch_gather_mv<MV, 8>(p, slots, grid, lds, st);
    }
}

}  // namespace

extern "C" {

CSDR_API int csdr_hsdb_load(const void* stream, size_t nbytes, void* hip_stream,
                            csdr_hsdb** out) {
    if (!out) return set_error(CSDR_E_INVALID, "hsdb_load: null out");
    *out = nullptr;
    csdr_hsdb* s = new (std::nothrow) csdr_hsdb();
    if (!s) return set_error(CSDR_E_INVALID, "hsdb_load: out of host memory");
    if (hipGetDevice(&s->device) != hipSuccess) {
        delete s;
        return set_error(CSDR_E_HIP, "hsdb_load: no HIP device");
    }
    int rc;
    try {
        rc = parse_and_upload(static_cast<const uint8_t*>(stream), nbytes,
                              static_cast<hipStream_t>(hip_stream), s);
    } catch (const std::bad_alloc&) {
        rc = set_error(CSDR_E_INVALID, "hsdb_load: out of host memory");
    }
    if (rc != CSDR_OK) {
        release(s);
        return rc;
    }
    *out = s;
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_free(csdr_hsdb* seg) {
    release(seg);
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_get_info(const csdr_hsdb* s, csdr_hsdb_info* info) {
    if (!s || !info) return set_error(CSDR_E_INVALID, "hsdb_get_info: null argument");
    info->rows = s->R;
    info->cols = s->C;
    info->tile_rows = s->tile_rows;
    info->tile_cols = s->tile_cols;
    info->n_atoms = s->K;
    info->n_stages = s->S;
    info->k_per_stage = s->k;
    info->slots = s->slots;
    info->n_block_cols = s->NB;
    info->chunk_blocks = s->NBc;
    info->edge_cols = s->Ce;
    info->is_hsdb = (uint32_t)s->is_hsdb;
    info->code_bytes = (uint64_t)s->n_tiles * s->slots * 4;
    info->device_bytes = s->device_bytes;
    return CSDR_OK;
}

CSDR_API size_t csdr_hsdb_workspace_bytes(const csdr_hsdb* s, int M) {
    if (!s || M <= 0) return 0;
    return ws_layout(s, M).total;
}

namespace {

int check_matmul_args(const csdr_hsdb* s, const void* x, int x_dtype, int M, void* workspace,
                      size_t workspace_bytes, const char* who) {
    if (!s || !x || M <= 0) return set_error(CSDR_E_INVALID, std::string(who) + ": bad argument");
    if (s->tile_rows != 1)
        return set_error(CSDR_E_FORMAT,
                         std::string(who) + ": fused matmul requires tile_rows == 1; use "
                                            "csdr_hsdb_decompress + a dense matmul for 2-D tiles");
    if (x_dtype != CSDR_F32 && x_dtype != CSDR_F16)
        return set_error(CSDR_E_INVALID, std::string(who) + ": x_dtype must be CSDR_F32 or CSDR_F16");
    if (s->NB == 0)
        return set_error(CSDR_E_UNSUPPORTED, std::string(who) + ": matrix narrower than one block");
    const WsLayout wl = ws_layout(s, M);
    if (!workspace || workspace_bytes < wl.total)
        return set_error(CSDR_E_WORKSPACE, std::string(who) + ": workspace needs " +
                                               std::to_string(wl.total) + " bytes");
    return CSDR_OK;
}

}  // namespace

CSDR_API int csdr_hsdb_dx(const csdr_hsdb* s, const void* x, int x_dtype, int M, void* workspace,
                          size_t workspace_bytes, void* hip_stream) {
    int rc = check_matmul_args(s, x, x_dtype, M, workspace, workspace_bytes, "hsdb_dx");
    if (rc) return rc;
    const WsLayout wl = ws_layout(s, M);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    float* P = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.P);
    if (s->tile_cols == 64) {
        dim3 grid((s->K + kThreads - 1) / kThreads, (s->NB + kDxBlocksPerWG - 1) / kDxBlocksPerWG,
                  M);
        if (x_dtype == CSDR_F16)
            dx_b64_kernel<_Float16><<<grid, kThreads, 0, st>>>(
                s->d_dict, static_cast<const _Float16*>(x), s->K, s->NB, M, P);
        else
            dx_b64_kernel<float><<<grid, kThreads, 0, st>>>(
                s->d_dict, static_cast<const float*>(x), s->K, s->NB, M, P);
    } else {
        const long long waves = (long long)s->NB * s->K * ((M + 7) / 8);
        const int grid = (int)((waves * 64 + kThreads - 1) / kThreads);
        if (x_dtype == CSDR_F16)
            dx_generic_kernel<_Float16><<<grid, kThreads, 0, st>>>(
                s->d_dict, static_cast<const _Float16*>(x), s->K, s->NB, s->tile_cols, M, P);
        else
            dx_generic_kernel<float><<<grid, kThreads, 0, st>>>(
                s->d_dict, static_cast<const float*>(x), s->K, s->NB, s->tile_cols, M, P);
    }
    CSDR_LAUNCH_CHECK("hsdb dx");
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_gather(const csdr_hsdb* s, const void* x, int x_dtype, int M, float* y,
                              void* workspace, size_t workspace_bytes, void* hip_stream) {
    int rc = check_matmul_args(s, x, x_dtype, M, workspace, workspace_bytes, "hsdb_gather");
    if (rc) return rc;
    if (!y) return set_error(CSDR_E_INVALID, "hsdb_gather: null y");
    const WsLayout wl = ws_layout(s, M);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    char* ws = static_cast<char*>(workspace);
    GatherParams p{};
    p.codes = s->d_codes;
    p.P = reinterpret_cast<float*>(ws + wl.P);
    p.slot_gamma = s->d_slot_gamma;
    p.edge = s->d_edge;
    p.x = x;
    p.y = y;
    p.ypart = reinterpret_cast<float*>(ws + wl.ypart);
    p.counters = reinterpret_cast<unsigned int*>(ws + wl.counters);
    p.x_f16 = (x_dtype == CSDR_F16);
    p.R = (int)s->R;
    p.K = (int)s->K;
    p.NB = (int)s->NB;
    p.NBc = (int)s->NBc;
    p.nchunks = (int)s->nchunks;
    p.slots = (int)s->slots;
    p.M = M;
    p.Ce = (int)s->Ce;
    p.C_full = (int)s->C_full;
    const int MV = (M == 1) ? 1 : 4;
    p.MVz = (M + MV - 1) / MV;
    int Rt = gather_rows_per_wg(MV);
    int maxit = (Rt * (int)s->NBc + kThreads - 1) / kThreads;
    while (maxit > 8) {
        Rt /= 2;
        maxit = (Rt * (int)s->NBc + kThreads - 1) / kThreads;
    }
    int mi = 1;
    while (mi < maxit) mi <<= 1;
    p.Rt = Rt;
    p.nrt = ((int)s->R + Rt - 1) / Rt;
    const size_t lds = ((size_t)s->NBc * s->K * MV + (size_t)Rt * s->NBc * MV) * 4;
    if (lds > 160 * 1024)
        return set_error(CSDR_E_UNSUPPORTED, "hsdb_gather: dictionary too large for LDS");
    const int grid = 8 * ((p.nchunks + 7) / 8) * p.nrt;
    const int slots_t = (s->slots == 4 || s->slots == 8 || s->slots == 16 || s->slots == 24)
                            ? (int)s->slots
                            : 0;
    hipError_t e = (MV == 1) ? launch_gather<1>(p, mi, slots_t, grid, lds, st)
                             : launch_gather<4>(p, mi, slots_t, grid, lds, st);
    if (e != hipSuccess)
        return set_error(CSDR_E_HIP, std::string("hsdb gather launch failed: ") +
                                         hipGetErrorString(e));
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_matmul(const csdr_hsdb* s, const void* x, int x_dtype, int M, float* y,
                              void* workspace, size_t workspace_bytes, void* hip_stream) {
    int rc = csdr_hsdb_dx(s, x, x_dtype, M, workspace, workspace_bytes, hip_stream);
    if (rc) return rc;
    return csdr_hsdb_gather(s, x, x_dtype, M, y, workspace, workspace_bytes, hip_stream);
}

CSDR_API int csdr_hsdb_decompress(const csdr_hsdb* s, float* w, void* hip_stream) {
    if (!s || !w) return set_error(CSDR_E_INVALID, "hsdb_decompress: bad argument");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const size_t work = (size_t)s->n_tiles * s->tile_rows * s->tile_cols;
    if (work) {
        decode_dense_kernel<<<grid_for(work), kThreads, 0, st>>>(*s, w);
        CSDR_LAUNCH_CHECK("hsdb decode");
    }
    if (s->edge_floats) {
        decode_edge_kernel<<<grid_for(s->edge_floats), kThreads, 0, st>>>(*s, w);
        CSDR_LAUNCH_CHECK("hsdb edge");
    }
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_export_codes(const csdr_hsdb* s, uint16_t* packed, uint16_t* coef_abs,
                                    void* hip_stream) {
    if (!s || !packed) return set_error(CSDR_E_INVALID, "hsdb_export_codes: bad argument");
    const size_t work = (size_t)s->n_tiles * s->slots;
    if (work) {
        export_codes_kernel<<<grid_for(work), kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(
            *s, packed, coef_abs);
        CSDR_LAUNCH_CHECK("hsdb export");
    }
    return CSDR_OK;
}

}  // extern "C"
