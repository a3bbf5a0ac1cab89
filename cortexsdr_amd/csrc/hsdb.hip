// hsdb.hip — device-resident HSDR/HSDB segments and their kernels (gfx950).
//
// Path (cortexSDR tree): HierarchicalSDRStrategy::matmulRowMajor
// (strategies/HierarchicalSDRStrategy.cpp:1257-1338) and decompress (:1340-1440), with the
// block-coded "HSDB" generalisation of research exp_c_kernel/benchmark.py:106-130.
//
// Math. W is R x C; tile (r, b) covers W[r, b*B : b*B+B] (1-row tiles, B = tile_cols) and
// is sum_j c_j * D[idx_j] over its S*k coded slots, c_j = gamma_{j/k} * signed fp16 |c|
// (binary HSDR: |c| = 1). Y = W.X is computed without W, for a group of up to 8 matrices
// per call, in two launches:
//   dx:     P[b][a][m] = D[a] . X[b*B : b*B+B, m] (the reference's Dx precompute), Y = 0
//   gather: Y[r][m] += sum_b sum_j c_j * P[b][idx_j][m] (+ fp32 edge strip . X)
//
// Device code layout (built at load time; 4 bytes per slot, the stream's own byte count):
//   word = (signed fp16 coefficient bits << 16) | atom index (15 bits)
// ordered chunk-major: block columns are grouped in chunks of NBc; chunk c holds, for
// every row r, the NBc tiles (r, c*NBc .. c*NBc+NBc-1) back to back, so the rows of one
// chunk are one contiguous run. 2-D tiles (tile_rows > 1, decode only) keep the stream's
// tile-major order.
//
// The M == 1 gather is persistent: a workgroup owns (chunk, row range), stages the chunk's
// P slice in LDS once and streams its run with three units of 16-byte loads in flight
// (each wave instruction reads 1 KiB contiguous), gathers from LDS and adds each row's
// total into Y with device-scope float atomics (other chunks of the row run on other
// workgroups), so the summation order over chunks is not fixed: results agree to fp32
// rounding, not bit for bit. Workgroups of one chunk are numbered to share an XCD
// (dispatch is round-robin over the 8 XCDs), which keeps the P slice in one L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"
#include "hsdb_impl.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Word 3 of a raw (stride 0) buffer resource on CDNA: 32-bit data format, no swizzle; with it a
// lane whose offset is at or past num_records reads zeros and makes no memory access.
constexpr int kRawBufferDword3 = 0x00020000;
constexpr int kCachePolicyNT = 2;  // buffer load cache policy: nontemporal (streaming)

// A switch from the environment: "0" is off, any other value on, unset is dflt.
bool env_flag(const char* name, bool dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return v[0] != '0';
}

constexpr uint32_t kMaxChunkBlocks = 16;
constexpr uint32_t kChunkPBytes = 16384;  // P slice of one chunk (nbc * K fp32), at most


// ------------------------------------------------------------------ matmul kernels

constexpr int kMaxGroup = 8;
constexpr int kMaxSlotsArg = 32;
constexpr int kStageBatch = 8;  // global loads in flight per thread while staging to LDS
constexpr int kMaxXopM = 16;  // columns an x op supports
constexpr int kMaxVecM = 8;   // columns of the streaming multi-column gather
constexpr int kAttnStatMax = 2048;  // (head, split) partials whose weights the combine keeps in LDS

// One coded matrix of a grouped launch.
struct MatDesc {
    const uint32_t* codes;
    const float* dict;
    const float* slot_gamma;
    const float* edge;
    const void* x;
    float* y;
    const float* bias;  // per output row, added once (nullable)
    float* P;  // NB * K * M floats of workspace
    const void* x2;  // second input of the x op (SiLU: the up projection)
    float* xe;       // x op: transformed edge-strip inputs, Ce x M (workspace), else null
    int R, K, NB, NBc, nchunks, slots, blen, Ce, C_full;
    int PB;                   // dx: block columns per workgroup (block length 64)
    int dx_base, dx_count;    // dx workgroup ids [base, base + count)
    int g_base, g_count;      // gather workgroup ids, base a multiple of 8
    int splits;               // gather workgroups per chunk
    int rows_per_wg;          // rows of a chunk handled by one gather workgroup
    int rsplit[4], rrpw[4];   // M == 1 gather: ranges and rows per range of the remainder chunks
    int Rt;                   // M > 1 gather: rows per workgroup
    float sgam[kMaxSlotsArg]; // gamma of each slot (slots <= kMaxSlotsArg; scalar loads)
    int gunif;                // every slot has gamma sgam[0]
};

struct Params {
    MatDesc m[kMaxGroup];
    int G, M, MVz, x_f16;
    int tm;  // token-major X (M x C) and Y (M x R) instead of feature-major (C x M, R x M)
    int accumulate;  // 1: Y += W.X (+ bias); 0: Y = W.X (+ bias)
    // input transform applied while staging x (csdr_hsdb_matmul_group_xop)
    int xop;          // CSDR_XOP_*
    const float* nw;  // RMSNorm weights (C)
    float* inv;       // M > 1: per (matrix, column) 1 / rms, [g * 16 + m] (workspace head)
    float eps;
    int nsplit, hd;   // attention combine: splits and head size of the partials in x
    int gtotal;       // 2 <= M <= 8: gather units of all matrices (the launch is padded to 8s)
    int p16;          // 5 <= M <= 8 on the multi-column gather: P is fp16 [block][atom][8]
};

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over each row of 16 lanes, result in every lane of the row: pair swap, quad swap,
// half-row mirror, row mirror (DPP moves, no LDS round trip).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x141>(v);  // row_half_mirror
    v += dpp_move<0x140>(v);  // row_mirror
    return v;
}

template <typename XT>
__device__ __forceinline__ float xval(const void* x, size_t i) {
    return csdr::to_f32(static_cast<const XT*>(x)[i]);
}
__device__ __forceinline__ float xload(const void* x, int f16, size_t i) {
    return f16 ? xval<_Float16>(x, i) : xval<float>(x, i);
}

// Element (feature k, column m) of X (and of the x op's second input), and element (row r,
// column m) of Y, in the call's layout: feature-major (the reference matmulRowMajor's C x M /
// R x M) or token-major (linear_forward's M x C / M x R).
__device__ __forceinline__ size_t xi(const Params& p, const MatDesc& d, int k, int m) {
    return p.tm ? (size_t)m * (d.C_full + d.Ce) + k : (size_t)k * p.M + m;
}
__device__ __forceinline__ size_t yi(const Params& p, const MatDesc& d, int r, int m) {
    return p.tm ? (size_t)m * d.R + r : (size_t)r * p.M + m;
}

// xs[i] = float(src[i]) for i < n by the whole workgroup, kStageBatch independent loads
// per thread in flight at a time (branch-free: out-of-range lanes reload the last element).
// (clamped loads and unconditional clamped stores: lanes past the end rewrite element n - 1
// with its own value; a conditional store would let the compiler sink each load into its
// branch and wait for all loads in flight before every store)
template <typename T, int NT = kThreads>
__device__ __forceinline__ void stage_to_lds(const T* __restrict__ src, int n, float* xs) {
    const int tid = threadIdx.x;
    for (int i0 = 0; i0 < n; i0 += NT * kStageBatch) {
        float v[kStageBatch];
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j)
            v[j] = csdr::to_f32(src[min(i0 + j * NT + tid, n - 1)]);
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j) xs[min(i0 + j * NT + tid, n - 1)] = v[j];
    }
}

// Copies n floats (n % 4 == 0, 16-byte aligned) global -> LDS, batched like stage_to_lds.
__device__ __forceinline__ void copy_to_lds4(const float* __restrict__ src, int n, float* dst) {
    const int tid = threadIdx.x;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    float4* d4 = reinterpret_cast<float4*>(dst);
    const int n4 = n >> 2;
    for (int i0 = 0; i0 < n4; i0 += kThreads * kStageBatch) {
        float4 v[kStageBatch];
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j) v[j] = s4[min(i0 + j * kThreads + tid, n4 - 1)];
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j) d4[min(i0 + j * kThreads + tid, n4 - 1)] = v[j];
    }
}

// ---- kernel 1 (dx): P[b][a][m] = D[a] . X[b*B : b*B+B, m] (the reference's Dx precompute)
// and Y = 0 (the gathers accumulate into Y). Visibility to the gather kernel comes from the
// dispatch boundary.
// ---- input transforms fused into the dx staging (x op)

// Workgroup sum of v (NT threads), result in every thread.
template <int NT = kThreads>
__device__ __forceinline__ float wg_sum(float v, float* red) {
    v = csdr::wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += red[i];
    return t;
}

// Attention split partials in attn_decode's workspace (M == 1, so n = heads * nsplit of them,
// partial i = head * nsplit + split): the n (max, sum) pairs first, then the n unnormalised
// head_dim vectors (from csdr::attn_vec_offset(n)).
__device__ __forceinline__ const float* attn_stats(const float* part, int h, int ns) {
    return part + (size_t)2 * h * ns;
}
__device__ __forceinline__ const float* attn_vecs(const float* part, int nh, int h, int ns,
                                                  int hd) {
    return part + csdr::attn_vec_offset((size_t)nh * ns) + (size_t)h * ns * hd;
}

// Attention output feature k (head k / hd, dim k % hd) of nh heads combined from the split
// partials.
__device__ __forceinline__ float attn_feature(const Params& p, const float* part, int nh, int k) {
    const int h = k / p.hd, dd = k - h * p.hd, ns = p.nsplit;
    const float* pst = attn_stats(part, h, ns);
    const float* pv = attn_vecs(part, nh, h, ns, p.hd) + dd;
    float Mx = -INFINITY;
    for (int s = 0; s < ns; ++s) Mx = fmaxf(Mx, pst[2 * s]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < ns; ++s) {
        const float ms = pst[2 * s];
        if (ms == -INFINITY) continue;
        const float w = expf(ms - Mx);
        den = fmaf(w, pst[2 * s + 1], den);
        num = fmaf(w, pv[(size_t)s * p.hd], num);
    }
    return den > 0.f ? num / den : 0.f;
}

// x op of element (feature k, column m) given the raw value v (and inv[m] for RMSNorm).
__device__ __forceinline__ float xop_apply(const Params& p, const MatDesc& d, float v, int k,
                                           int m, const float* inv) {
    if (p.xop == CSDR_XOP_RMSNORM) return v * inv[m] * p.nw[k];
    if (p.xop == CSDR_XOP_SILU_MUL) {
        const float u = static_cast<const float*>(d.x2)[xi(p, d, k, m)];
        return (v * (1.0f / (1.0f + expf(-v)))) * u;
    }
    return v;
}

// Stages x features [64 b0, 64 (b0 + nb)) x M columns into xs (fp32, [feature][column])
// with the call's x op applied (RMSNorm, SiLU(x) * x2, attention combine); with do_xe also
// writes the transformed edge-strip inputs to d.xe. A workgroup of NT threads; ends with a
// barrier.
template <int NT = kThreads>
__device__ void stage_x_chunk(const Params& p, const MatDesc& d, int b0, int nb, float* xs,
                              bool do_xe) {
    const int tid = threadIdx.x;
    const int M = p.M;
    float* const xe = d.xe;
    const size_t xbase = (size_t)b0 * 64 * M;
    const int nx = nb * 64 * M;
    __shared__ float inv[kMaxXopM];
    __shared__ float red[NT / 64];
    if (p.xop == CSDR_XOP_RMSNORM) {
        // 1 / rms of every column over all C features (each workgroup recomputes it: x is
        // a few KiB, L2-resident)
        const float* xf = static_cast<const float*>(d.x);
        const int C = d.C_full + d.Ce;
        for (int m = 0; m < M; ++m) {
            float ss = 0.f;
            for (int k = tid; k < C; k += NT) {
                const float v = xf[xi(p, d, k, m)];
                ss = fmaf(v, v, ss);
            }
            ss = wg_sum<NT>(ss, red);
            if (tid == 0) inv[m] = 1.0f / sqrtf(ss / (float)C + p.eps);
        }
    }
    if (p.xop == CSDR_XOP_ATTN) {
        // per head of this range: split weights exp(m_s - max) and 1 / sum(w_s l_s) in
        // LDS once, then every feature is one weighted sum over the splits
        const float* part = static_cast<const float*>(d.x);
        const int hd = p.hd, ns = p.nsplit, nh = (d.C_full + d.Ce) / hd;
        const int h0 = (b0 * 64) / hd, h1 = (b0 * 64 + nx - 1) / hd + 1;
        float* wts = xs + nx;  // (h1 - h0) x (ns + 1)
        for (int h = h0 + tid; h < h1; h += NT) {
            const float* pst = attn_stats(part, h, ns);
            float Mx = -INFINITY;
            for (int s2 = 0; s2 < ns; ++s2) Mx = fmaxf(Mx, pst[2 * s2]);
            float den = 0.f;
            float* wh = wts + (h - h0) * (ns + 1);
            for (int s2 = 0; s2 < ns; ++s2) {
                const float ms = pst[2 * s2];
                const float w = ms == -INFINITY ? 0.f : expf(ms - Mx);
                wh[s2] = w;
                den = fmaf(w, pst[2 * s2 + 1], den);
            }
            wh[ns] = den > 0.f ? 1.0f / den : 0.f;
        }
        __syncthreads();
        for (int i = tid; i < nx; i += NT) {
            const int k = b0 * 64 + i, h = k / hd, dd = k - h * hd;
            const float* wh = wts + (h - h0) * (ns + 1);
            const float* po = attn_vecs(part, nh, h, ns, hd) + dd;
            float num = 0.f;
            for (int s2 = 0; s2 < ns; ++s2) num = fmaf(wh[s2], po[(size_t)s2 * hd], num);
            xs[i] = num * wh[ns];
        }
    } else if (p.tm && M > 1) {
        // token-major X: element (feature f0 + i / M, column i % M), kStageBatch loads in flight
        const int f0 = b0 * 64;
        for (int i0 = 0; i0 < nx; i0 += NT * kStageBatch) {
            float v[kStageBatch];
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) {
                const int i = min(i0 + j * NT + tid, nx - 1);
                v[j] = xload(d.x, p.x_f16, xi(p, d, f0 + i / M, i % M));
            }
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) xs[min(i0 + j * NT + tid, nx - 1)] = v[j];
        }
    } else if (p.x_f16) {
        stage_to_lds<_Float16, NT>(static_cast<const _Float16*>(d.x) + xbase, nx, xs);
    } else {
        stage_to_lds<float, NT>(static_cast<const float*>(d.x) + xbase, nx, xs);
    }
    if (p.xop == CSDR_XOP_RMSNORM || p.xop == CSDR_XOP_SILU_MUL) {
        __syncthreads();
        for (int i = tid; i < nx; i += NT) {
            const int k = b0 * 64 + i / M, m = i % M;
            xs[i] = xop_apply(p, d, xs[i], k, m, inv);
        }
        if (do_xe && xe) {
            const float* xf = static_cast<const float*>(d.x);
            for (int t = tid; t < d.Ce * M; t += NT) {
                const int cc = t / M, m = t % M;
                const int k = d.C_full + cc;
                xe[t] = xop_apply(p, d, xf[xi(p, d, k, m)], k, m, inv);
            }
        }
    } else if (p.xop == CSDR_XOP_ATTN && do_xe && xe) {
        const float* part = static_cast<const float*>(d.x);
        const int nh = (d.C_full + d.Ce) / p.hd;
        for (int t = tid; t < d.Ce; t += NT) xe[t] = attn_feature(p, part, nh, d.C_full + t);
    }
    __syncthreads();
}

// M == 1 staging of x features [64 b0, 64 (b0 + nb)) (nb * 64 <= 4 NT) with the call's x op
// applied, into xs, and with do_xe the transformed edge-strip inputs into d.xe. Every global
// load is issued before the first wait, so the staging costs one memory round trip where the
// generic one makes up to three dependent ones (RMSNorm: the sum of squares, then x, then the
// weights). The attention combine weighs each split by exp(m_j - M) / sum_j exp(m_j - M) l_j,
// computed once per head into LDS (a single split is a division; more partials than the LDS
// table holds take one pass with a running maximum). Ends with a barrier.
// XOP: the call's x op (CSDR_XOP_*), fixed at compile time so that each kind gets only the
// registers it needs.
template <int NT, int XOP>
__device__ void stage_x_m1(const Params& p, const MatDesc& d, int b0, int nb, float* xs,
                           bool do_xe) {
    constexpr int kPer = 4;         // features per thread
    constexpr int kSlots = kPer + 1;  // + the edge-strip input
    const int tid = threadIdx.x;
    const int nx = nb * 64, f0 = b0 * 64;
    const int C = d.C_full + d.Ce;
    __shared__ float red[NT / 64];
    int feat[kSlots];
#pragma unroll
    for (int i = 0; i < kPer; ++i) feat[i] = f0 + min(tid + i * NT, nx - 1);
    feat[kPer] = min(d.C_full + tid, C - 1);
    float v[kSlots];
    if constexpr (XOP == CSDR_XOP_ATTN) {
        // thread t: features 4t .. 4t + 3 of the range, one head (head_dim % 4 == 0), one
        // 16-byte load per split
        const float* part = static_cast<const float*>(d.x);
        const int hd = p.hd, ns = p.nsplit, nh = C / hd;
        const int nst = nh * ns;  // (head, split) partials
        const int fl = min(4 * tid, nx - 4), f = f0 + fl;
        const int h = ((hd & (hd - 1)) == 0) ? f >> (__ffs(hd) - 1) : f / hd;
        const float* pst = attn_stats(part, h, ns);
        const float4* pv = reinterpret_cast<const float4*>(attn_vecs(part, nh, h, ns, hd) + (f - h * hd));
        const int vs = hd / 4;  // float4 stride between splits
        constexpr int kSB = 12;  // splits per round trip
        float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ns == 1) {
            // one split: its sum over its normaliser
            const float m = pst[0], l = pst[1];
            const float4 o = pv[0];
            if (m != -INFINITY && l > 0.f) r = make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
        } else if (ns <= 64 && nst * 2 <= kAttnStatMax) {
            // The split weights w_j = exp(m_j - M) / sum_j exp(m_j - M) l_j depend on the head
            // only: thread (head, split) pairs in lane groups of GS >= ns splits (max and sum
            // by shuffles within the group), loaded in the same round trip as this thread's
            // first partial values, weights into LDS; then each feature is a weighted sum.
            __shared__ float wst[kAttnStatMax];
            constexpr int kStatPT = kAttnStatMax / NT;
            int GS = 1;
            while (GS < ns) GS <<= 1;
            const int ngs = nh * GS;  // < 2 nst
            // (every load is issued, at clamped indices: a conditional load here made the
            // compiler wait for all earlier loads before each one)
            float2 ml[kStatPT];
#pragma unroll
            for (int k = 0; k < kStatPT; ++k) {
                const int e = min(tid + k * NT, ngs - 1), hh = min(e / GS, nh - 1),
                          j = min(e % GS, ns - 1);
                ml[k] = reinterpret_cast<const float2*>(part)[hh * ns + j];
            }
            // the values of the first two rounds of kSB splits (2 kSB covers the splits of
            // every shape measured here), in flight during the weights
            float4 oa[kSB], ob[kSB];
#pragma unroll
            for (int j = 0; j < kSB; ++j) oa[j] = pv[min(j, ns - 1) * vs];
#pragma unroll
            for (int j = 0; j < kSB; ++j) ob[j] = pv[min(kSB + j, ns - 1) * vs];
#pragma unroll
            for (int k = 0; k < kStatPT; ++k) {
                if (k * NT >= ngs) break;
                const int e = tid + k * NT, hh = e / GS, j = e % GS;
                const bool live = hh < nh && j < ns;
                const float m = live ? ml[k].x : -INFINITY;
                float M = m;
                for (int off = GS >> 1; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
                const float ex = m == -INFINITY ? 0.f : expf(m - M);
                float den = live ? ex * ml[k].y : 0.f;
                for (int off = GS >> 1; off > 0; off >>= 1) den += __shfl_xor(den, off, 64);
                if (live) wst[hh * ns + j] = den > 0.f ? ex / den : 0.f;
            }
            __syncthreads();
            const float* wr = wst + h * ns;
            // the first two rounds are summed from the loads issued above. Every load is issued,
            // at clamped indices, and every value used (with weight 0 past the last split), so
            // that no load is left to wait on its own: loads placed under a per-split branch
            // ran one round trip at a time.
            auto add_round = [&](const float4 (&o)[kSB], int s0) {
#pragma unroll
                for (int j = 0; j < kSB; ++j) {
                    const int sj = s0 + j;
                    const float w = sj < ns ? wr[min(sj, ns - 1)] : 0.f;
                    r.x = fmaf(w, o[j].x, r.x);
                    r.y = fmaf(w, o[j].y, r.y);
                    r.z = fmaf(w, o[j].z, r.z);
                    r.w = fmaf(w, o[j].w, r.w);
                }
            };
            add_round(oa, 0);
            add_round(ob, kSB);
            // more than 2 kSB splits: the rest a round at a time
            for (int s0 = 2 * kSB; s0 < ns; s0 += kSB) {
#pragma unroll
                for (int j = 0; j < kSB; ++j) oa[j] = pv[min(s0 + j, ns - 1) * vs];
                add_round(oa, s0);
            }
        } else {
            // more partials than the LDS table holds: one pass over the splits, four at a
            // time, with a running maximum (online softmax)
            constexpr int kSBo = 4;
            float M = -INFINITY, den = 0.f;
            float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s0 = 0; s0 < ns; s0 += kSBo) {
                float ms[kSBo], ls[kSBo];
                float4 os[kSBo];
#pragma unroll
                for (int j = 0; j < kSBo; ++j) {
                    const int sj = min(s0 + j, ns - 1);
                    ms[j] = pst[2 * sj];
                    ls[j] = pst[2 * sj + 1];
                    os[j] = pv[sj * vs];
                }
#pragma unroll
                for (int j = 0; j < kSBo; ++j) {
                    if (s0 + j >= ns || ms[j] == -INFINITY) continue;
                    const float Mn = fmaxf(M, ms[j]);
                    const float a = expf(M - Mn), b = expf(ms[j] - Mn);
                    den = fmaf(den, a, b * ls[j]);
                    num.x = fmaf(num.x, a, b * os[j].x);
                    num.y = fmaf(num.y, a, b * os[j].y);
                    num.z = fmaf(num.z, a, b * os[j].z);
                    num.w = fmaf(num.w, a, b * os[j].w);
                    M = Mn;
                }
            }
            if (den > 0.f) r = make_float4(num.x / den, num.y / den, num.z / den, num.w / den);
        }
        if (4 * tid < nx) *reinterpret_cast<float4*>(xs + 4 * tid) = r;
        if (do_xe && d.xe && tid < d.Ce) d.xe[tid] = attn_feature(p, part, nh, d.C_full + tid);
        __syncthreads();
        return;
    } else {
        float w[kSlots];
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
            v[i] = xload(d.x, p.x_f16, (size_t)feat[i]);
            if constexpr (XOP == CSDR_XOP_RMSNORM) w[i] = p.nw[feat[i]];
            if constexpr (XOP == CSDR_XOP_SILU_MUL) w[i] = static_cast<const float*>(d.x2)[feat[i]];
        }
        if constexpr (XOP == CSDR_XOP_RMSNORM) {
            // 1 / rms over all C features (x ops take fp32 x)
            const float* xf = static_cast<const float*>(d.x);
            float ss = 0.f;
            for (int j0 = 0; j0 < C; j0 += NT * kStageBatch) {
                float t[kStageBatch];
#pragma unroll
                for (int j = 0; j < kStageBatch; ++j) t[j] = xf[min(j0 + j * NT + tid, C - 1)];
#pragma unroll
                for (int j = 0; j < kStageBatch; ++j)
                    if (j0 + j * NT + tid < C) ss = fmaf(t[j], t[j], ss);
            }
            ss = wg_sum<NT>(ss, red);
            const float inv = 1.0f / sqrtf(ss / (float)C + p.eps);
#pragma unroll
            for (int i = 0; i < kSlots; ++i) v[i] = v[i] * inv * w[i];
        } else if constexpr (XOP == CSDR_XOP_SILU_MUL) {
#pragma unroll
            for (int i = 0; i < kSlots; ++i) v[i] = (v[i] * (1.0f / (1.0f + expf(-v[i])))) * w[i];
        }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (tid + i * NT < nx) xs[tid + i * NT] = v[i];
    if (do_xe && XOP != CSDR_XOP_NONE && d.xe && tid < d.Ce) d.xe[tid] = v[kPer];
    __syncthreads();
}

// XOP: p.xop at compile time (the M == 1 staging's registers depend on it)
template <int XOP>
__global__ __launch_bounds__(kThreads) void dx_kernel(Params p) {
    extern __shared__ float smem[];
    const int wg = blockIdx.x;
    int g = 0;
    while (g + 1 < p.G && wg >= p.m[g + 1].dx_base) ++g;
    const MatDesc& d = p.m[g];
    const int u = wg - d.dx_base;
    const int tid = threadIdx.x;
    const int M = p.M;
    {
        // Y initialisation for the gathers' accumulation: 0 or bias, or left as it is (+ bias)
        const size_t ytot = (size_t)d.R * M;
        const size_t yper = (ytot + d.dx_count - 1) / d.dx_count;
        const size_t ye = min(ytot, (size_t)(u + 1) * yper);
        // (kept with no bias: nothing to do, and no read of y to wait for)
        if (!p.accumulate || d.bias) {
            for (size_t i = (size_t)u * yper + tid; i < ye; i += kThreads) {
                const float bv = d.bias ? d.bias[p.tm ? i % d.R : i / M] : 0.0f;
                d.y[i] = p.accumulate ? d.y[i] + bv : bv;
            }
        }
    }
    if (d.blen == 64) {
        // 16 lanes per atom: lane l holds D[a][4l .. 4l+3] (one coalesced 16-byte load; a
        // wave reads 4 whole rows). The x range of this workgroup is staged in LDS in one
        // coalesced pass; per (block, column) each lane does 4 FMAs against its 4 x values
        // and a 4-step DPP butterfly sums the 16 lanes.
        const int l16 = tid & 15;
        const int na16 = (d.K + 15) / 16;
        const int ag = u % na16, bg = u / na16;
        const int a = ag * 16 + (tid >> 4);
        const int b0 = bg * d.PB;
        const int nb = min(d.PB, d.NB - b0);
        const bool live = a < d.K;
        float4 dv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) dv = reinterpret_cast<const float4*>(d.dict + (size_t)a * 64)[l16];
        float* xs = smem;  // [bb][t][m], nb * 64 * M floats (x rows are contiguous)
        if (M == 1 && nb * 64 <= 4 * kThreads)
            stage_x_m1<kThreads, XOP>(p, d, b0, nb, xs, u == 0);
        else
            stage_x_chunk(p, d, b0, nb, xs, u == 0);
        float* const Pout = d.P + (size_t)b0 * d.K * M + (size_t)a * M;  // + bb*K*M + m
        const size_t pstride = (size_t)d.K * M;
        int bb = 0;
        if (M == 1) {
            // four independent (block) dot products per step so the DPP chains interleave
            for (; bb + 4 <= nb; bb += 4) {
                float sum[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 xv =
                        *reinterpret_cast<const float4*>(xs + (bb + q) * 64 + 4 * l16);
                    float t = dv.x * xv.x;
                    t = fmaf(dv.y, xv.y, t);
                    t = fmaf(dv.z, xv.z, t);
                    sum[q] = fmaf(dv.w, xv.w, t);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) sum[q] = row16_sum(sum[q]);
                if (live && l16 == 0) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) Pout[(bb + q) * pstride] = sum[q];
                }
            }
        }
        for (; bb < nb; ++bb) {
            for (int m = 0; m < M; ++m) {
                float4 xv;
                if (M == 1) {
                    xv = *reinterpret_cast<const float4*>(xs + bb * 64 + 4 * l16);
                } else {
                    const float* xp = xs + ((size_t)bb * 64 + 4 * l16) * M + m;
                    xv = make_float4(xp[0], xp[M], xp[2 * M], xp[3 * M]);
                }
                float sum = dv.x * xv.x;
                sum = fmaf(dv.y, xv.y, sum);
                sum = fmaf(dv.z, xv.z, sum);
                sum = fmaf(dv.w, xv.w, sum);
                sum = row16_sum(sum);
                if (live && l16 == 0) Pout[bb * pstride + m] = sum;
            }
        }
    } else {
        // any block length (the reference's own 1-row geometry has blocks of C features): one
        // wave per (b, a, group of 8 columns), lane-strided dot. Rounds of kR features per
        // lane with every load of a round issued before its first use, at clamped indices and
        // with the element type's branch around the round (a load per feature under that
        // branch ran one round trip per feature); lanes past the block keep their sums.
        constexpr int kR = 8;
        const int lane = tid & 63;
        const int mg = (M + 7) / 8;
        const long long item = (long long)u * (kThreads / 64) + (tid >> 6);
        if (item < (long long)d.NB * d.K * mg) {
            const int gi = (int)(item % mg);
            const long long ba = item / mg;
            const int b = (int)(ba / d.K), a = (int)(ba % d.K);
            const int m0 = gi * 8, nm = min(8, M - m0);
            float acc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
            const float* drow = d.dict + (size_t)a * d.blen;
            for (int t0 = 0; t0 < d.blen; t0 += 64 * kR) {
                float dv[kR];
                size_t xo[kR];
#pragma unroll
                for (int r = 0; r < kR; ++r) {
                    const int t = min(t0 + r * 64 + lane, d.blen - 1);
                    dv[r] = drow[t];
                    xo[r] = xi(p, d, b * d.blen + t, m0);
                }
                if (nm == 1) {
                    float xv[kR];
                    if (p.x_f16) {
#pragma unroll
                        for (int r = 0; r < kR; ++r) xv[r] = xval<_Float16>(d.x, xo[r]);
                    } else {
#pragma unroll
                        for (int r = 0; r < kR; ++r) xv[r] = xval<float>(d.x, xo[r]);
                    }
#pragma unroll
                    for (int r = 0; r < kR; ++r)
                        if (t0 + r * 64 + lane < d.blen) acc[0] = fmaf(dv[r], xv[r], acc[0]);
                } else {
                    // the columns of feature t: xo + j (feature-major) or + j * C (token-major)
                    const size_t cs = p.tm ? (size_t)(d.C_full + d.Ce) : 1;
                    float xv[kR][8];
                    if (p.x_f16) {
#pragma unroll
                        for (int r = 0; r < kR; ++r)
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                xv[r][j] = xval<_Float16>(d.x, xo[r] + (size_t)min(j, nm - 1) * cs);
                    } else {
#pragma unroll
                        for (int r = 0; r < kR; ++r)
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                xv[r][j] = xval<float>(d.x, xo[r] + (size_t)min(j, nm - 1) * cs);
                    }
#pragma unroll
                    for (int r = 0; r < kR; ++r)
                        if (t0 + r * 64 + lane < d.blen)
#pragma unroll
                            for (int j = 0; j < 8; ++j) acc[j] = fmaf(dv[r], xv[r][j], acc[j]);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = csdr::wave_sum(acc[j]);
            if (lane == 0)
                for (int j = 0; j < nm; ++j) d.P[((size_t)b * d.K + a) * M + m0 + j] = acc[j];
        }
    }
}

// ---- kernel 1 at M == 1 with 64-long blocks: P[b][a] = D[a] . x_b as a
// small product P^T (K x NB) = D (K x 64) . [x_0 .. x_NB-1] (64 x NB) on the fp32 matrix
// cores (v_mfma_f32_16x16x4_f32). Workgroup = NT / 64 waves x 16 atoms and 16 block
// columns, wave w the atoms 16 w .. 16 w + 15 of the workgroup's; lane l supplies atom l % 16
// (A) and block column l % 16 (B), and the contraction over a block's 64 features runs with
// lane group l / 16 taking features 16 (l / 16) .. + 15 in its 16 steps, so each lane's
// operands are one contiguous 64-byte run of the dictionary row and of x, loaded straight
// from memory (no LDS, no cross-lane sums). Lane l ends with P[block l % 16][atoms
// 4 (l / 16) .. + 3]. Y is initialised as in dx_kernel; the x op (RMSNorm with its statistic
// over all C features, or SiLU . x2) is applied to the B operand in registers; the attention
// combine is staged for the workgroup's blocks in LDS first (stage_x_m1).
template <int XOP, int NT>
__device__ __forceinline__ void dx1_body(const Params& p, int wg) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    constexpr int kAtoms = NT / 4;  // 16 per wave
    int g = 0;
    while (g + 1 < p.G && wg >= p.m[g + 1].dx_base) ++g;
    const MatDesc& d = p.m[g];
    const int u = wg - d.dx_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    {
        const size_t ytot = (size_t)d.R;
        const size_t yper = (ytot + d.dx_count - 1) / d.dx_count;
        const size_t ye = min(ytot, (size_t)(u + 1) * yper);
        // (kept with no bias: nothing to do, and no read of y to wait for)
        if (!p.accumulate || d.bias) {
            for (size_t i = (size_t)u * yper + tid; i < ye; i += NT) {
                const float bv = d.bias ? d.bias[i] : 0.0f;
                d.y[i] = p.accumulate ? d.y[i] + bv : bv;
            }
        }
    }
    const int na = (d.K + kAtoms - 1) / kAtoms;
    const int ag = u % na, bg = u / na;
    const int a = min(ag * kAtoms + wave * 16 + li, d.K - 1);
    const int b = min(bg * 16 + li, d.NB - 1);
    const int f0 = b * 64 + lg * 16;  // this lane's 16 features
    f4 dv[4];
    {
        const f4* src = reinterpret_cast<const f4*>(d.dict + (size_t)a * 64 + lg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) dv[i] = src[i];
    }
    float xv[16];
    if constexpr (XOP == CSDR_XOP_ATTN) {
        // the split-attention combine for the workgroup's 16 blocks (1024 features, one per
        // 4 threads' float4) into LDS, then this lane's 16 features from there
        __shared__ __attribute__((aligned(16))) float xs_attn[16 * 64];
        const int b0 = bg * 16;
        stage_x_m1<NT, XOP>(p, d, b0, min(16, d.NB - b0), xs_attn, u == 0);  // (ends in a barrier)
        const f4* src = reinterpret_cast<const f4*>(xs_attn + (b - b0) * 64 + lg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f4 v = src[i];
            xv[4 * i] = v.x;
            xv[4 * i + 1] = v.y;
            xv[4 * i + 2] = v.z;
            xv[4 * i + 3] = v.w;
        }
    } else if (p.x_f16) {
        const u4* src = reinterpret_cast<const u4*>(static_cast<const _Float16*>(d.x) + f0);
        const u4 h0 = src[0], h1 = src[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[2 * i] = csdr::h2f(h0[i] & 0xFFFFu);
            xv[2 * i + 1] = csdr::h2f(h0[i] >> 16);
            xv[8 + 2 * i] = csdr::h2f(h1[i] & 0xFFFFu);
            xv[9 + 2 * i] = csdr::h2f(h1[i] >> 16);
        }
    } else {
        const f4* src = reinterpret_cast<const f4*>(static_cast<const float*>(d.x) + f0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f4 v = src[i];
            xv[4 * i] = v.x;
            xv[4 * i + 1] = v.y;
            xv[4 * i + 2] = v.z;
            xv[4 * i + 3] = v.w;
        }
    }
    const int C = d.C_full + d.Ce;
    float inv = 1.0f;
    if constexpr (XOP == CSDR_XOP_RMSNORM) {
        // 1 / rms over all C features (x ops take fp32 x); this lane's norm weights are
        // loaded first, so that their round trip overlaps the statistic's
        float nwv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) nwv[i] = p.nw[f0 + i];
        __shared__ float red[NT / 64];
        const float* xf = static_cast<const float*>(d.x);
        float ss = 0.f;
        for (int j0 = 0; j0 < C; j0 += NT * kStageBatch) {
            float t[kStageBatch];
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) t[j] = xf[min(j0 + j * NT + tid, C - 1)];
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j)
                if (j0 + j * NT + tid < C) ss = fmaf(t[j], t[j], ss);
        }
        ss = wg_sum<NT>(ss, red);
        inv = 1.0f / sqrtf(ss / (float)C + p.eps);
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[i] = xv[i] * inv * nwv[i];
    } else if constexpr (XOP == CSDR_XOP_SILU_MUL) {
        const float* x2 = static_cast<const float*>(d.x2) + f0;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            xv[i] = (xv[i] * (1.0f / (1.0f + expf(-xv[i])))) * x2[i];
    }
    if (XOP != CSDR_XOP_NONE && XOP != CSDR_XOP_ATTN && u == 0 && d.xe) {
        // the transformed edge-strip inputs (the attention combine writes its own)
        for (int t = tid; t < d.Ce; t += NT) {
            const int f = d.C_full + t;
            float x = xload(d.x, p.x_f16, (size_t)f);
            if constexpr (XOP == CSDR_XOP_RMSNORM) x = x * inv * p.nw[f];
            if constexpr (XOP == CSDR_XOP_SILU_MUL)
                x = (x * (1.0f / (1.0f + expf(-x)))) * static_cast<const float*>(d.x2)[f];
            d.xe[t] = x;
        }
    }
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(dv[s >> 2][s & 3], xv[s], acc, 0, 0, 0);
    const int bo = bg * 16 + li, ao = ag * kAtoms + wave * 16 + 4 * lg;
    if (bo < d.NB) {
        float* out = d.P + (size_t)bo * d.K + ao;
        if (ao + 3 < d.K && (d.K & 3) == 0) {
            // streamed past this XCD's L2: the gather reads P from every XCD (headline step
            // 15.64 -> 15.42 us)
            __builtin_nontemporal_store(acc, reinterpret_cast<f4*>(out));
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (ao + v < d.K) out[v] = acc[v];
        }
    }
}

template <int XOP>
__global__ __launch_bounds__(kThreads) void dx1_mfma_kernel(Params p) {
    dx1_body<XOP, kThreads>(p, (int)blockIdx.x);
}

// ---- RMSNorm statistics at M > 1: p.inv[g * 16 + m] = 1 / sqrt(mean_k x[k][m]^2 + eps) for
// matrix g = blockIdx.y, column m = blockIdx.x (one workgroup per column, once per call, so
// the dx workgroups read M values instead of all C x M inputs each).
__global__ __launch_bounds__(kThreads) void rms_inv_kernel(Params p) {
    const MatDesc& d = p.m[blockIdx.y];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int C = d.C_full + d.Ce;
    const float* xf = static_cast<const float*>(d.x);
    __shared__ float red[kThreads / 64];
    float ss = 0.0f;
    for (int k0 = 0; k0 < C; k0 += kThreads * kStageBatch) {
        float v[kStageBatch];
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j) v[j] = xf[xi(p, d, min(k0 + j * kThreads + tid, C - 1), m)];
#pragma unroll
        for (int j = 0; j < kStageBatch; ++j)
            if (k0 + j * kThreads + tid < C) ss = fmaf(v[j], v[j], ss);
    }
    ss = wg_sum<kThreads>(ss, red);
    if (tid == 0) p.inv[blockIdx.y * 16 + m] = 1.0f / sqrtf(ss / (float)C + p.eps);
}

// ---- kernel 1 at 2 <= M <= 16 with 64-long blocks: P[b][a][m] = D[a] . X'[64b : 64b + 64, m]
// on the fp32 matrix cores, the M = 1 product widened: the N dimension of
// v_mfma_f32_16x16x4_f32 runs over (block column, column) pairs, 16 / MC block columns of MC
// columns per 16-wide tile (columns past M contribute zeros and are not stored). Workgroup =
// 4 waves x 16 atoms by one N tile. The tile's X' (X with the call's x op: RMSNorm by
// rms_inv_kernel's column statistic, or SiLU . x2) is staged once in LDS with coalesced loads,
// as [pair][feature] rows padded to 68 floats (the 16-byte reads of 8 consecutive pairs then
// meet distinct banks). Lane l supplies atom l % 16 (A, one contiguous 64-byte run of the
// dictionary row) and pair l % 16 (B, four 16-byte LDS reads); lane group l / 16 takes features
// 16 (l / 16) .. + 15 of the block in its 16 steps. Lane l ends with P[pair l % 16][atoms
// 4 (l / 16) .. + 3]. Y is initialised as in dx_kernel.
constexpr int kXsStride = 68;

template <int XOP, int MC>
__global__ __launch_bounds__(kThreads) void dxmm_kernel(Params p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    static_assert(MC == 2 || MC == 4 || MC == 8 || MC == 16, "MC");
    static_assert(kThreads == 256, "one X element per thread and pass");
    constexpr int BPT = 16 / MC;  // block columns per N tile
    __shared__ __attribute__((aligned(16))) float xs[16 * kXsStride];
    const int wg = blockIdx.x;
    int g = 0;
    while (g + 1 < p.G && wg >= p.m[g + 1].dx_base) ++g;
    const MatDesc& d = p.m[g];
    const int u = wg - d.dx_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int M = p.M;
    const int na = (d.K + 63) / 64;
    const int ag = u % na, ng = u / na;
    const int a0 = ag * 64 + wave * 16;
    // dictionary operand first (the longest round trip), then the X tile
    f4 dv[4];
    {
        const f4* src = reinterpret_cast<const f4*>(d.dict + (size_t)min(a0 + li, d.K - 1) * 64 +
                                                    lg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) dv[i] = src[i];
    }
    {
        // 16 pairs x 64 features, 4 per thread (the element type's branch around all four
        // loads: a branch per load left each to wait for the ones before it)
        float v[4], w2[4], iv[4];
        int dst[4];
        bool ok[4];
        size_t xo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // e -> (block column bl of the tile, column m, feature f) in memory order: features
            // fastest for token-major X (M x C), columns fastest for feature-major (C x M)
            const int e = i * kThreads + tid;
            const int bl = e / (64 * MC), r = e - bl * 64 * MC;
            int m, f;
            if (p.tm) {
                m = r / 64;
                f = r - m * 64;
            } else {
                f = r / MC;
                m = r - f * MC;
            }
            const int n = bl * MC + m;
            const int b = ng * BPT + bl;
            ok[i] = b < d.NB && m < M;
            const int fg = min(b, d.NB - 1) * 64 + f, mg = min(m, M - 1);
            xo[i] = xi(p, d, fg, mg);
            if constexpr (XOP == CSDR_XOP_RMSNORM) {
                iv[i] = p.inv[g * 16 + mg];
                w2[i] = p.nw[fg];
            }
            if constexpr (XOP == CSDR_XOP_SILU_MUL) w2[i] = static_cast<const float*>(d.x2)[xo[i]];
            dst[i] = n * kXsStride + f;
        }
        if (p.x_f16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = xval<_Float16>(d.x, xo[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = xval<float>(d.x, xo[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = v[i];
            if constexpr (XOP == CSDR_XOP_RMSNORM) x = x * iv[i] * w2[i];
            if constexpr (XOP == CSDR_XOP_SILU_MUL) x = (x * (1.0f / (1.0f + expf(-x)))) * w2[i];
            xs[dst[i]] = ok[i] ? x : 0.0f;
        }
    }
    {
        const size_t ytot = (size_t)d.R * M;
        const size_t yper = (ytot + d.dx_count - 1) / d.dx_count;
        const size_t ye = min(ytot, (size_t)(u + 1) * yper);
        // (kept with no bias: nothing to do, and no read of y to wait for)
        if (!p.accumulate || d.bias) {
            for (size_t i = (size_t)u * yper + tid; i < ye; i += kThreads) {
                const float bv = d.bias ? d.bias[p.tm ? i % d.R : i / M] : 0.0f;
                d.y[i] = p.accumulate ? d.y[i] + bv : bv;
            }
        }
    }
    if (u == 0 && XOP != CSDR_XOP_NONE && d.xe) {
        // the transformed edge-strip inputs, [cc][m]
        for (int t = tid; t < d.Ce * M; t += kThreads) {
            const int cc = t / M, m = t - cc * M, f = d.C_full + cc;
            const size_t xo = xi(p, d, f, m);
            float x = xload(d.x, p.x_f16, xo);
            if constexpr (XOP == CSDR_XOP_RMSNORM) x = x * p.inv[g * 16 + m] * p.nw[f];
            if constexpr (XOP == CSDR_XOP_SILU_MUL)
                x = (x * (1.0f / (1.0f + expf(-x)))) * static_cast<const float*>(d.x2)[xo];
            d.xe[t] = x;
        }
    }
    __syncthreads();
    f4 xb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        xb[i] = *reinterpret_cast<const f4*>(xs + li * kXsStride + lg * 16 + 4 * i);
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(dv[s >> 2][s & 3], xb[s >> 2][s & 3], acc, 0, 0, 0);
    const int bj = ng * BPT + li / MC, mj = li % MC;
    if constexpr (MC == 8) {
        if (p.p16) {
            // fp16 P, [block][atom][8] with the columns past M zero (their X' was staged as
            // zeros): 16 bytes per (block, atom), a pair of columns per even lane
            uint32_t* out = reinterpret_cast<uint32_t*>(d.P) + (size_t)bj * d.K * 4 + (mj >> 1);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float o = dpp_move<0xB1>(acc[v]);  // the odd column's value
                const int a = a0 + 4 * lg + v;
                const uint32_t w = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)acc[v]) |
                                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)o) << 16);
                if (bj < d.NB && !(mj & 1) && a < d.K) __builtin_nontemporal_store(w, out + (size_t)a * 4);
            }
            return;
        }
    }
    if (bj < d.NB && mj < M) {
        float* out = d.P + (size_t)bj * d.K * M + mj;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int a = a0 + 4 * lg + v;  // (streamed past this XCD's L2, as in dx1_body)
            if (a < d.K) __builtin_nontemporal_store(acc[v], out + (size_t)a * M);
        }
    }
}

// Finds this gather workgroup's matrix and (chunk, split); false for padding slots.
// Workgroups of one chunk are numbered to share an XCD (dispatch is round-robin over the
// 8 XCDs), so that chunk's P slice is fetched into one L2 only.
__device__ __forceinline__ bool gather_slot(const Params& p, int& g, int& c, int& sidx) {
    const int wg = blockIdx.x;
    g = -1;
    for (int i = 0; i < p.G; ++i)
        if (wg >= p.m[i].g_base && wg < p.m[i].g_base + p.m[i].g_count) g = i;
    if (g < 0) return false;
    const MatDesc& d = p.m[g];
    const int u = wg - d.g_base;
    const int j = u >> 3;
    const int cl = j / d.splits;
    sidx = j - cl * d.splits;
    c = cl * 8 + (u & 7);
    return c < d.nchunks;
}

__device__ __forceinline__ float edge_term(const Params& p, const MatDesc& d, int r, int m) {
    float s = 0.0f;
    const float* e = d.edge + (size_t)r * d.Ce;
    if (d.xe) {
        for (int cc = 0; cc < d.Ce; ++cc) s = fmaf(e[cc], d.xe[(size_t)cc * p.M + m], s);
        return s;
    }
    for (int cc = 0; cc < d.Ce; ++cc)
        s = fmaf(e[cc], xload(d.x, p.x_f16, xi(p, d, d.C_full + cc, m)), s);
    return s;
}

// ---- kernel 2, M == 1: the gather, 1024-thread workgroups
// Workgroup = (matrix, chunk c, row range s), about kGWgsPerCu per CU in all, each streaming about the same code bytes
// (plan_gather_splits), numbered chunk-fastest so that consecutive ids (which dispatch
// round-robin over the 8 XCDs) spread every matrix over all XCDs. The workgroup issues its
// chunk's P slice loads (nbc * K floats, written by the dx launch), then each of its 16 waves
// issues the first DEPTH 1 KiB loads of its contiguous sixteenth of the code run (bounded
// buffer loads, kept in a ring of registers); P goes to LDS and the waves stream their parts:
// per lane a fixed tile and slot quarter (each row of a chunk spans a power of two of 16-byte
// pieces, 64 % pieces == 0), row totals as DPP / shuffle butterflies over the row's lanes,
// kept in LDS, and after the stream one device-scope float atomic per (row, chunk) into Y
// (initialised by the dx launch).
constexpr int kGThreads = 1024;
constexpr int kGWaves = kGThreads / 64;
constexpr int kGDepth = 4;  // code loads in flight per wave
constexpr int kGWgsPerCu = 2;  // gather workgroups per CU (measured: 2 ahead of 1 by ~6%)
constexpr int kGMinWgBytes = 16384;  // code bytes per gather workgroup, at least (cfg4 decode: 694
                                     // tokens/s vs 681 at 1, 684 at 32 KiB)
constexpr size_t kGMaxP = 4 * 4 * kGThreads;  // P slice floats: 4 float4 per thread
// rows per gather workgroup (their totals wait in LDS): with a 64 KiB P slice two workgroups
// still fit in a CU's 160 KiB
constexpr int kGMaxRows = 3840;

// Slot gamma i of a matrix as a wave-uniform scalar: the readfirstlane keeps the per-lane
// select over these values a select (otherwise the compiler turns it into a per-lane memory
// load, whose wait then lands inside the streaming loops)
__device__ __forceinline__ float sgam_at(const MatDesc& d, int i) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, d.sgam[i])));
}

// kGWgsPerCu 1024-thread workgroups per CU = 8 waves per SIMD: at most 64 VGPRs
// P4: K % 4 == 0, the P slice is staged as float4
template <int SLOTS, int DEPTH, bool P4>
__device__ __forceinline__ void gatherw_body(const Params& p, int wg) {
    extern __shared__ float smem[];
    int g = 0;
    while (g + 1 < p.G && wg >= p.m[g + 1].g_base) ++g;
    const MatDesc& d = p.m[g];
    // workgroup -> (chunk, row range): the full chunks' ranges first, chunk-fastest (so that
    // consecutive ids, which dispatch round-robin over the XCDs, spread each chunk), then each
    // remainder chunk's ranges
    const int u = wg - d.g_base;
    const int nfull = d.NB / d.NBc;
    int c, sidx, rpw;
    if (u < nfull * d.splits) {
        c = u % nfull;
        sidx = u / nfull;
        rpw = d.rows_per_wg;
    } else {
        int v = u - nfull * d.splits, j = 0;
        while (j < 4 && v >= d.rsplit[j]) v -= d.rsplit[j++];
        if (j == 4) return;
        c = nfull + j;
        sidx = v;
        rpw = d.rrpw[j];
    }
    uint32_t b0u, nbcu;
    csdr::chunk_span((uint32_t)c, (uint32_t)d.NB, (uint32_t)d.NBc, b0u, nbcu);
    const int b0 = (int)b0u, nbc = (int)nbcu;
    const int rbeg = sidx * rpw;
    const int rend = min(d.R, rbeg + rpw);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // The workgroup's P slice loads (nbc * K <= kGMaxP floats, written by the dx launch) are
    // issued first, then every wave's first DEPTH code loads, and only then are the P values
    // stored to LDS: VMEM loads complete in issue order, so P issued behind the code loads of
    // all waves (most of the launch's bytes at once) would wait for them.
    constexpr int PPB = SLOTS / 4;  // 16-byte pieces per tile
    const int ppr = nbc * PPB;      // pieces per row: a power of two <= 64
    const int npieces = (rend - rbeg) * ppr;
    const int nload = (npieces + 63) >> 6;
    // wave w streams its own contiguous part of the run (wave loads [w per, (w + 1) per));
    // the trip count is wave-uniform
    const int per = (nload + kGWaves - 1) / kGWaves;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int nk = max(0, min(per, nload - wv * per));
    // The wave's part is read through a raw buffer resource bounded to its valid bytes: every
    // load is issued unconditionally (the compiler then waits for exactly the load it needs,
    // where a conditional load would make it wait for all loads in flight), and a load at or
    // past the end returns zeros without touching memory.
    const int wfirst = wv * per * 64;  // the wave's first piece in the run
    const int wvalid = max(0, min(per * 64, npieces - wfirst));
    const uint32_t* wbase = d.codes + (size_t)b0 * d.R * SLOTS + (size_t)rbeg * nbc * SLOTS +
                            (size_t)wfirst * 4;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)wbase, (short)0, wvalid * 16, kRawBufferDword3);
    constexpr int kStep = 64;  // pieces between a wave's consecutive loads
    auto piece = [&](int k) -> u32x4 {
        return __builtin_amdgcn_raw_buffer_load_b128(rs, (k * kStep + lane) * 16, 0, kCachePolicyNT);
    };

    float* Ps = smem;               // nbc * K floats
    float* xe = Ps + d.NBc * d.K;   // Ce (< 64) floats
    float* rowt = xe + 64;          // rend - rbeg <= kGMaxRows row totals
    const bool edge = (c == d.nchunks - 1) && d.Ce > 0;
    const float* Pg = d.P + (size_t)b0 * d.K;
    const int np = nbc * d.K;
    const int np4 = np >> 2;
    const float4* s4 = reinterpret_cast<const float4*>(Pg);
    float4* d4 = reinterpret_cast<float4*>(Ps);
    // clamped loads and stores, no branches (lanes past the end rewrite the last element with
    // its own value): a conditional store lets the compiler sink its load into the branch and
    // wait for every load in flight before it
    // (four named values, not an array: an array held across the scheduling barrier below is
    // kept in scratch memory)
    float4 pv0{}, pv1{}, pv2{}, pv3{};
    if constexpr (P4) {
        // nontemporal: the slice was just streamed out by the dx launch (headline step 15.35 ->
        // 14.72 us; a gather that re-reads a slice still in its L2 is slower this way)
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v* sv = reinterpret_cast<const f4v*>(Pg);
        auto ld = [&](int i) {
            const f4v v = __builtin_nontemporal_load(sv + i);
            return make_float4(v.x, v.y, v.z, v.w);
        };
        pv0 = ld(min(tid, np4 - 1));
        pv1 = ld(min(kGThreads + tid, np4 - 1));
        pv2 = ld(min(2 * kGThreads + tid, np4 - 1));
        pv3 = ld(min(3 * kGThreads + tid, np4 - 1));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the P loads ahead of the code loads
    // a ring of DEPTH + 1 register buffers: piece k sits in buf[k % (DEPTH + 1)], and the load of
    // piece k + DEPTH goes into the buffer that piece k - 1 has left, so no live value is ever
    // overwritten and the compiler needs no register copies (which would wait for the loads)
    constexpr int NBUF = DEPTH + 1;
    u32x4 buf[NBUF];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) buf[k] = piece(k);
    if constexpr (P4) {
        d4[min(tid, np4 - 1)] = pv0;
        d4[min(kGThreads + tid, np4 - 1)] = pv1;
        d4[min(2 * kGThreads + tid, np4 - 1)] = pv2;
        d4[min(3 * kGThreads + tid, np4 - 1)] = pv3;
    } else {
        stage_to_lds<float, kGThreads>(Pg, np, Ps);
    }
    __syncthreads();

    // per lane a fixed tile and slot quarter; word = (signed fp16 coefficient << 16) | index,
    // the low half is the index itself (bit 15 is 0)
    const int pl = lane & (ppr - 1);
    const int lg_ppr = __builtin_ctz((unsigned)ppr);
    const int bb = pl / PPB, h = pl - bb * PPB;
    const float* Pb = Ps + bb * d.K;
    float gm[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        gm[e] = sgam_at(d, e);
#pragma unroll
        for (int hh = 1; hh < PPB; ++hh)
            if (h == hh) gm[e] = sgam_at(d, hh * 4 + e);
    }
    const bool gu = d.gunif != 0;
    const float g0 = d.sgam[0];
    const bool head = (pl == 0);
    const int q0 = wfirst + lane;  // this lane's piece in the wave's first load
    // one piece: lane partial, row total over the row's lanes, the head lane keeps it
    auto consume = [&](const u32x4& w, int k) {
        const int qp = q0 + k * kStep;
        const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
        float acc = 0.0f;
        if (gu) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = fmaf(csdr::h2f(w4[e] >> 16), Pb[(uint16_t)w4[e]], acc);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = fmaf(gm[e] * csdr::h2f(w4[e] >> 16), Pb[(uint16_t)w4[e]], acc);
        }
        if (qp >= npieces) acc = 0.0f;
        if (ppr > 1) acc += dpp_move<0xB1>(acc);   // quad_perm [1,0,3,2]
        if (ppr > 2) acc += dpp_move<0x4E>(acc);   // quad_perm [2,3,0,1]
        if (ppr > 4) acc += dpp_move<0x141>(acc);  // row_half_mirror
        if (ppr > 8) acc += dpp_move<0x140>(acc);  // row_mirror
        if (ppr > 16) acc += __shfl_xor(acc, 16, 64);
        if (ppr > 32) acc += __shfl_xor(acc, 32, 64);
        if (head && qp < npieces) rowt[qp >> lg_ppr] = gu ? acc * g0 : acc;
    };
    // Whole groups of NBUF pieces with no exit inside (an exit that rejoins the loop would
    // leave the compiler unsure how many loads are in flight at the top, and it would wait for
    // nearly all), then the last nk % NBUF pieces, whose loads were all issued already.
    int k0 = 0;
    for (; k0 + NBUF <= nk; k0 += NBUF) {
#pragma unroll
        for (int jj = 0; jj < NBUF; ++jj) {
            const u32x4 w = buf[jj];
            buf[(jj + DEPTH) % NBUF] = piece(k0 + jj + DEPTH);
            consume(w, k0 + jj);
        }
    }
#pragma unroll
    for (int jj = 0; jj < NBUF - 1; ++jj)
        if (k0 + jj < nk) consume(buf[jj], k0 + jj);
    // Row totals into Y after the stream, one device-scope atomic per row, 64 rows per
    // instruction (atomics inside the stream would count among its loads in flight and make
    // the compiler wait for all of them), with the top-right strip on the last chunk.
    if (edge && tid < d.Ce) xe[tid] = d.xe ? d.xe[tid] : xload(d.x, p.x_f16, (size_t)d.C_full + tid);
    __syncthreads();
    for (int rr = tid; rr < rend - rbeg; rr += kGThreads) {
        float v = rowt[rr];
        if (edge) {
            const float* er = d.edge + (size_t)(rbeg + rr) * d.Ce;
            for (int cc = 0; cc < d.Ce; ++cc) v = fmaf(er[cc], xe[cc], v);
        }
        __hip_atomic_fetch_add(d.y + rbeg + rr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int SLOTS, int DEPTH, bool P4>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(kGWgsPerCu * 4)))
void gatherw_kernel(Params p) {
    gatherw_body<SLOTS, DEPTH, P4>(p, (int)blockIdx.x);
}

// ---- kernel 2, 2 <= M <= 8: the same streaming gather with MC columns per code read
// Workgroup = (matrix, chunk, row range) as in gatherw_kernel; the chunk's P slice is staged
// in LDS as [block][atom][MC] fp32 (columns past M zero), so each slot's MC values are one or
// two LDS reads and every code word feeds MC fused multiply-adds: the codes are read from HBM
// once for all M columns. A lane takes one tile (one row's slots of one block column), so a
// row's partial sums meet across the chunk's block columns only (one DPP step per doubling),
// and every slot's stage gain is the same for all lanes. Row totals (MC per row) wait
// in LDS and go into Y with one device-scope atomic per (row, column) after the stream. WPE:
// waves per SIMD the register budget is pinned for (1 workgroup per CU for the 128 KiB slice
// at MC = 8, 2 below).
constexpr int kGvMinRows = 256;  // rows per workgroup the LDS share must hold, at least

// The 2 <= M <= 8 gather's stream for one chunk width: LPR lanes per row (lane = block column
// of the row), `buf` holding the first TD tiles already issued. Lanes past the wave's valid
// tiles read zeros (coefficient 0), and a row's lanes are all valid or all past the end, so no
// selects are needed before the row reductions.
template <int SLOTS, int MC, int TD, int LPR, bool P16, typename TileFn>
__device__ __forceinline__ void gatherv_stream(const MatDesc& d, const float* Ps, float* rowt,
                                               u32x4 (*buf)[SLOTS / 4], TileFn tile, int nk,
                                               int wfirst, int ntiles) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    constexpr int PPB = SLOTS / 4;
    constexpr int G = MC / 4;
    constexpr int kStep = 64;
    constexpr int lg_lpr = LPR == 1 ? 0 : LPR == 2 ? 1 : LPR == 4 ? 2 : LPR == 8 ? 3
                         : LPR == 16 ? 4 : LPR == 32 ? 5 : 6;
    const int lane = threadIdx.x & 63;
    const int bb = lane & (LPR - 1);
    const int ebase = bb * d.K;
    float gm[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) gm[j] = sgam_at(d, j);
    const bool head = (bb == 0);
    const int q0 = wfirst + lane;
    auto consume = [&](const u32x4* w, int k) {
        const int tq = q0 + k * kStep;
        float acc[MC];
#pragma unroll
        for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
            const uint32_t word = w[j >> 2][j & 3];
            const float cf = gm[j] * csdr::h2f(word >> 16);
            const int e = ebase + (int)(uint16_t)word;
            if constexpr (P16) {
                // 8 fp16 columns in one 16-byte read (multiply-adds with an fp16 operand)
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const u32x4 v = *reinterpret_cast<const u32x4*>(Ps + (size_t)e * 4);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // (the element through a scalar: a bit cast of the vector element
                    // expression v[k] itself compiles to a read of element 0 only)
                    const uint32_t dw = v[k];
                    const h2 pr = __builtin_bit_cast(h2, dw);
                    acc[2 * k] = fmaf(cf, (float)pr[0], acc[2 * k]);
                    acc[2 * k + 1] = fmaf(cf, (float)pr[1], acc[2 * k + 1]);
                }
            } else if constexpr (MC == 2) {
                const f2 v = *reinterpret_cast<const f2*>(Ps + (size_t)e * 2);
                acc[0] = fmaf(cf, v.x, acc[0]);
                acc[1] = fmaf(cf, v.y, acc[1]);
            } else {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const f4 v = *reinterpret_cast<const f4*>(Ps + (size_t)e * MC + 4 * h);
                    acc[4 * h] = fmaf(cf, v.x, acc[4 * h]);
                    acc[4 * h + 1] = fmaf(cf, v.y, acc[4 * h + 1]);
                    acc[4 * h + 2] = fmaf(cf, v.z, acc[4 * h + 2]);
                    acc[4 * h + 3] = fmaf(cf, v.w, acc[4 * h + 3]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MC; ++m) {
            float a = acc[m];
            if constexpr (LPR > 1) a += dpp_move<0xB1>(a);
            if constexpr (LPR > 2) a += dpp_move<0x4E>(a);
            if constexpr (LPR > 4) a += dpp_move<0x141>(a);
            if constexpr (LPR > 8) a += dpp_move<0x140>(a);
            if constexpr (LPR > 16) a += __shfl_xor(a, 16, 64);
            if constexpr (LPR > 32) a += __shfl_xor(a, 32, 64);
            acc[m] = a;
        }
        if (head && tq < ntiles) {
            float* rt = rowt + (size_t)(tq >> lg_lpr) * MC;
            if constexpr (MC >= 4) {
#pragma unroll
                for (int m4 = 0; m4 < MC; m4 += 4)
                    *reinterpret_cast<f4*>(rt + m4) = f4{acc[m4], acc[m4 + 1], acc[m4 + 2], acc[m4 + 3]};
            } else {
#pragma unroll
                for (int m = 0; m < MC; ++m) rt[m] = acc[m];
            }
        }
    };
    constexpr int NBUF = TD + 1;
    int k0 = 0;
    for (; k0 + NBUF <= nk; k0 += NBUF) {
#pragma unroll
        for (int jj = 0; jj < NBUF; ++jj) {
            u32x4 w[PPB];
#pragma unroll
            for (int i = 0; i < PPB; ++i) w[i] = buf[jj][i];
            tile(k0 + jj + TD, buf[(jj + TD) % NBUF]);
            consume(w, k0 + jj);
        }
    }
#pragma unroll
    for (int jj = 0; jj < NBUF - 1; ++jj)
        if (k0 + jj < nk) consume(buf[jj], k0 + jj);
}

template <int SLOTS, int MC, int DEPTH, int WPE, bool P16>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(WPE)))
void gatherv_kernel(Params p) {
    static_assert(!P16 || MC == 8, "fp16 P has 8 columns");
    extern __shared__ float smem[];
    // Workgroups go to the eight XCDs round-robin (workgroup b on XCD b % 8). XCD x takes the
    // x-th eighth of the units in chunk-major order, so the row ranges of one chunk share the
    // L2 that holds its P slice (MC columns make the slice a quarter of the chunk's codes and
    // more: fetched into several L2s it would double the HBM bytes). The launch is padded to
    // a multiple of 8; padding workgroups exit.
    const int per_xcd = (p.gtotal + 7) >> 3;
    const int wg = ((int)blockIdx.x & 7) * per_xcd + ((int)blockIdx.x >> 3);
    if (wg >= p.gtotal) return;
    int g = 0;
    while (g + 1 < p.G && wg >= p.m[g + 1].g_base) ++g;
    const MatDesc& d = p.m[g];
    const int u = wg - d.g_base;
    const int nfull = d.NB / d.NBc;
    int c, sidx, rpw;
    if (u < nfull * d.splits) {
        c = u / d.splits;
        sidx = u - c * d.splits;
        rpw = d.rows_per_wg;
    } else {
        int v = u - nfull * d.splits, j = 0;
        while (j < 4 && v >= d.rsplit[j]) v -= d.rsplit[j++];
        if (j == 4) return;
        c = nfull + j;
        sidx = v;
        rpw = d.rrpw[j];
    }
    uint32_t b0u, nbcu;
    csdr::chunk_span((uint32_t)c, (uint32_t)d.NB, (uint32_t)d.NBc, b0u, nbcu);
    const int b0 = (int)b0u, nbc = (int)nbcu;
    const int rbeg = sidx * rpw;
    const int rend = min(d.R, rbeg + rpw);
    const int M = p.M;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    constexpr int PPB = SLOTS / 4;  // 16-byte pieces per tile
    // tiles in flight per wave: about DEPTH pieces, at least two tiles
    constexpr int TD = DEPTH / PPB > 2 ? DEPTH / PPB : 2;
    const int ntiles = (rend - rbeg) * nbc;  // tile t = (row t / nbc, block column t % nbc)
    const int nload = (ntiles + 63) >> 6;
    const int per = (nload + kGWaves - 1) / kGWaves;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int nk = max(0, min(per, nload - wv * per));
    const int wfirst = wv * per * 64;
    const int wvalid = max(0, min(per * 64, ntiles - wfirst));
    const uint32_t* wbase = d.codes + (size_t)b0 * d.R * SLOTS + (size_t)rbeg * nbc * SLOTS +
                            (size_t)wfirst * SLOTS;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)wbase, (short)0, wvalid * SLOTS * 4, kRawBufferDword3);
    auto tile = [&](int k, u32x4* out) {
        const int o = (k * 64 + lane) * SLOTS * 4;
#pragma unroll
        for (int i = 0; i < PPB; ++i)
            out[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + i * 16, 0, kCachePolicyNT);
    };

    float* Ps = smem;  // NBc * K * MC floats (fp16 P: NBc * K * 8 halves)
    float* xe = Ps + (size_t)d.NBc * d.K * (P16 ? 4 : MC);  // Ce (< 64) x MC floats
    float* rowt = xe + 64 * MC;                 // (rend - rbeg) x MC row totals
    const bool edge = (c == d.nchunks - 1) && d.Ce > 0;

    // The P slice loads go out first (L2 / Infinity Cache hits: queued behind the code loads'
    // HBM misses they would wait for them), then the wave's first code loads, which overlap
    // the P round trip and the barrier.
    constexpr int NBUF = TD + 1;
    u32x4 buf[NBUF][PPB];
    typedef float f4 __attribute__((ext_vector_type(4)));
    if (P16 || (M == MC && (d.K * MC) % 4 == 0)) {
        // P slice: global [block][atom][M] (fp16 P: [block][atom][8] halves) -> LDS, a
        // straight copy of 16-byte pieces (at most 8 per thread: one round trip)
        const f4* Pg = P16 ? reinterpret_cast<const f4*>(d.P) + (size_t)b0 * d.K
                           : reinterpret_cast<const f4*>(d.P + (size_t)b0 * d.K * M);
        f4* Pl = reinterpret_cast<f4*>(Ps);
        const int n4 = nbc * d.K * (P16 ? 4 : MC) / 4;
        for (int i0 = 0; i0 < n4; i0 += kGThreads * 8) {
            f4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {  // nontemporal, as the M == 1 gather's P slice
                typedef float f4v __attribute__((ext_vector_type(4)));
                v[j] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(Pg) +
                                                  min(i0 + j * kGThreads + tid, n4 - 1));
            }
            if (i0 == 0) {
#pragma unroll
                for (int k = 0; k < TD; ++k) tile(k, buf[k]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) Pl[min(i0 + j * kGThreads + tid, n4 - 1)] = v[j];
        }
    } else {
#pragma unroll
        for (int k = 0; k < TD; ++k) tile(k, buf[k]);
        // P slice: global [block][atom][M] -> LDS [block][atom][MC], kStageBatch loads in flight
        const float* Pg = d.P + (size_t)b0 * d.K * M;
        const int n = nbc * d.K * MC;
        for (int i0 = 0; i0 < n; i0 += kGThreads * kStageBatch) {
            float v[kStageBatch];
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) {
                const int i = min(i0 + j * kGThreads + tid, n - 1);
                const int e = i / MC, m = i - e * MC;
                v[j] = Pg[(size_t)e * M + min(m, M - 1)];
                if (m >= M) v[j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) Ps[min(i0 + j * kGThreads + tid, n - 1)] = v[j];
        }
    }
    __syncthreads();

    // the stream, specialised on the lanes per row (the chunk's block columns, a power of two),
    // so each column's row reduction is a straight DPP / shuffle sequence
    switch (nbc) {
        case 1: gatherv_stream<SLOTS, MC, TD, 1, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        case 2: gatherv_stream<SLOTS, MC, TD, 2, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        case 4: gatherv_stream<SLOTS, MC, TD, 4, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        case 8: gatherv_stream<SLOTS, MC, TD, 8, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        case 16: gatherv_stream<SLOTS, MC, TD, 16, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        case 32: gatherv_stream<SLOTS, MC, TD, 32, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
        default: gatherv_stream<SLOTS, MC, TD, 64, P16>(d, Ps, rowt, buf, tile, nk, wfirst, ntiles); break;
    }
    // the top-right strip's inputs of the last chunk: [cc][m] (x-op transformed when given)
    if (edge) {
        for (int t = tid; t < d.Ce * MC; t += kGThreads) {
            const int cc = t / MC, m = t - cc * MC;
            float v = 0.0f;
            if (m < M)
                v = d.xe ? d.xe[(size_t)cc * M + m] : xload(d.x, p.x_f16, xi(p, d, d.C_full + cc, m));
            xe[t] = v;
        }
    }
    __syncthreads();
    const int nr = rend - rbeg;
    for (int t = tid; t < nr * M; t += kGThreads) {
        // consecutive threads on consecutive Y addresses in either layout
        const int rr = p.tm ? t % nr : t / M, m = p.tm ? t / nr : t - (t / M) * M;
        float v = rowt[(size_t)rr * MC + m];
        if (edge) {
            const float* er = d.edge + (size_t)(rbeg + rr) * d.Ce;
            for (int cc = 0; cc < d.Ce; ++cc) v = fmaf(er[cc], xe[cc * MC + m], v);
        }
        __hip_atomic_fetch_add(d.y + yi(p, d, rbeg + rr, m), v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- kernel 2, any M / any slot count: workgroup = (chunk, row tile of Rt rows); the
// chunk's P slice is staged MV columns at a time, code words are read per pair.
template <int MV>
__global__ __launch_bounds__(kThreads) void gatherm_kernel(Params p) {
    extern __shared__ float smem[];
    int g, c, sidx;
    if (!gather_slot(p, g, c, sidx)) return;
    const MatDesc& d = p.m[g];
    const int tid = threadIdx.x;
    const int M = p.M;
    uint32_t b0u, nbcu;
    csdr::chunk_span((uint32_t)c, (uint32_t)d.NB, (uint32_t)d.NBc, b0u, nbcu);
    const int b0 = (int)b0u, nbc = (int)nbcu;
    const int r0 = sidx * d.Rt;
    const int nr = min(d.Rt, d.R - r0);
    if (nr <= 0) return;
    const int npairs = nr * nbc;
    const uint32_t* cb =
        d.codes + (size_t)b0 * d.R * d.slots + (size_t)r0 * nbc * d.slots;
    float* Ps = smem;                              // nbc * K * MV
    float* part = smem + (size_t)d.NBc * d.K * MV; // Rt * NBc * MV
    const bool last_chunk = (c == d.nchunks - 1);
    for (int z = 0; z < p.MVz; ++z) {
        const int m0 = z * MV;
        if (z > 0) __syncthreads();
        const float* Pg = d.P + (size_t)b0 * d.K * M;
        // (kStageBatch loads in flight per thread, at clamped indices: a load under the
        // column test waited for the one before it)
        const int np = nbc * d.K * MV;
        for (int i0 = 0; i0 < np; i0 += kThreads * kStageBatch) {
            float v[kStageBatch];
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) {
                const int i = min(i0 + j * kThreads + tid, np - 1);
                const int e = i / MV, mm = i - e * MV;
                v[j] = Pg[(size_t)e * M + min(m0 + mm, M - 1)];
            }
#pragma unroll
            for (int j = 0; j < kStageBatch; ++j) {
                const int i = i0 + j * kThreads + tid;
                if (i < np) Ps[i] = (m0 + (i % MV) < M) ? v[j] : 0.0f;
            }
        }
        __syncthreads();
        for (int pi = tid; pi < npairs; pi += kThreads) {
            const int bb = pi % nbc;
            const float* Pb = Ps + (size_t)bb * d.K * MV;
            const uint32_t* src = cb + (size_t)pi * d.slots;
            float acc[MV];
#pragma unroll
            for (int mm = 0; mm < MV; ++mm) acc[mm] = 0.0f;
            // the pair's code words and gains 8 at a time, all loaded before the first is used
            // and all used (slots past the last repeat it with a zero coefficient): a load per
            // slot under the loop's exit ran a round trip per slot
            for (int s0 = 0; s0 < d.slots; s0 += 8) {
                uint32_t wv[8];
                float gv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int sj = min(s0 + j, d.slots - 1);
                    wv[j] = src[sj];
                    gv[j] = d.slot_gamma[sj];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t w = wv[j];
                    const float cf = s0 + j < d.slots ? gv[j] * csdr::h2f(w >> 16) : 0.0f;
                    const float* pv = Pb + (size_t)(w & 0x7FFFu) * MV;
#pragma unroll
                    for (int mm = 0; mm < MV; ++mm) acc[mm] = fmaf(cf, pv[mm], acc[mm]);
                }
            }
#pragma unroll
            for (int mm = 0; mm < MV; ++mm) part[pi * MV + mm] = acc[mm];
        }
        __syncthreads();
        for (int t = tid; t < nr * MV; t += kThreads) {
            const int rr = t / MV, mm = t - rr * MV;
            const int m = m0 + mm;
            if (m >= M) continue;
            float sum = 0.0f;
            for (int bb = 0; bb < nbc; ++bb) sum += part[(rr * nbc + bb) * MV + mm];
            const int r = r0 + rr;
            if (last_chunk && d.Ce > 0) sum += edge_term(p, d, r, m);
            __hip_atomic_fetch_add(d.y + yi(p, d, r, m), sum, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ decode / export

__device__ __forceinline__ size_t code_offset(const csdr_hsdb& s, uint32_t t) {
    if (s.tile_rows != 1) return (size_t)t * s.slots;
    const uint32_t r = t / s.NB, b = t - r * s.NB;
    return csdr::tile_word_offset(r, b, s.R, s.NB, s.NBc, s.slots);
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

// Rows of W (1-row tiles) into out[blockIdx.y][C]: each row's tiles decoded as
// decode_dense_kernel does, then its edge columns. Row blockIdx.y's index is read from device
// memory (a token id) when row_dev is given; an index outside [0, R) leaves its row untouched.
__global__ __launch_bounds__(kThreads) void decode_row_kernel(csdr_hsdb s,
                                                              const int* __restrict__ row_dev,
                                                              int row_host, float* __restrict__ out) {
    const int r = row_dev ? row_dev[blockIdx.y] : row_host;
    if (r < 0 || r >= (int)s.R) return;
    out += (size_t)blockIdx.y * s.C;
    const uint32_t B = s.tile_cols;
    for (uint32_t g = blockIdx.x * kThreads + threadIdx.x; g < s.C; g += gridDim.x * kThreads) {
        if (g >= s.C_full) {
            out[g] = s.d_edge[(size_t)r * s.Ce + (g - s.C_full)];
            continue;
        }
        const uint32_t b = g / B, e = g - b * B;
        const uint32_t* w = s.d_codes + code_offset(s, (uint32_t)r * s.NB + b);
        float acc = 0.0f;
        for (uint32_t j = 0; j < s.slots; ++j) {
            const uint32_t wd = w[j];
            const float cf = s.d_slot_gamma[j] * csdr::h2f(wd >> 16);
            acc = fmaf(cf, s.d_dict[(size_t)(wd & 0x7FFFu) * B + e], acc);
        }
        out[g] = acc;
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

// ---- device dictionaries shared between segments
// Segments on one device whose dictionaries have the same bytes and tile shape share one
// device copy (fp32, and the fp16 matrix-core copy for 64-wide 1-row tiles), as the
// reference's shared-dictionary archive (HSDA) shares one dictionary among many code streams
// (HierarchicalSDRStrategy.cpp:1904-2081). Reference counted; CSDR_HSDB_SHARE_DICT=0 gives
// every segment its own copy.
struct DictEntry {
    int device = 0;
    uint32_t tile_rows = 0, tile_cols = 0, K = 0;
    std::vector<uint8_t> bytes;
    float* d32 = nullptr;
    _Float16* d16p = nullptr;
    size_t dev_bytes = 0;
    int refs = 0;
};
std::mutex g_dict_mu;
std::vector<DictEntry*> g_dicts;

int acquire_dict(csdr_hsdb* s, const uint8_t* dict, size_t b_dict, hipStream_t st) {
    const bool share = env_flag("CSDR_HSDB_SHARE_DICT", true);
    const bool want16 = s->tile_rows == 1 && s->tile_cols == 64;
    std::lock_guard<std::mutex> lock(g_dict_mu);
    if (share) {
        for (DictEntry* e : g_dicts) {
            if (e->device == s->device && e->tile_rows == s->tile_rows &&
                e->tile_cols == s->tile_cols && e->K == s->K && e->bytes.size() == b_dict &&
                std::memcmp(e->bytes.data(), dict, b_dict) == 0) {
                ++e->refs;
                s->dict_ref = e;
                s->d_dict = e->d32;
                s->d_dict16p = e->d16p;
                s->device_bytes += e->dev_bytes;
                return CSDR_OK;
            }
        }
    }
    auto* e = new DictEntry;
    e->device = s->device;
    e->tile_rows = s->tile_rows;
    e->tile_cols = s->tile_cols;
    e->K = s->K;
    e->bytes.assign(dict, dict + b_dict);
    e->refs = 1;
    auto fail = [&](hipError_t err) {
        if (e->d32) (void)hipFree(e->d32);
        if (e->d16p) (void)hipFree(e->d16p);
        delete e;
        return set_error(CSDR_E_HIP, std::string("hsdb_load: ") + hipGetErrorString(err));
    };
    hipError_t err = hipMalloc(&e->d32, std::max<size_t>(b_dict, 4));
    if (err != hipSuccess) return fail(err);
    err = hipMemcpyAsync(e->d32, dict, b_dict, hipMemcpyHostToDevice, st);
    if (err != hipSuccess) return fail(err);
    e->dev_bytes = b_dict;
    if (want16) {
        // the fp16 copy (round to nearest even), each 64-row in the matrix-core k order
        // (csdr::kperm64), for the batched product
        const size_t n = (size_t)s->K * 64;
        std::vector<_Float16> dict16(n);
        std::vector<float> d32(n);
        std::memcpy(d32.data(), dict, n * 4);
        for (size_t i = 0; i < n; ++i)
            dict16[(i & ~(size_t)63) + csdr::kperm64((int)(i & 63))] = (_Float16)d32[i];
        err = hipMalloc(&e->d16p, n * 2);
        if (err != hipSuccess) return fail(err);
        err = hipMemcpyAsync(e->d16p, dict16.data(), n * 2, hipMemcpyHostToDevice, st);
        if (err == hipSuccess) err = hipStreamSynchronize(st);  // dict16 dies with this call
        if (err != hipSuccess) return fail(err);
        e->dev_bytes += n * 2;
    }
    s->dict_ref = e;
    s->d_dict = e->d32;
    s->d_dict16p = e->d16p;
    s->device_bytes += e->dev_bytes;
    if (share) g_dicts.push_back(e);
    return CSDR_OK;
}

void release_dict(csdr_hsdb* s) {
    auto* e = static_cast<DictEntry*>(s->dict_ref);
    if (!e) return;
    std::lock_guard<std::mutex> lock(g_dict_mu);
    if (--e->refs == 0) {
        (void)hipFree(e->d32);
        if (e->d16p) (void)hipFree(e->d16p);
        g_dicts.erase(std::remove(g_dicts.begin(), g_dicts.end(), e), g_dicts.end());
        delete e;
    }
    s->dict_ref = nullptr;
    s->d_dict = nullptr;
    s->d_dict16p = nullptr;
}

const char* const kHostCodesMsg =
    "hsdb: the segment's codes are host-resident (csdr_hsdb_load_host); a decoder streams "
    "them per layer, or load the segment with csdr_hsdb_load";

// Stream parse with the reference's checks (HierarchicalSDRStrategy.cpp:1265-1290 and
// readBuffer's truncation check) plus index < n_atoms.
int parse_and_upload(const uint8_t* buf, size_t n, hipStream_t st, csdr_hsdb* s,
                     bool host_codes = false) {
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

    // chunking of block columns (1-row tiles): the P slice of a chunk (nbc * K fp32, staged
    // in LDS by the M == 1 products) at most kChunkPBytes
    if (s->tile_rows == 1) {
        const size_t cap = kChunkPBytes;
        uint32_t nbc = kMaxChunkBlocks;
        while (nbc > 1 && (size_t)nbc * s->K * 4 > cap) nbc >>= 1;
        while (nbc > 1 && nbc > s->NB) nbc >>= 1;
        s->NBc = nbc;
        s->nchunks = s->NB ? csdr::n_chunks(s->NB, nbc) : 0;
    }

    // build the device words
    std::vector<uint32_t> words(n_codes);
    size_t tile_dst = 0;
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
            if (j == 0) {
                const uint32_t r = (uint32_t)(t / s->NB), b = (uint32_t)(t - (size_t)r * s->NB);
                tile_dst = csdr::tile_word_offset(r, b, s->R, s->NB, s->NBc, s->slots);
            }
            dst = tile_dst + j;
        }
        words[dst] = (h << 16) | idx;
    }
    std::vector<float> slot_gamma(std::max<uint32_t>(s->slots, 1), 0.0f);
    for (uint32_t j = 0; j < s->slots; ++j)
        std::memcpy(&slot_gamma[j], buf + off_gamma + 4u * (j / s->k), 4);
    for (uint32_t j = 0; j < s->slots && j < 32; ++j) s->h_slot_gamma[j] = slot_gamma[j];

    const size_t b_dict = (size_t)s->K * tile_dim * 4;
    const size_t b_codes = n_codes * 4;
    const size_t b_gamma = slot_gamma.size() * 4;
    const size_t b_edge = edge_bytes;
    {
        const int rc = acquire_dict(s, buf + off_dict, b_dict, st);
        if (rc) return rc;
    }
    if (host_codes) {
        // pinned, so a decoder's staging copies run as DMA (and can be graph nodes)
        CSDR_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&s->h_codes),
                                     std::max<size_t>(b_codes, 4), hipHostMallocDefault));
        if (b_codes) std::memcpy(s->h_codes, words.data(), b_codes);
    } else {
        CSDR_HIP_CHECK(hipMalloc(&s->d_codes, std::max<size_t>(b_codes, 4)));
        s->device_bytes += b_codes;
    }
    CSDR_HIP_CHECK(hipMalloc(&s->d_slot_gamma, b_gamma));
    CSDR_HIP_CHECK(hipMalloc(&s->d_edge, std::max<size_t>(b_edge, 4)));
    s->device_bytes += b_gamma + b_edge;
    if (b_codes && s->d_codes)
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
    release_dict(s);
    if (s->d_codes) (void)hipFree(s->d_codes);
    if (s->h_codes) (void)hipHostFree(s->h_codes);
    if (s->d_slot_gamma) (void)hipFree(s->d_slot_gamma);
    if (s->d_edge) (void)hipFree(s->d_edge);
    delete s;
}



// Block columns per dx workgroup (block length 64): about `work` (block, column) dot
// products per 16-lane group.
inline int producer_blocks(int M) {
    constexpr int kWork = 16;
    return M >= kWork ? 1 : kWork / M;
}

size_t p_bytes(const csdr_hsdb* s, int M) {
    return csdr::align_up((size_t)s->NB * s->K * M * 4, 256) +
           csdr::align_up((size_t)s->Ce * M * 4, 256);  // x-op edge inputs
}

// Workspace of the P path (dx + gather launches).
size_t p_path_ws_bytes(int n, const csdr_hsdb* const* segs, int M) {
    size_t t = csdr::kWsHead;
    for (int i = 0; i < n; ++i) t += p_bytes(segs[i], M);
    return t;
}

// Workspace of a full product at batch M, large enough for every batch <= M as well (the
// matrix-core path can need less than the P path at a smaller M).
// Enough for every path and phase a call at this M can take: the matrix-core path of a plain
// product, and the P path of x-op calls (M <= 16) and of the separate dx / gather phases.
size_t group_ws_bytes(int n, const csdr_hsdb* const* segs, int M) {
    if (csdr::mfma_eligible(n, segs, M))
        return std::max(csdr::mfma_workspace_bytes(n, segs, M), p_path_ws_bytes(n, segs, M));
    return p_path_ws_bytes(n, segs, M);
}

template <bool P4>
void launch_gatherw_p(const Params& p, int slots, int grid, size_t lds, hipStream_t st) {
    switch (slots) {
        case 4:
            gatherw_kernel<4, kGDepth, P4><<<grid, kGThreads, lds, st>>>(p);
            break;
        case 8:
            gatherw_kernel<8, kGDepth, P4><<<grid, kGThreads, lds, st>>>(p);
            break;
        default:
            gatherw_kernel<16, kGDepth, P4><<<grid, kGThreads, lds, st>>>(p);
            break;
    }
}

void launch_gatherw(const Params& p, int slots, int grid, size_t lds, hipStream_t st) {
    bool p4 = true;
    for (int i = 0; i < p.G; ++i) p4 = p4 && (p.m[i].K & 3) == 0;
    if (p4)
        launch_gatherw_p<true>(p, slots, grid, lds, st);
    else
        launch_gatherw_p<false>(p, slots, grid, lds, st);
}

inline int gatherv_mc(int M) { return M <= 2 ? 2 : (M <= 4 ? 4 : 8); }
// 5 <= M <= 8 with CSDR_HSDB_P16=1 (off by default): P in fp16, 8 columns in 16 bytes per
// (block, atom); the slice is half as large, two workgroups per CU and one LDS read per slot.
// One rounding per P value (about 2e-4 relative) which a decoder's layers compound.
inline bool gatherv_p16(int M) { return gatherv_mc(M) == 8 && env_flag("CSDR_HSDB_P16", false); }
inline int gatherv_wgs_per_cu(int mc, bool p16) { return mc == 8 && !p16 ? 1 : 2; }
inline size_t gatherv_p_atom_bytes(int mc, bool p16) { return p16 ? 16 : (size_t)mc * 4; }

// The 2 <= M <= 8 gather: MC = M rounded up to 2, 4 or 8; the 128 KiB fp32 P slice of MC = 8
// allows one workgroup per CU (4 waves per SIMD for the register budget), the smaller ones and
// the fp16 slice two.
template <int MC, int WPE, bool P16>
void launch_gatherv_mc(const Params& p, int slots, int grid, size_t lds, hipStream_t st) {
    constexpr int kDepth = MC == 8 && !P16 ? 6 : 4;
    const void* fn = nullptr;
    switch (slots) {
        case 4: fn = reinterpret_cast<const void*>(&gatherv_kernel<4, MC, kDepth, WPE, P16>); break;
        case 8: fn = reinterpret_cast<const void*>(&gatherv_kernel<8, MC, kDepth, WPE, P16>); break;
        default: fn = reinterpret_cast<const void*>(&gatherv_kernel<16, MC, kDepth, WPE, P16>); break;
    }
    if (lds > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    switch (slots) {
        case 4: gatherv_kernel<4, MC, kDepth, WPE, P16><<<grid, kGThreads, lds, st>>>(p); break;
        case 8: gatherv_kernel<8, MC, kDepth, WPE, P16><<<grid, kGThreads, lds, st>>>(p); break;
        default: gatherv_kernel<16, MC, kDepth, WPE, P16><<<grid, kGThreads, lds, st>>>(p); break;
    }
}

void launch_gatherv(const Params& p, int slots, int grid, size_t lds, hipStream_t st) {
    switch (gatherv_mc(p.M)) {
        case 2: launch_gatherv_mc<2, 8, false>(p, slots, grid, lds, st); break;
        case 4: launch_gatherv_mc<4, 8, false>(p, slots, grid, lds, st); break;
        default:
            if (p.p16)
                launch_gatherv_mc<8, 8, true>(p, slots, grid, lds, st);
            else
                launch_gatherv_mc<8, 4, false>(p, slots, grid, lds, st);
            break;
    }
}

// Row ranges for the M == 1 gather, balanced by bytes: a workgroup of a chunk of nbc block
// columns gets about U / nbc rows, U = all block-rows / target, so every workgroup streams
// about the same code bytes whatever its chunk's width. Per matrix, the full chunks share one
// split count (splits, rows_per_wg) and each remainder chunk (at most 4, widths NBc/2, ...,
// largest first) has its own (rsplit[j], rrpw[j]). Starting from floor(rows * width / U)
// ranges per chunk, ranges are added one class at a time (all full chunks of a matrix, or one
// remainder chunk) to the class with the most block-rows per workgroup while the total stays
// within the target.
void plan_gather_splits(Params& p, int n, long long target, int max_rows, long long round) {
    struct Cls {
        int g, j;       // matrix, remainder index (-1: the full chunks)
        int width, count, R;
        int splits;
    };
    Cls cls[kMaxGroup * 5];
    int ncls = 0;
    long long total_br = 0;  // block-rows of all matrices
    for (int i = 0; i < n; ++i) total_br += (long long)p.m[i].R * p.m[i].NB;
    const double U = std::max(1.0, (double)total_br / (double)std::max(1LL, target));
    long long used = 0;
    for (int i = 0; i < n; ++i) {
        const MatDesc& d = p.m[i];
        const int nfull = d.NB / d.NBc;
        auto add = [&](int j, int width, int count) {
            Cls c{i, j, width, count, d.R, 1};
            c.splits = (int)std::max(1.0, std::floor((double)d.R * width / U));
            c.splits = std::max(c.splits, (d.R + max_rows - 1) / max_rows);
            c.splits = std::min(c.splits, d.R);
            used += (long long)c.splits * count;
            cls[ncls++] = c;
        };
        if (nfull) add(-1, d.NBc, nfull);
        int j = 0;
        for (int bit = d.NBc >> 1; bit; bit >>= 1)
            if ((d.NB % d.NBc) & bit) add(j++, bit, 1);
    }
    // more workgroups than one round of the chip holds (the row limit forces it): fill whole
    // rounds, so the last one is not a fraction of the chip doing full-size work units
    if (used > target && round > 0) target = (used + round - 1) / round * round;
    for (;;) {
        int best = -1;
        double best_b = 0.0;
        for (int k = 0; k < ncls; ++k) {
            const Cls& c = cls[k];
            if (c.splits >= c.R || used + c.count > target) continue;
            const double b = (double)c.R * c.width / c.splits;
            if (b > best_b) {
                best_b = b;
                best = k;
            }
        }
        if (best < 0) break;
        ++cls[best].splits;
        used += cls[best].count;
    }
    int base = 0;
    for (int i = 0; i < n; ++i) {
        MatDesc& d = p.m[i];
        d.splits = 0;
        d.rows_per_wg = 1;
        for (int j = 0; j < 4; ++j) d.rsplit[j] = d.rrpw[j] = 0;
        int count = 0;
        for (int k = 0; k < ncls; ++k) {
            const Cls& c = cls[k];
            if (c.g != i) continue;
            const int rpw = (c.R + c.splits - 1) / c.splits;
            const int sp = (c.R + rpw - 1) / rpw;  // every range non-empty
            if (c.j < 0) {
                d.splits = sp;
                d.rows_per_wg = rpw;
            } else {
                d.rsplit[c.j] = sp;
                d.rrpw[c.j] = rpw;
            }
            count += sp * c.count;
        }
        d.g_base = base;
        d.g_count = count;
        base += count;
    }
}

constexpr int kPhaseDx = 1;
constexpr int kPhaseGather = 2;

struct XopArgs {
    int xop = CSDR_XOP_NONE;
    const void* const* x2 = nullptr;
    const float* nw = nullptr;
    float eps = 0.f;
    int nsplit = 0, hd = 0;
};

// fp16 P on the multi-column gather: at 5 <= M <= 8 where the thread-per-atom dx kernel (64-long
// blocks) writes P
bool group_p16(int n, const csdr_hsdb* const* segs, int M) {
    bool on = M >= 2 && M <= kMaxVecM && gatherv_p16(M);
    for (int i = 0; i < n && on; ++i) on = segs[i] && segs[i]->tile_cols == 64;
    return on;
}

// 2 <= M <= 8: the streaming multi-column gather reads every code once for all columns (fp32
// accumulation; P in fp32, or optionally fp16 at 5 <= M <= 8), where the matrix-core path decodes each
// weight through the LDS dictionary; it needs 1-row tiles of 4, 8 or 16 slots (the same count
// in the group) and a P slice within the gather's budget.
bool vec_path(int n, const csdr_hsdb* const* segs, int M) {
    bool vec = M >= 2 && M <= kMaxVecM;
    for (int i = 0; i < n && vec; ++i) {
        const csdr_hsdb* s = segs[i];
        const int mc = gatherv_mc(M);
        const bool p16 = group_p16(n, segs, M);
        const size_t lds = (size_t)s->NBc * s->K * gatherv_p_atom_bytes(mc, p16) +
                           (size_t)(64 + kGvMinRows) * 4 * mc;
        vec = s->tile_rows == 1 && s->NB > 0 && (s->slots == 4 || s->slots == 8 || s->slots == 16) &&
              s->slots == segs[0]->slots && lds <= (size_t)160 * 1024 / gatherv_wgs_per_cu(mc, p16);
    }
    return vec;
}

// A plain product (both phases, no x op) at batch M takes the matrix-core path.
bool plain_takes_mfma(int n, const csdr_hsdb* const* segs, int M) {
    return !vec_path(n, segs, M) && csdr::mfma_eligible(n, segs, M);
}

// Workspace a plain product at batch M needs on the path it takes.
size_t plain_ws_bytes(int n, const csdr_hsdb* const* segs, int M) {
    return plain_takes_mfma(n, segs, M) ? csdr::mfma_workspace_bytes(n, segs, M)
                                        : p_path_ws_bytes(n, segs, M);
}

int matmul_group(int n, const csdr_hsdb* const* segs, const void* const* xs, int x_dtype, int M,
                 float* const* ys, void* workspace, size_t workspace_bytes, hipStream_t st,
                 int phases = kPhaseDx | kPhaseGather, const float* const* bias = nullptr,
                 int flags = 0, const XopArgs& xa = XopArgs()) {
    if (n <= 0 || n > kMaxGroup || !segs || !xs || !ys || M <= 0)
        return set_error(CSDR_E_INVALID, "hsdb_matmul: bad argument (group of 1.." +
                                             std::to_string(kMaxGroup) + ")");
    if (x_dtype != CSDR_F32 && x_dtype != CSDR_F16)
        return set_error(CSDR_E_INVALID, "hsdb_matmul: x_dtype must be CSDR_F32 or CSDR_F16");
    for (int i = 0; i < n; ++i) {
        if (!segs[i] || !xs[i] || !ys[i])
            return set_error(CSDR_E_INVALID, "hsdb_matmul: null entry");
        if (!csdr::codes_on_device(segs[i]))
            return set_error(CSDR_E_UNSUPPORTED, kHostCodesMsg);
    }
    if (xa.xop != CSDR_XOP_NONE) {
        if (x_dtype != CSDR_F32 || M > kMaxXopM)
            return set_error(CSDR_E_INVALID, "hsdb_matmul: x ops take fp32 x and M <= " +
                                                 std::to_string(kMaxXopM));
        if (xa.xop == CSDR_XOP_RMSNORM && !xa.nw)
            return set_error(CSDR_E_INVALID, "hsdb_matmul: RMSNorm x op needs weights");
        if (xa.xop == CSDR_XOP_ATTN && (M != 1 || xa.nsplit <= 0 || xa.hd <= 0 || xa.hd % 4))
            return set_error(CSDR_E_INVALID, "hsdb_matmul: attention x op needs M == 1, splits, hd % 4 == 0");
        for (int i = 0; i < n; ++i) {
            if (segs[i]->tile_cols != 64)
                return set_error(CSDR_E_UNSUPPORTED, "hsdb_matmul: x ops need 64-column blocks");
            if (xa.xop == CSDR_XOP_SILU_MUL && (!xa.x2 || !xa.x2[i]))
                return set_error(CSDR_E_INVALID, "hsdb_matmul: SiLU x op needs x2");
        }
    }
    const bool tm = (flags & CSDR_HSDB_TOKEN_MAJOR) && M > 1;
    // 2 <= M <= 8: the streaming multi-column gather reads every code once for all columns
    // (fp32 unless CSDR_HSDB_P16=1), where the matrix-core path decodes each weight through the LDS
    // dictionary; it needs 1-row tiles of 4, 8 or 16 slots (the same count in the group) and
    // a P slice within the gather's budget
    const bool vec = vec_path(n, segs, M);
    if (phases == (kPhaseDx | kPhaseGather) && xa.xop == CSDR_XOP_NONE &&
        plain_takes_mfma(n, segs, M))
        return csdr::mfma_matmul(n, segs, xs, x_dtype, M, ys, bias,
                                 (flags & CSDR_HSDB_ACCUMULATE) ? 1 : 0, tm ? 1 : 0, workspace,
                                 workspace_bytes, st);
    const size_t need = p_path_ws_bytes(n, segs, M);
    if (!workspace || workspace_bytes < need)
        return set_error(CSDR_E_WORKSPACE,
                         "hsdb_matmul: workspace needs " + std::to_string(need) + " bytes");
    Params p{};
    p.G = n;
    p.M = M;
    p.p16 = vec && group_p16(n, segs, M) ? 1 : 0;
    // generic gather: P staged 4 columns at a time when that fits in LDS, else 1
    size_t max_pk = 0;
    for (int i = 0; i < n; ++i) max_pk = std::max(max_pk, (size_t)segs[i]->NBc * segs[i]->K);
    const int MV = (M == 1 || max_pk * 4 * 4 > 96 * 1024) ? 1 : 4;
    p.MVz = (M + MV - 1) / MV;
    p.x_f16 = (x_dtype == CSDR_F16);
    p.tm = tm ? 1 : 0;
    p.accumulate = (flags & CSDR_HSDB_ACCUMULATE) ? 1 : 0;
    p.xop = xa.xop;
    p.nw = xa.nw;
    p.eps = xa.eps;
    p.nsplit = xa.nsplit;
    p.hd = xa.hd;
    char* ws = static_cast<char*>(workspace);
    size_t off = csdr::kWsHead;
    p.inv = reinterpret_cast<float*>(ws);
    // the register-resident M == 1 gather needs every matrix at 4, 8 or 16 slots (16-byte
    // pieces) and the same count across the group; anything else takes the generic gather
    int slots = -1;
    bool fast = (M == 1);
    int ndx = 0;
    size_t lds_dx = 0, lds_g = 0;
    // 2 <= M <= 16 with 64-long blocks everywhere: the thread-per-atom dx kernel
    bool dxm = M >= 2 && M <= kMaxXopM;
    for (int i = 0; i < n; ++i) dxm = dxm && segs[i] && segs[i]->tile_cols == 64;
    // M == 1 with 64-long blocks and 16-byte aligned inputs: the matrix-core dx kernel
    bool dx1 = M == 1;
    for (int i = 0; i < n && dx1; ++i) {
        const uintptr_t al = reinterpret_cast<uintptr_t>(xs[i]) |
                             (xa.xop == CSDR_XOP_SILU_MUL ? reinterpret_cast<uintptr_t>(xa.x2[i]) : 0);
        dx1 = segs[i] && segs[i]->tile_cols == 64 && al % 16 == 0;
    }
    const int dxm_mc = M <= 2 ? 2 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16));
    for (int i = 0; i < n; ++i) {
        const csdr_hsdb* s = segs[i];
        if (!s || !xs[i] || !ys[i]) return set_error(CSDR_E_INVALID, "hsdb_matmul: null entry");
        if (s->tile_rows != 1)
            return set_error(CSDR_E_FORMAT,
                             "hsdb_matmul: fused matmul requires tile_rows == 1; use "
                             "csdr_hsdb_decompress + a dense matmul for 2-D tiles");
        if (s->NB == 0)
            return set_error(CSDR_E_UNSUPPORTED, "hsdb_matmul: matrix narrower than one block");
        if (!(s->slots == 4 || s->slots == 8 || s->slots == 16)) fast = false;
        if ((size_t)s->NBc * s->K > kGMaxP) fast = false;  // the gather's P slice registers
        if (slots >= 0 && (int)s->slots != slots) fast = false;
        slots = (int)s->slots;
        MatDesc& d = p.m[i];
        d.codes = s->d_codes;
        d.dict = s->d_dict;
        d.slot_gamma = s->d_slot_gamma;
        d.gunif = 1;
        for (uint32_t q = 0; q < s->slots && q < (uint32_t)kMaxSlotsArg; ++q) {
            d.sgam[q] = s->h_slot_gamma[q];
            if (d.sgam[q] != d.sgam[0]) d.gunif = 0;
        }
        d.edge = s->d_edge;
        d.x = xs[i];
        d.y = ys[i];
        d.bias = bias ? bias[i] : nullptr;
        d.P = reinterpret_cast<float*>(ws + off);
        d.x2 = (xa.xop == CSDR_XOP_SILU_MUL) ? xa.x2[i] : nullptr;
        d.xe = (xa.xop != CSDR_XOP_NONE && s->Ce > 0)
                   ? reinterpret_cast<float*>(ws + off +
                                              csdr::align_up((size_t)s->NB * s->K * M * 4, 256))
                   : nullptr;
        off += p_bytes(s, M);
        d.R = (int)s->R;
        d.K = (int)s->K;
        d.NB = (int)s->NB;
        d.NBc = (int)s->NBc;
        d.nchunks = (int)s->nchunks;
        d.slots = (int)s->slots;
        d.blen = (int)s->tile_cols;
        d.Ce = (int)s->Ce;
        d.C_full = (int)s->C_full;
        d.PB = producer_blocks(M);
        if (dx1) {
            d.PB = 16;
            d.dx_count = ((d.K + 63) / 64) * ((d.NB + 15) / 16);
        } else if (dxm) {
            // 64 atoms by one 16-wide tile of (block column, column) pairs per workgroup
            d.dx_count = ((d.K + 63) / 64) * ((d.NB * dxm_mc + 15) / 16);
        } else if (d.blen == 64) {
            d.dx_count = ((d.K + 15) / 16) * ((d.NB + d.PB - 1) / d.PB);
            size_t extra = 0;
            if (xa.xop == CSDR_XOP_ATTN)  // split weights of the heads a workgroup covers
                extra = ((size_t)d.PB * 64 / std::max(1, xa.hd) + 2) * (xa.nsplit + 1) * 4;
            lds_dx = std::max(lds_dx, (size_t)d.PB * 64 * M * 4 + extra);
        } else {
            const long long items = (long long)d.NB * d.K * ((M + 7) / 8);
            d.dx_count = (int)((items + kThreads / 64 - 1) / (kThreads / 64));
        }
        d.dx_base = ndx;
        ndx += d.dx_count;
    }
    int dev = 0, ncu = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            v > 0)
            ncu = v;
    }
    int base = 0;
    if (fast || vec) {
        // M == 1: kGWgsPerCu workgroups per CU; 2 <= M <= 8: as many as the P slice of MC
        // columns allows; fewer for small groups: at least kGMinWgBytes of codes per workgroup
        // (each one stages a P slice first)
        const int mc = fast ? 1 : gatherv_mc(M);
        const bool p16 = !fast && p.p16;
        const int wpc = fast ? kGWgsPerCu : gatherv_wgs_per_cu(mc, p16);
        long long target = (long long)ncu * wpc;
        // rows per workgroup: M == 1 kGMaxRows; else what the LDS share left by the widest P
        // slice holds (row totals of mc floats)
        int max_rows = kGMaxRows;
        if (!fast) {
            size_t pk = 0;
            for (int i = 0; i < n; ++i) pk = std::max(pk, (size_t)segs[i]->NBc * segs[i]->K);
            const size_t share = (size_t)160 * 1024 / wpc;
            max_rows = (int)std::min<size_t>(
                kGMaxRows, (share - pk * gatherv_p_atom_bytes(mc, p16) - 64 * mc * 4) / (mc * 4));
        }
        long long code_bytes = 0;
        for (int i = 0; i < n; ++i) code_bytes += (long long)p.m[i].R * p.m[i].NB * slots * 4;
        const long long min_bytes = kGMinWgBytes;
        target = std::max(1LL, std::min(target, code_bytes / std::max(1LL, min_bytes)));
        plan_gather_splits(p, n, target, max_rows, (long long)ncu * wpc);
        for (int i = 0; i < n; ++i) {
            const MatDesc& d = p.m[i];
            int rows = d.splits ? d.rows_per_wg : 0;  // rows per workgroup
            for (int j = 0; j < 4; ++j)
                if (d.rsplit[j]) rows = std::max(rows, d.rrpw[j]);
            lds_g = std::max(lds_g, (size_t)d.NBc * d.K * (fast ? 4 : gatherv_p_atom_bytes(mc, p16)) +
                                        (size_t)(64 + rows) * 4 * mc);
            base += d.g_count;
        }
    } else {
        for (int i = 0; i < n; ++i) {
            MatDesc& d = p.m[i];
            d.Rt = MV == 1 ? 256 : 64;
            while (d.Rt > 16 && (size_t)d.Rt * d.NBc > 2048) d.Rt /= 2;
            d.splits = (d.R + d.Rt - 1) / d.Rt;
            lds_g = std::max(lds_g, ((size_t)d.NBc * d.K * MV + (size_t)d.Rt * d.NBc * MV) * 4);
            d.g_base = base;
            d.g_count = (d.nchunks + 7) / 8 * 8 * d.splits;
            base += d.g_count;
        }
    }
    if (lds_g > 160 * 1024 || lds_dx > 160 * 1024)
        return set_error(CSDR_E_UNSUPPORTED, "hsdb_matmul: dictionary too large for LDS");
    if ((phases & kPhaseDx) && dx1) {
        switch (p.xop) {
            case CSDR_XOP_RMSNORM: dx1_mfma_kernel<CSDR_XOP_RMSNORM><<<ndx, kThreads, 0, st>>>(p); break;
            case CSDR_XOP_SILU_MUL: dx1_mfma_kernel<CSDR_XOP_SILU_MUL><<<ndx, kThreads, 0, st>>>(p); break;
            case CSDR_XOP_ATTN: dx1_mfma_kernel<CSDR_XOP_ATTN><<<ndx, kThreads, 0, st>>>(p); break;
            default: dx1_mfma_kernel<CSDR_XOP_NONE><<<ndx, kThreads, 0, st>>>(p); break;
        }
        CSDR_LAUNCH_CHECK("hsdb dx");
    } else if ((phases & kPhaseDx) && dxm) {
        if (p.xop == CSDR_XOP_RMSNORM) {
            rms_inv_kernel<<<dim3(M, n), kThreads, 0, st>>>(p);
            CSDR_LAUNCH_CHECK("hsdb rms");
        }
        auto go = [&](auto kern) { kern<<<ndx, kThreads, 0, st>>>(p); };
        const int key = p.xop * 100 + dxm_mc;
        switch (key) {
            case CSDR_XOP_NONE * 100 + 2: go(dxmm_kernel<CSDR_XOP_NONE, 2>); break;
            case CSDR_XOP_NONE * 100 + 4: go(dxmm_kernel<CSDR_XOP_NONE, 4>); break;
            case CSDR_XOP_NONE * 100 + 8: go(dxmm_kernel<CSDR_XOP_NONE, 8>); break;
            case CSDR_XOP_NONE * 100 + 16: go(dxmm_kernel<CSDR_XOP_NONE, 16>); break;
            case CSDR_XOP_RMSNORM * 100 + 2: go(dxmm_kernel<CSDR_XOP_RMSNORM, 2>); break;
            case CSDR_XOP_RMSNORM * 100 + 4: go(dxmm_kernel<CSDR_XOP_RMSNORM, 4>); break;
            case CSDR_XOP_RMSNORM * 100 + 8: go(dxmm_kernel<CSDR_XOP_RMSNORM, 8>); break;
            case CSDR_XOP_RMSNORM * 100 + 16: go(dxmm_kernel<CSDR_XOP_RMSNORM, 16>); break;
            case CSDR_XOP_SILU_MUL * 100 + 2: go(dxmm_kernel<CSDR_XOP_SILU_MUL, 2>); break;
            case CSDR_XOP_SILU_MUL * 100 + 4: go(dxmm_kernel<CSDR_XOP_SILU_MUL, 4>); break;
            case CSDR_XOP_SILU_MUL * 100 + 8: go(dxmm_kernel<CSDR_XOP_SILU_MUL, 8>); break;
            case CSDR_XOP_SILU_MUL * 100 + 16: go(dxmm_kernel<CSDR_XOP_SILU_MUL, 16>); break;
            default: return set_error(CSDR_E_INVALID, "hsdb_matmul: x op not available at M > 1");
        }
        CSDR_LAUNCH_CHECK("hsdb dx");
    } else if (phases & kPhaseDx) {
        switch (p.xop) {
            case CSDR_XOP_RMSNORM:
                dx_kernel<CSDR_XOP_RMSNORM><<<ndx, kThreads, lds_dx, st>>>(p);
                break;
            case CSDR_XOP_SILU_MUL:
                dx_kernel<CSDR_XOP_SILU_MUL><<<ndx, kThreads, lds_dx, st>>>(p);
                break;
            case CSDR_XOP_ATTN:
                dx_kernel<CSDR_XOP_ATTN><<<ndx, kThreads, lds_dx, st>>>(p);
                break;
            default:
                dx_kernel<CSDR_XOP_NONE><<<ndx, kThreads, lds_dx, st>>>(p);
                break;
        }
        CSDR_LAUNCH_CHECK("hsdb dx");
    }
    if (phases & kPhaseGather) {
        if (fast)
            launch_gatherw(p, slots, base, lds_g, st);
        else if (vec) {
            p.gtotal = base;
            launch_gatherv(p, slots, (base + 7) / 8 * 8, lds_g, st);
        }
        else if (MV == 1)
            gatherm_kernel<1><<<base, kThreads, lds_g, st>>>(p);
        else
            gatherm_kernel<4><<<base, kThreads, lds_g, st>>>(p);
        CSDR_LAUNCH_CHECK("hsdb gather");
    }
    return CSDR_OK;
}

// ---- the allocation-free product's scratch memory
// A file-scope device array that holds the product's workspace (P slices, or the transposed
// X of the matrix-core path) for callers that cannot allocate (code under HIP graph capture,
// serving loops). Each device holds its own copy for the life of the process; its address on
// a device comes from hipGetSymbolAddress, taken once per device with that device current
// (the array's name in host code is not a device address). Every call on a device shares
// that device's copy, so calls that overlap on one device race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's scratch address (taken on its first use), or null with the error recorded.
void* scratch_for(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        set_error(CSDR_E_INVALID, "hsdb_matmul_noalloc: device ordinal out of range");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error(CSDR_E_HIP, std::string("hsdb_matmul_noalloc: hipGetSymbolAddress: ") +
                                      hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
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

CSDR_API int csdr_hsdb_load_host(const void* stream, size_t nbytes, void* hip_stream,
                                 csdr_hsdb** out) {
    if (!out) return set_error(CSDR_E_INVALID, "hsdb_load_host: null out");
    *out = nullptr;
    csdr_hsdb* s = new (std::nothrow) csdr_hsdb();
    if (!s) return set_error(CSDR_E_INVALID, "hsdb_load_host: out of host memory");
    if (hipGetDevice(&s->device) != hipSuccess) {
        delete s;
        return set_error(CSDR_E_HIP, "hsdb_load_host: no HIP device");
    }
    int rc;
    try {
        rc = parse_and_upload(static_cast<const uint8_t*>(stream), nbytes,
                              static_cast<hipStream_t>(hip_stream), s, true);
    } catch (const std::bad_alloc&) {
        rc = set_error(CSDR_E_INVALID, "hsdb_load_host: out of host memory");
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
    return group_ws_bytes(1, &s, M);
}

CSDR_API size_t csdr_hsdb_group_workspace_bytes(int n, const csdr_hsdb* const* segs, int M) {
    if (n <= 0 || !segs || M <= 0) return 0;
    for (int i = 0; i < n; ++i)
        if (!segs[i]) return 0;
    return group_ws_bytes(n, segs, M);
}

CSDR_API int csdr_hsdb_matmul(const csdr_hsdb* s, const void* x, int x_dtype, int M, float* y,
                              void* workspace, size_t workspace_bytes, void* hip_stream) {
    return matmul_group(1, &s, &x, x_dtype, M, &y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_hsdb_matmul_noalloc(const csdr_hsdb* s, const void* x, int x_dtype, int M,
                                      float* y, void* hip_stream) {
    if (!s || !x || !y || M <= 0)
        return set_error(CSDR_E_INVALID, "hsdb_matmul_noalloc: bad argument");
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess)
        return set_error(CSDR_E_HIP, "hsdb_matmul_noalloc: no HIP device");
    if (dev != s->device)
        return set_error(CSDR_E_INVALID,
                         "hsdb_matmul_noalloc: the segment lives on device " +
                             std::to_string(s->device) + ", the current device is " +
                             std::to_string(dev));
    // sized for the path this plain product takes (a matrix-core product needs only its
    // transposed X, far less than the P path would at the same M)
    const size_t need = plain_ws_bytes(1, &s, M);
    if (need > kScratchBytes)
        return set_error(CSDR_E_WORKSPACE,
                         "hsdb_matmul_noalloc: this product needs " + std::to_string(need) +
                             " bytes of scratch, the allocation-free entry point has " +
                             std::to_string(kScratchBytes) +
                             "; use csdr_hsdb_matmul with a caller workspace");
    void* ws = scratch_for(dev);
    if (!ws) return CSDR_E_HIP;
    return matmul_group(1, &s, &x, x_dtype, M, &y, ws, kScratchBytes,
                        static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_hsdb_matmul_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream) {
    return matmul_group(n, segs, x, x_dtype, M, y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_hsdb_matmul_group_ex(int n, const csdr_hsdb* const* segs, const void* const* x,
                                       int x_dtype, int M, float* const* y,
                                       const float* const* bias, int flags, void* workspace,
                                       size_t workspace_bytes, void* hip_stream) {
    return matmul_group(n, segs, x, x_dtype, M, y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream), kPhaseDx | kPhaseGather, bias,
                        flags);
}

CSDR_API int csdr_hsdb_matmul_group_xop(int n, const csdr_hsdb* const* segs,
                                        const void* const* x, const void* const* x2, int M,
                                        float* const* y, const float* const* bias, int flags,
                                        int xop, const float* norm_w, float eps, int attn_splits,
                                        int attn_head_dim, void* workspace,
                                        size_t workspace_bytes, void* hip_stream) {
    if (xop < CSDR_XOP_NONE || xop > CSDR_XOP_ATTN)
        return set_error(CSDR_E_INVALID, "hsdb_matmul_group_xop: unknown x op");
    XopArgs xa;
    xa.xop = xop;
    xa.x2 = x2;
    xa.nw = norm_w;
    xa.eps = eps;
    xa.nsplit = attn_splits;
    xa.hd = attn_head_dim;
    return matmul_group(n, segs, x, CSDR_F32, M, y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream), kPhaseDx | kPhaseGather, bias,
                        flags, xa);
}

CSDR_API int csdr_hsdb_decode_row(const csdr_hsdb* s, const int* row_dev, int row_host, float* out,
                                  void* hip_stream) {
    if (!s || !out) return set_error(CSDR_E_INVALID, "hsdb_decode_row: bad argument");
    if (!csdr::codes_on_device(s)) return set_error(CSDR_E_UNSUPPORTED, kHostCodesMsg);
    if (s->tile_rows != 1)
        return set_error(CSDR_E_FORMAT, "hsdb_decode_row: needs 1-row tiles");
    if (!row_dev && (row_host < 0 || (uint32_t)row_host >= s->R))
        return set_error(CSDR_E_INVALID, "hsdb_decode_row: row out of range");
    decode_row_kernel<<<grid_for(s->C), kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(
        *s, row_dev, row_host, out);
    CSDR_LAUNCH_CHECK("hsdb decode_row");
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_decode_rows(const csdr_hsdb* s, const int* rows_dev, int n, float* out,
                                   void* hip_stream) {
    if (!s || !rows_dev || !out || n <= 0 || n > 65535)
        return set_error(CSDR_E_INVALID, "hsdb_decode_rows: bad argument");
    if (!csdr::codes_on_device(s)) return set_error(CSDR_E_UNSUPPORTED, kHostCodesMsg);
    if (s->tile_rows != 1)
        return set_error(CSDR_E_FORMAT, "hsdb_decode_rows: needs 1-row tiles");
    decode_row_kernel<<<dim3(grid_for(s->C), n), kThreads, 0,
                        static_cast<hipStream_t>(hip_stream)>>>(*s, rows_dev, 0, out);
    CSDR_LAUNCH_CHECK("hsdb decode_rows");
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_dx_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                int x_dtype, int M, float* const* y, void* workspace,
                                size_t workspace_bytes, void* hip_stream) {
    return matmul_group(n, segs, x, x_dtype, M, y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream), kPhaseDx);
}

CSDR_API int csdr_hsdb_gather_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream) {
    return matmul_group(n, segs, x, x_dtype, M, y, workspace, workspace_bytes,
                        static_cast<hipStream_t>(hip_stream), kPhaseGather);
}

CSDR_API int csdr_hsdb_decompress(const csdr_hsdb* s, float* w, void* hip_stream) {
    if (!s || !w) return set_error(CSDR_E_INVALID, "hsdb_decompress: bad argument");
    if (!csdr::codes_on_device(s)) return set_error(CSDR_E_UNSUPPORTED, kHostCodesMsg);
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
    if (!csdr::codes_on_device(s)) return set_error(CSDR_E_UNSUPPORTED, kHostCodesMsg);
    const size_t work = (size_t)s->n_tiles * s->slots;
    if (work) {
        export_codes_kernel<<<grid_for(work), kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(
            *s, packed, coef_abs);
        CSDR_LAUNCH_CHECK("hsdb export");
    }
    return CSDR_OK;
}

}  // extern "C"
