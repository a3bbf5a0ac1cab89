// decoder_ops.hip — decoder elementwise ops, flash-decode attention and token selection
// for the compressed-weight decoder (gfx950).
//
// Reference (cortexSDR tree, api/cortex_sdk.cpp): rms_norm :1208-1232, silu_mul :1245-1256,
// get_rope_cache / apply_rope_inplace :1363-1423 (adjacent pairs, freq = theta^(-i/d)),
// repeat_kv_heads :1453-1478 (q head h reads kv head h / (Hq/Hkv)), select_best_from_logits
// :1005-1030 (logit/temperature - penalty if repeated; strict '>' keeps the first maximum;
// non-finite skipped); attention as kernels/attention_kernels.cpp:26-113 with a cache, the
// behaviour kernels/flash_attention.cpp:165-247 intends.
//
// Positions and lengths are read from device memory (int32) so that a decode step can be
// captured once in a HIP graph and replayed for every token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include <cmath>
#include <string>

#include "common.hpp"

namespace {

using csdr::attn_vec_offset;
using csdr::set_error;

constexpr int kThreads = 256;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = csdr::wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = -INFINITY;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s = fmaxf(s, red[i]);
    return s;
}

// ---------------------------------------------------------------- RMSNorm

// One workgroup per row (blockDim 256 or 1024); each thread keeps its elements in registers
// between the sum of squares and the scaling (at most 8 per thread, else re-read).
__global__ __launch_bounds__(1024) void rms_norm_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w, int n,
                                                        float eps, float* __restrict__ y) {
    __shared__ float red[1024 / 64];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    const int nt = blockDim.x;
    float xv[8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int i = threadIdx.x + j * nt;
        xv[j] = i < n ? xr[i] : 0.f;
        ss = fmaf(xv[j], xv[j], ss);
    }
    for (int i = threadIdx.x + 8 * nt; i < n; i += nt) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int i = threadIdx.x + j * nt;
        if (i < n) yr[i] = xv[j] * inv * w[i];
    }
    for (int i = threadIdx.x + 8 * nt; i < n; i += nt) yr[i] = xr[i] * inv * w[i];
}

// ---------------------------------------------------------------- SiLU(g) * u

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float* __restrict__ g,
                                                            const float* __restrict__ u,
                                                            size_t n, float* __restrict__ y) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads) {
        const float x = g[i];
        const float sig = 1.0f / (1.0f + expf(-x));
        y[i] = (x * sig) * u[i];
    }
}

// ---------------------------------------------------------------- RoPE + KV append

// q: ntok x Hq x hd, k: ntok x Hkv x hd (rotated in place); v: ntok x Hkv x hd.
// Token t sits at position pos0 + t (pos0 = *pos_dev). K and V go to the fp16 caches laid
// out [position][kv head][hd] with row capacity max_ctx. One workgroup per (token, head):
// blocks [0, Hq) rotate query heads, [Hq, Hq + Hkv) rotate a key head and append it (and the
// value head) to the caches.
__global__ __launch_bounds__(64) void rope_kv_kernel(float* __restrict__ q,
                                                     float* __restrict__ k,
                                                     const float* __restrict__ v, int ntok,
                                                     int Hq, int Hkv, int hd,
                                                     const int* __restrict__ pos_dev,
                                                     float theta, _Float16* kcache,
                                                     _Float16* vcache, int max_ctx) {
    const int t = blockIdx.x / (Hq + Hkv);
    const int head = blockIdx.x % (Hq + Hkv);
    const int pos = *pos_dev + t;
    const int half = hd / 2;
    const int rot = hd - (hd % 2);
    float* base = head < Hq ? q + ((size_t)t * Hq + head) * hd
                            : k + ((size_t)t * Hkv + (head - Hq)) * hd;
    for (int e = threadIdx.x; e < half; e += 64) {
        const int i2 = 2 * e;
        if (i2 >= rot) continue;
        const float freq = powf(theta, -((float)i2 / (float)hd));
        const float ang = (float)pos * freq;
        const float c = cosf(ang), sn = sinf(ang);
        const float x0 = base[i2], x1 = base[i2 + 1];
        // explicit fma forms, the same in the fused attention, so both paths round alike
        base[i2] = fmaf(x0, c, -(x1 * sn));
        base[i2 + 1] = fmaf(x0, sn, x1 * c);
    }
    if (head < Hq || pos >= max_ctx) return;
    __syncthreads();
    const int kh = head - Hq;
    const size_t src = ((size_t)t * Hkv + kh) * hd;
    const size_t dst = ((size_t)pos * Hkv + kh) * hd;
    for (int e = threadIdx.x; e < hd; e += 64) {
        kcache[dst + e] = (_Float16)base[e];
        vcache[dst + e] = (_Float16)v[src + e];
    }
}

// ---------------------------------------------------------------- flash-decode attention

// Split attention over positions [s*S, min(L, (s+1)*S)) (n <= 256) for the GW query heads (of
// one batch entry) that share KV head kvh, staged through LDS: every K and V piece of the
// split's rows is loaded up front (one memory round trip) and stored to LDS as fp16, rows
// padded by 16 bytes against bank conflicts; scores with one thread per position (its K row
// read once, the query heads broadcast from LDS); softmax statistics per head by one wave;
// P.V with threads over the (head, dim) outputs, reading V columns from LDS (no cross-lane
// reductions). Writes part = (max score m, sum of exp l, o[hd] = sum exp * v) per head, or
// the normalised output when the call has one split and an output.
// ROPE: the query is rotated in registers at position L - 1, position L - 1's key and value
// come from the projections (k_new rotated, both rounded to fp16 as the cache holds them),
// and the workgroup whose split holds L - 1 appends them to the caches.
struct RopeArgs {
    const float* knew;  // B x Hkv x HD (fp32, unrotated)
    const float* vnew;
    _Float16* kcw;      // fp16 caches (written at position L - 1)
    _Float16* vcw;
    float theta;
    float* kcw32;       // fp32 caches (the fp32 K/V form of attn_split_kernel)
    float* vcw32;
};

// Eight consecutive K or V values of one cache row, as the cache stores them (fp16: one
// 16-byte piece; fp32: two), read as fp32.
template <typename KT>
struct Row8;
template <>
struct Row8<_Float16> {
    h8 v;
    __device__ static Row8 load(const _Float16* p) {
        Row8 r;
        r.v = __builtin_nontemporal_load(reinterpret_cast<const h8*>(p));  // read once per step
        return r;
    }
    __device__ void store(_Float16* p) const { *reinterpret_cast<h8*>(p) = v; }
    __device__ float get(int i) const { return (float)v[i]; }
    __device__ void set(int i, float x) { v[i] = (_Float16)x; }  // the cache's rounding
};
template <>
struct Row8<float> {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 a, b;
    __device__ static Row8 load(const float* p) {
        Row8 r;
        r.a = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));  // read once per step
        r.b = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p) + 1);
        return r;
    }
    __device__ void store(float* p) const {
        reinterpret_cast<f4*>(p)[0] = a;
        reinterpret_cast<f4*>(p)[1] = b;
    }
    __device__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
    __device__ void set(int i, float x) {
        if (i < 4) a[i] = x;
        else b[i - 4] = x;
    }
};
template <typename KT>
__device__ __forceinline__ KT* cache_w(const RopeArgs& ra, bool v);
template <>
__device__ __forceinline__ _Float16* cache_w<_Float16>(const RopeArgs& ra, bool v) {
    return v ? ra.vcw : ra.kcw;
}
template <>
__device__ __forceinline__ float* cache_w<float>(const RopeArgs& ra, bool v) {
    return v ? ra.vcw32 : ra.kcw32;
}

constexpr int kAttnMaxS = 256;  // positions per split, at most (one thread per position)

// Split partials in the workspace: n = B * Hq * nsplit of them, partial i = (b * Hq + h) *
// nsplit + s; the n (max, sum) pairs come first (a consumer loads the whole table coalesced),
// then, from the next 16-byte boundary (attn_vec_offset), the n unnormalised HD-vectors.

// LDS bytes of attn_lds_kernel<HD, GW> at split length S
constexpr size_t attn_lds_bytes(int HD, int GW, int S) {
    return (size_t)2 * S * (HD + 8) * 2 + (size_t)GW * HD * 4 + (size_t)GW * S * 4 +
           (size_t)GW * 2 * 4 + (size_t)kThreads * 4;
}

template <int HD, int GW, bool ROPE>
__global__ __launch_bounds__(kThreads) void attn_lds_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ kc, const _Float16* __restrict__ vc,
    const int* __restrict__ lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
    float* __restrict__ part, float* __restrict__ out, int nsplit, RopeArgs ra) {
    constexpr int HDP = HD + 8;                             // padded row, halves
    constexpr int PPR = HD / 8;                             // 16-byte pieces per row
    constexpr int kPPT = kAttnMaxS * PPR / kThreads;        // pieces per thread, at most
    extern __shared__ float smem[];
    _Float16* tk = reinterpret_cast<_Float16*>(smem);       // S x HDP
    _Float16* tv = tk + (size_t)S * HDP;                    // S x HDP
    float* qs = reinterpret_cast<float*>(tv + (size_t)S * HDP);  // GW x HD
    float* sc = qs + GW * HD;                               // GW x S
    float* stat = sc + GW * S;                              // GW x 2
    float* red = stat + GW * 2;                             // kThreads
    const int G = Hq / Hkv;
    const size_t npart = (size_t)(gridDim.x / Hkv) * Hq * nsplit;  // partials in the workspace
    const int b = blockIdx.x / Hkv, kvh = blockIdx.x % Hkv;
    const int s = blockIdx.y;
    const int h0 = kvh * G + blockIdx.z * GW;
    const int nh = min(GW, G - (int)blockIdx.z * GW);
    // a length beyond the cache capacity is clamped to it (no K/V row past T is read or written)
    const int L = min(max(lens ? lens[b] : len_host, 0), T);
    const int p0 = s * S, p1 = min(L, p0 + S);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool direct = (nsplit == 1 && out != nullptr);
    if (p0 >= p1) {  // empty split (the length is below this split's range)
        for (int g = 0; g < nh; ++g) {
            const int bh = b * Hq + h0 + g;
            const size_t pi = (size_t)bh * nsplit + s;
            float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
            float* pst = part + 2 * pi;              // its (max, sum)
            if (!direct) {
                if (tid == 0) {
                    pst[0] = -INFINITY;
                    pst[1] = 0.f;
                }
                for (int i = tid; i < HD; i += kThreads) pp[i] = 0.f;
            } else {
                for (int i = tid; i < HD; i += kThreads) out[(size_t)bh * HD + i] = 0.f;
            }
        }
        return;
    }
    const int n = p1 - p0;
    const size_t rstride = (size_t)Hkv * HD;
    const _Float16* kb = kc + ((size_t)b * T * Hkv + kvh) * HD;
    const _Float16* vb = vc + ((size_t)b * T * Hkv + kvh) * HD;

    // 1. the split's K and V rows, every load issued before the first use
    h8 kr[kPPT], vr[kPPT];
#pragma unroll
    for (int k = 0; k < kPPT; ++k) {
        const int idx = tid + k * kThreads, p = idx / PPR, j = idx - p * PPR;
        if (p < n) {
            kr[k] = *reinterpret_cast<const h8*>(kb + (size_t)(p0 + p) * rstride + j * 8);
            vr[k] = *reinterpret_cast<const h8*>(vb + (size_t)(p0 + p) * rstride + j * 8);
        }
    }
    // the query heads (rotated at L - 1), into LDS
    const int plast = L - 1;
    for (int e = tid; e < nh * (HD / 2); e += kThreads) {
        const int g = e / (HD / 2), i2 = 2 * (e - g * (HD / 2));
        const float* qh = q + ((size_t)b * Hq + h0 + g) * HD;
        float x0 = qh[i2], x1 = qh[i2 + 1];
        if constexpr (ROPE) {
            const float freq = powf(ra.theta, -((float)i2 / (float)HD));
            const float ang = (float)plast * freq;
            const float c = cosf(ang), sn = sinf(ang);
            const float r0 = fmaf(x0, c, -(x1 * sn)), r1 = fmaf(x0, sn, x1 * c);
            x0 = r0;
            x1 = r1;
        }
        qs[g * HD + i2] = x0;
        qs[g * HD + i2 + 1] = x1;
    }
    // (with ROPE the row of position L - 1 is written below, from the new key and value, and
    // by no other thread: the cache row there is not written yet)
#pragma unroll
    for (int k = 0; k < kPPT; ++k) {
        const int idx = tid + k * kThreads, p = idx / PPR, j = idx - p * PPR;
        if (p < n && !(ROPE && p0 + p == plast)) {
            *reinterpret_cast<h8*>(tk + (size_t)p * HDP + j * 8) = kr[k];
            *reinterpret_cast<h8*>(tv + (size_t)p * HDP + j * 8) = vr[k];
        }
    }
    if constexpr (ROPE) {
        // position L - 1: the new key (rotated) and value, rounded to fp16, in the tile and,
        // from the split that holds it, appended to the caches
        if (plast >= p0 && plast < p1 && tid < HD / 2) {
            const int i2 = 2 * tid;
            const float* kn = ra.knew + ((size_t)b * Hkv + kvh) * HD;
            const float* vn = ra.vnew + ((size_t)b * Hkv + kvh) * HD;
            const float freq = powf(ra.theta, -((float)i2 / (float)HD));
            const float ang = (float)plast * freq;
            const float c = cosf(ang), sn = sinf(ang);
            const float k0 = kn[i2], k1 = kn[i2 + 1];
            const _Float16 a0 = (_Float16)fmaf(k0, c, -(k1 * sn));
            const _Float16 a1 = (_Float16)fmaf(k0, sn, k1 * c);
            const _Float16 w0 = (_Float16)vn[i2], w1 = (_Float16)vn[i2 + 1];
            const int pr = plast - p0;
            tk[(size_t)pr * HDP + i2] = a0;
            tk[(size_t)pr * HDP + i2 + 1] = a1;
            tv[(size_t)pr * HDP + i2] = w0;
            tv[(size_t)pr * HDP + i2 + 1] = w1;
            if (blockIdx.z == 0) {
                const size_t at = ((size_t)b * T + plast) * rstride + (size_t)kvh * HD + i2;
                ra.kcw[at] = a0;
                ra.kcw[at + 1] = a1;
                ra.vcw[at] = w0;
                ra.vcw[at + 1] = w1;
            }
        }
    }
    __syncthreads();

    // 2. scores: thread p over the query heads
    if (tid < n) {
        float acc[GW];
#pragma unroll
        for (int g = 0; g < GW; ++g) acc[g] = 0.f;
        const _Float16* kr0 = tk + (size_t)tid * HDP;
#pragma unroll 4
        for (int j = 0; j < PPR; ++j) {
            const h8 kv = *reinterpret_cast<const h8*>(kr0 + j * 8);
#pragma unroll
            for (int g = 0; g < GW; ++g) {
                if (g < nh) {
                    const float4 qa = *reinterpret_cast<const float4*>(qs + g * HD + j * 8);
                    const float4 qb = *reinterpret_cast<const float4*>(qs + g * HD + j * 8 + 4);
                    float d = acc[g];
                    d = fmaf(qa.x, (float)kv[0], d);
                    d = fmaf(qa.y, (float)kv[1], d);
                    d = fmaf(qa.z, (float)kv[2], d);
                    d = fmaf(qa.w, (float)kv[3], d);
                    d = fmaf(qb.x, (float)kv[4], d);
                    d = fmaf(qb.y, (float)kv[5], d);
                    d = fmaf(qb.z, (float)kv[6], d);
                    d = fmaf(qb.w, (float)kv[7], d);
                    acc[g] = d;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < GW; ++g)
            if (g < nh) sc[g * S + tid] = acc[g] * scale;
    }
    __syncthreads();

    // 3. softmax statistics per head (wave w handles heads w, w + 4, ...)
    for (int g = wave; g < nh; g += kThreads / 64) {
        float m = -INFINITY;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, sc[g * S + j]);
        m = wave_max(m);
        float l = 0.f;
        for (int j = lane; j < n; j += 64) {
            const float e = expf(sc[g * S + j] - m);
            sc[g * S + j] = e;
            l += e;
        }
        l = csdr::wave_sum(l);
        if (lane == 0) {
            stat[g * 2] = m;
            stat[g * 2 + 1] = l;
        }
    }
    __syncthreads();

    // 4. P.V over the (head, dim) outputs; positions split into `parts` interleaved ranges
    // when there are fewer outputs than threads
    const int O = nh * HD;
    const int parts = O >= kThreads ? 1 : kThreads / O;
    auto finish = [&](int o, float v) {
        const int g = o / HD, d = o - g * HD;
        const int bh = b * Hq + h0 + g;
        if (direct) {
            out[(size_t)bh * HD + d] = v / stat[g * 2 + 1];
        } else {
            const size_t pi = (size_t)bh * nsplit + s;
            float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
            float* pst = part + 2 * pi;              // its (max, sum)
            pp[d] = v;
            if (d == 0) {
                pst[0] = stat[g * 2];
                pst[1] = stat[g * 2 + 1];
            }
        }
    };
    if (parts == 1) {
        for (int o = tid; o < O; o += kThreads) {
            const int g = o / HD, d = o - g * HD;
            const float* e = sc + g * S;
            float acc = 0.f;
            for (int p = 0; p < n; ++p) acc = fmaf(e[p], (float)tv[(size_t)p * HDP + d], acc);
            finish(o, acc);
        }
    } else {
        const int o = tid % O, pt = tid / O;
        float acc = 0.f;
        if (pt < parts) {
            const int g = o / HD, d = o - g * HD;
            const float* e = sc + g * S;
            for (int p = pt; p < n; p += parts)
                acc = fmaf(e[p], (float)tv[(size_t)p * HDP + d], acc);
        }
        red[tid] = acc;
        __syncthreads();
        if (tid < O) {
            float v = 0.f;
            for (int k = 0; k < parts; ++k) v += red[tid + k * O];
            finish(tid, v);
        }
    }
}

// Lane-per-position form, for one query head per KV head (no grouped heads to share a staged
// K/V tile): LPP = HD/8 lanes hold one position's 16-byte K/V pieces (one coalesced HD*2-byte
// row per position); every K and V row of the split is loaded before the first use; scores go
// through LDS for the softmax; P.V accumulates per lane and reduces across lanes and waves.
// Same partials and ROPE behaviour as attn_lds_kernel.
// KT: the cache element (fp16, or fp32 for the fp32 K/V cache; fp32 splits hold at most 128
// positions, kAttnMaxS32, to keep the split's rows in registers).
constexpr int kAttnMaxS32 = 128;
template <int HD, int GW, bool ROPE, typename KT = _Float16>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(
    const float* __restrict__ q, const KT* __restrict__ kc, const KT* __restrict__ vc,
    const int* __restrict__ lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
    float* __restrict__ part, float* __restrict__ out, int nsplit, RopeArgs ra) {
    constexpr int LPP = HD / 8;          // lanes per position
    constexpr int NG = kThreads / LPP;   // positions in flight per pass
    constexpr int GPW = 64 / LPP;        // position groups per wave
    __shared__ float sc[GW][256];
    __shared__ float stat[GW][2];
    __shared__ float red[kThreads / 64][GW][HD];
    const int G = Hq / Hkv;
    const size_t npart = (size_t)(gridDim.x / Hkv) * Hq * nsplit;  // partials in the workspace
    const int b = blockIdx.x / Hkv, kvh = blockIdx.x % Hkv;
    const int s = blockIdx.y;
    const int h0 = kvh * G + blockIdx.z * GW;
    const int nh = min(GW, G - (int)blockIdx.z * GW);
    // a length beyond the cache capacity is clamped to it (no K/V row past T is read or written)
    const int L = min(max(lens ? lens[b] : len_host, 0), T);
    const int p0 = s * S, p1 = min(L, p0 + S);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lg = tid / LPP, li = tid % LPP;
    const bool direct = (nsplit == 1 && out != nullptr);
    if (p0 >= p1) {  // empty split (the length is below this split's range)
        for (int g = 0; g < nh; ++g) {
            const int bh = b * Hq + h0 + g;
            const size_t pi = (size_t)bh * nsplit + s;
            float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
            float* pst = part + 2 * pi;              // its (max, sum)
            if (!direct) {
                if (tid == 0) {
                    pst[0] = -INFINITY;
                    pst[1] = 0.f;
                }
                for (int i = tid; i < HD; i += kThreads) pp[i] = 0.f;
            } else {
                for (int i = tid; i < HD; i += kThreads) out[(size_t)bh * HD + i] = 0.f;
            }
        }
        return;
    }
    // Loads, in the order they are used: the query rows and the new K/V row, then every K row
    // of this lane's positions, then every V row (one memory round trip for the split). All are
    // issued unconditionally (heads past the group and positions past the split repeat the last
    // one), so the compiler's waits count exactly: the RoPE waits for the first loads only, the
    // scores for each K row as it arrives, and the softmax runs while the V rows stream in.
    float qv[GW][8];
#pragma unroll
    for (int g = 0; g < GW; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            qv[g][i] = q[((size_t)b * Hq + h0 + min(g, nh - 1)) * HD + li * 8 + i];
    float kn[8], vn[8];
    if constexpr (ROPE) {
        const float* knp = ra.knew + ((size_t)b * Hkv + kvh) * HD + li * 8;
        const float* vnp = ra.vnew + ((size_t)b * Hkv + kvh) * HD + li * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            kn[i] = knp[i];
            vn[i] = vnp[i];
        }
    }
    // (the scheduling barriers keep the three groups of loads in this order)
    __builtin_amdgcn_sched_barrier(0);
    const size_t rstride = (size_t)Hkv * HD;
    const KT* kb = kc + ((size_t)b * T * Hkv + kvh) * HD + li * 8;
    const KT* vb = vc + ((size_t)b * T * Hkv + kvh) * HD + li * 8;
    constexpr int kMaxPass = (sizeof(KT) == 4 ? kAttnMaxS32 : kAttnMaxS) / NG;
    const int npass = (p1 - p0 + NG - 1) / NG;
    Row8<KT> kr[kMaxPass], vr[kMaxPass];
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j)
        kr[j] = Row8<KT>::load(kb + (size_t)min(p0 + lg + j * NG, p1 - 1) * rstride);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j)
        vr[j] = Row8<KT>::load(vb + (size_t)min(p0 + lg + j * NG, p1 - 1) * rstride);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < GW; ++g)
        if (g >= nh)
#pragma unroll
            for (int i = 0; i < 8; ++i) qv[g][i] = 0.f;
    const int plast = L - 1;
    Row8<KT> knew{}, vnew{};
    if constexpr (ROPE) {
        // rotate this lane's 8 query dims of every head, and the new key, at position L - 1;
        // each pair's (cos, sin) evaluated once per workgroup (the lanes of a position group
        // share dims) while the K/V loads are in flight
        __shared__ float2 cs[HD / 2];
        for (int i = tid; i < HD / 2; i += kThreads) {
            const float freq = powf(ra.theta, -((float)(2 * i) / (float)HD));
            const float ang = (float)plast * freq;
            cs[i] = make_float2(cosf(ang), sinf(ang));
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const float2 csv = cs[(li * 8 + i) / 2];
            const float c = csv.x, sn = csv.y;
#pragma unroll
            for (int g = 0; g < GW; ++g) {
                const float x0 = qv[g][i], x1 = qv[g][i + 1];
                qv[g][i] = fmaf(x0, c, -(x1 * sn));
                qv[g][i + 1] = fmaf(x0, sn, x1 * c);
            }
            const float k0 = kn[i], k1 = kn[i + 1];
            knew.set(i, fmaf(k0, c, -(k1 * sn)));
            knew.set(i + 1, fmaf(k0, sn, k1 * c));
            vnew.set(i, vn[i]);
            vnew.set(i + 1, vn[i + 1]);
        }
        if (blockIdx.z == 0 && plast >= p0 && plast < p1 && lg == (plast - p0) % NG) {
            knew.store(cache_w<KT>(ra, false) + ((size_t)b * T + plast) * rstride + kvh * HD +
                       li * 8);
            vnew.store(cache_w<KT>(ra, true) + ((size_t)b * T + plast) * rstride + kvh * HD +
                       li * 8);
        }
    }
    // scores
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
        const int p = p0 + lg + j * NG;
        if (j >= npass || p >= p1) continue;
        const Row8<KT> kv = (ROPE && p == plast) ? knew : kr[j];
#pragma unroll
        for (int g = 0; g < GW; ++g) {
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(qv[g][i], kv.get(i), d);
#pragma unroll
            for (int off = LPP / 2; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
            if (li == 0 && g < nh) sc[g][p - p0] = d * scale;
        }
    }
    __syncthreads();
    // softmax statistics per head (wave w handles heads w, w + 4, ...)
    const int n = p1 - p0;
    for (int g = wave; g < nh; g += kThreads / 64) {
        float m = -INFINITY;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, sc[g][j]);
        m = wave_max(m);
        float l = 0.f;
        for (int j = lane; j < n; j += 64) {
            const float e = expf(sc[g][j] - m);
            sc[g][j] = e;
            l += e;
        }
        l = csdr::wave_sum(l);
        if (lane == 0) {
            stat[g][0] = m;
            stat[g][1] = l;
        }
    }
    __syncthreads();
    // P.V: this lane's 8 dims over its positions, then across position groups
    float o[GW][8];
#pragma unroll
    for (int g = 0; g < GW; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
        const int p = p0 + lg + j * NG;
        if (j >= npass || p >= p1) continue;
        const Row8<KT> vv = (ROPE && p == plast) ? vnew : vr[j];
#pragma unroll
        for (int g = 0; g < GW; ++g) {
            const float e = sc[g][p - p0];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[g][i] = fmaf(e, vv.get(i), o[g][i]);
        }
    }
#pragma unroll
    for (int g = 0; g < GW; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = o[g][i];
#pragma unroll
            for (int off = LPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
            o[g][i] = v;
        }
    (void)GPW;
    if (lane < LPP) {
#pragma unroll
        for (int g = 0; g < GW; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) red[wave][g][li * 8 + i] = o[g][i];
    }
    __syncthreads();
    for (int e = tid; e < nh * HD; e += kThreads) {
        const int g = e / HD, d = e % HD;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) sum += red[w][g][d];
        const int bh = b * Hq + h0 + g;
        if (direct) {
            out[(size_t)bh * HD + d] = sum / stat[g][1];
        } else {
            const size_t pi = (size_t)bh * nsplit + s;
            float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
            float* pst = part + 2 * pi;              // its (max, sum)
            pp[d] = sum;
            if (d == 0) {
                pst[0] = stat[g][0];
                pst[1] = stat[g][1];
            }
        }
    }
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Grouped-query decode attention on the matrix cores, for 2..16 query heads per KV head: one
// workgroup of 16 waves per (batch entry, KV head, split of up to 256 positions). The splits
// spread the K/V reads over many CUs: one workgroup per KV head holding 640 positions (cfg4)
// measured 13.9 us against 5.9 us for 128-position splits, its loads limited by what one CU
// keeps in flight.
//  * loads: each wave's K rows go straight from memory into v_mfma_f32_16x16x16f16 B operands
//    (lane: position tile * 16 + lane % 16, dims [lane / 16 * HD / 4, + HD / 4); the
//    contraction runs over the dims in that order and the query operand is read in the same
//    order); V rows are staged in LDS; every load is issued before the first wait;
//  * scores (q * scale) K^T: q rotated (ROPE) and scaled in fp32, then split into fp16 hi + lo
//    (two MFMAs per 16 dims, fp32 accumulate: the fp32 product to about 2^-22);
//  * softmax per head, one wave per head, in LDS;
//  * O = P V: P split into hi + lo, V read from LDS four positions per lane; the 16 waves are
//    (HD / 16 dim tiles) x (position groups), and the groups are summed through LDS.
constexpr int kMW = 16;  // waves per workgroup
constexpr int kMThreads = kMW * 64;
constexpr int kAttnMfmaMaxG = 16;  // query heads per KV head: the rows of one MFMA tile

constexpr size_t attn_mfma_lds_bytes(int HD, int G, int S) {
    return (size_t)S * (HD + 8) * 2 + (size_t)2 * 16 * HD * 2 + (size_t)HD * 2 +
           (size_t)G * S * 4 + 16 * 2 * 4 + (size_t)(kMW / (HD / 16) - 1) * (HD / 16) * 64 * 16;
}

template <int HD, bool ROPE>
__global__ __launch_bounds__(kMThreads) void attn_mfma_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ kc, const _Float16* __restrict__ vc,
    const int* __restrict__ lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
    float* __restrict__ part, float* __restrict__ out, int nsplit, RopeArgs ra) {
    constexpr int SMAX = kAttnMaxS;
    constexpr int HDP = HD + 8;                      // padded V row, halves
    constexpr int NDT = HD / 16;                     // 16-dim output tiles
    constexpr int NPG = kMW / NDT;                   // position groups of P.V
    constexpr int DPL = HD / 4;                      // dims per lane group in the score operands
    constexpr int KPL = DPL / 8;                     // 16-byte K pieces per lane and tile
    constexpr int TW = (SMAX / 16 + kMW - 1) / kMW;  // position tiles per wave, at most
    constexpr int PPR = HD / 8;                      // 16-byte pieces per row
    constexpr int VPT = SMAX * PPR / kMThreads;      // V pieces per thread, at most
    static_assert(VPT * kMThreads == SMAX * PPR, "V pieces must divide evenly");
    extern __shared__ float smem[];
    const int G = Hq / Hkv;
    const size_t npart = (size_t)(gridDim.x / Hkv) * Hq * nsplit;  // partials in the workspace
    const int b = blockIdx.x / Hkv, kvh = blockIdx.x % Hkv, s = blockIdx.y;
    const int h0 = kvh * G;
    // a length beyond the cache capacity is clamped to it (no K/V row past T is read or written)
    const int L = min(max(lens ? lens[b] : len_host, 0), T);
    const int p0 = s * S, p1 = min(L, p0 + S);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c16 = lane & 15, g4 = lane >> 4;
    const bool direct = (nsplit == 1 && out != nullptr);
    if (p0 >= p1) {  // empty split (the length is below this split's range)
        for (int e = tid; e < G * HD; e += kMThreads) {
            const int g = e / HD, d = e - g * HD;
            const int bh = b * Hq + h0 + g;
            if (direct) {
                out[(size_t)bh * HD + d] = 0.f;
            } else {
                const size_t pi = (size_t)bh * nsplit + s;
                float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
                float* pst = part + 2 * pi;              // its (max, sum)
                pp[d] = 0.f;
                if (d == 0) {
                    pst[0] = -INFINITY;
                    pst[1] = 0.f;
                }
            }
        }
        return;
    }
    const int n = p1 - p0, n16 = (n + 15) & ~15;
    const int plast = L - 1;
    const size_t rstride = (size_t)Hkv * HD;
    const _Float16* kb = kc + ((size_t)b * T * Hkv + kvh) * HD;
    const _Float16* vb = vc + ((size_t)b * T * Hkv + kvh) * HD;
    _Float16* tv = reinterpret_cast<_Float16*>(smem);     // S x HDP
    _Float16* qh = tv + (size_t)S * HDP;                   // 16 x HD: q hi
    _Float16* ql = qh + 16 * HD;                           // 16 x HD: q lo
    _Float16* kn = ql + 16 * HD;                           // HD: the new key (ROPE)
    float* sc = reinterpret_cast<float*>(kn + HD);         // G x S: scores, then P
    float* stat = sc + (size_t)G * S;                      // 16 x (max, sum)
    floatx4* red = reinterpret_cast<floatx4*>(stat + 32);  // (NPG - 1) x NDT x 64

    // 1. loads. Rows past the split's n positions are clamped (their scores are masked).
    h8 kr[TW][KPL];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int tile = wave + t * kMW;
        if (tile * 16 < n) {
            const int p = min(tile * 16 + c16, n - 1);
            const _Float16* src = kb + (size_t)(p0 + p) * rstride + g4 * DPL;
#pragma unroll
            for (int j = 0; j < KPL; ++j) kr[t][j] = *reinterpret_cast<const h8*>(src + j * 8);
        }
    }
    h8 vr[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int idx = tid + k * kMThreads, p = idx / PPR, j = idx - p * PPR;
        if (p < n) vr[k] = *reinterpret_cast<const h8*>(vb + (size_t)(p0 + p) * rstride + j * 8);
    }
    // the query heads, rotated at L - 1 and scaled, as fp16 hi + lo
    for (int e = tid; e < G * (HD / 2); e += kMThreads) {
        const int g = e / (HD / 2), i2 = 2 * (e - g * (HD / 2));
        const float* qp = q + ((size_t)b * Hq + h0 + g) * HD;
        float x0 = qp[i2], x1 = qp[i2 + 1];
        if constexpr (ROPE) {
            const float freq = powf(ra.theta, -((float)i2 / (float)HD));
            const float ang = (float)plast * freq;
            const float c = cosf(ang), sn = sinf(ang);
            const float r0 = fmaf(x0, c, -(x1 * sn)), r1 = fmaf(x0, sn, x1 * c);
            x0 = r0;
            x1 = r1;
        }
        x0 *= scale;
        x1 *= scale;
        const _Float16 a0 = (_Float16)x0, a1 = (_Float16)x1;
        qh[g * HD + i2] = a0;
        qh[g * HD + i2 + 1] = a1;
        ql[g * HD + i2] = (_Float16)(x0 - (float)a0);
        ql[g * HD + i2 + 1] = (_Float16)(x1 - (float)a1);
    }
    // V rows into LDS, zeros on [n, n16) (P is zero there; the rows must be finite). With ROPE
    // the row of position L - 1 is written below, from the new value, and by no other thread.
    const h8 zero8 = {};
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int idx = tid + k * kMThreads, p = idx / PPR, j = idx - p * PPR;
        if (p < n16 && !(ROPE && p0 + p == plast))
            *reinterpret_cast<h8*>(tv + (size_t)p * HDP + j * 8) = p < n ? vr[k] : zero8;
    }
    if constexpr (ROPE) {
        // position L - 1: the new key (rotated) and value, rounded to fp16, into LDS and, from
        // the split that holds it, appended to the caches
        if (plast >= p0 && plast < p1 && tid < HD / 2) {
            const int i2 = 2 * tid;
            const float* knp = ra.knew + ((size_t)b * Hkv + kvh) * HD;
            const float* vnp = ra.vnew + ((size_t)b * Hkv + kvh) * HD;
            const float freq = powf(ra.theta, -((float)i2 / (float)HD));
            const float ang = (float)plast * freq;
            const float c = cosf(ang), sn = sinf(ang);
            const float k0 = knp[i2], k1 = knp[i2 + 1];
            const _Float16 a0 = (_Float16)fmaf(k0, c, -(k1 * sn));
            const _Float16 a1 = (_Float16)fmaf(k0, sn, k1 * c);
            const _Float16 w0 = (_Float16)vnp[i2], w1 = (_Float16)vnp[i2 + 1];
            const int pr = plast - p0;
            kn[i2] = a0;
            kn[i2 + 1] = a1;
            tv[(size_t)pr * HDP + i2] = w0;
            tv[(size_t)pr * HDP + i2 + 1] = w1;
            const size_t at = ((size_t)b * T + plast) * rstride + (size_t)kvh * HD + i2;
            ra.kcw[at] = a0;
            ra.kcw[at + 1] = a1;
            ra.vcw[at] = w0;
            ra.vcw[at + 1] = w1;
        }
    }
    __syncthreads();

    // 2. scores: wave w takes position tiles w, w + 16, ...; A rows past G repeat head G - 1
    const int hr = min(c16, G - 1);
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int tile = wave + t * kMW;
        if (tile * 16 >= n) break;
        const int p = tile * 16 + c16;
        if constexpr (ROPE) {
            if (p0 + p == plast) {
#pragma unroll
                for (int j = 0; j < KPL; ++j)
                    kr[t][j] = *reinterpret_cast<const h8*>(kn + g4 * DPL + j * 8);
            }
        }
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
            const h8 kv = kr[t][ks / 2];
            const half4 bk = (ks & 1) ? __builtin_shufflevector(kv, kv, 4, 5, 6, 7)
                                      : __builtin_shufflevector(kv, kv, 0, 1, 2, 3);
            const int qo = hr * HD + g4 * DPL + ks * 4;
            const half4 ah = *reinterpret_cast<const half4*>(qh + qo);
            const half4 al = *reinterpret_cast<const half4*>(ql + qo);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bk, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bk, acc, 0, 0, 0);
        }
        // lane holds heads 4 (lane / 16) + i at position p
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = g4 * 4 + i;
            if (h < G) sc[h * S + p] = p < n ? acc[i] : -INFINITY;
        }
    }
    __syncthreads();

    // 3. softmax statistics, wave h for head h; P = exp(s - max) in place, zero on [n, n16)
    if (wave < G) {
        float* row = sc + wave * S;
        float m = -INFINITY;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, row[j]);
        m = wave_max(m);
        float l = 0.f;
        for (int j = lane; j < n16; j += 64) {
            const float e = j < n ? expf(row[j] - m) : 0.f;
            row[j] = e;
            l += e;
        }
        l = csdr::wave_sum(l);
        if (lane == 0) {
            stat[wave * 2] = m;
            stat[wave * 2 + 1] = l;
        }
    }
    __syncthreads();

    // 4. O = P V: wave = (dim tile dt, position group pg), 16 positions per step
    const int dt = wave % NDT, pg = wave / NDT;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
    for (int kt = pg; kt * 16 < n16; kt += NPG) {
        const float4 pv = *reinterpret_cast<const float4*>(sc + hr * S + kt * 16 + g4 * 4);
        half4 ph, pl;
        ph[0] = (_Float16)pv.x;
        ph[1] = (_Float16)pv.y;
        ph[2] = (_Float16)pv.z;
        ph[3] = (_Float16)pv.w;
        pl[0] = (_Float16)(pv.x - (float)ph[0]);
        pl[1] = (_Float16)(pv.y - (float)ph[1]);
        pl[2] = (_Float16)(pv.z - (float)ph[2]);
        pl[3] = (_Float16)(pv.w - (float)ph[3]);
        const _Float16* vp = tv + (size_t)(kt * 16 + g4 * 4) * HDP + dt * 16 + c16;
        half4 bv;
        bv[0] = vp[0];
        bv[1] = vp[HDP];
        bv[2] = vp[2 * HDP];
        bv[3] = vp[3 * HDP];
        o = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, bv, o, 0, 0, 0);
        o = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, bv, o, 0, 0, 0);
    }
    if (pg > 0) red[((pg - 1) * NDT + dt) * 64 + lane] = o;
    __syncthreads();
    if (pg == 0) {
#pragma unroll
        for (int k = 1; k < NPG; ++k) o += red[((k - 1) * NDT + dt) * 64 + lane];
        const int d = dt * 16 + c16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = g4 * 4 + i;
            if (h >= G) continue;
            const int bh = b * Hq + h0 + h;
            if (direct) {
                out[(size_t)bh * HD + d] = o[i] / stat[h * 2 + 1];
            } else {
                const size_t pi = (size_t)bh * nsplit + s;
                float* pp = part + attn_vec_offset(npart) + pi * HD;  // the partial's vector
                float* pst = part + 2 * pi;              // its (max, sum)
                pp[d] = o[i];
                if (d == 0) {
                    pst[0] = stat[h * 2];
                    pst[1] = stat[h * 2 + 1];
                }
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ part,
                                                          int nsplit, float* __restrict__ out) {
    const int bh = blockIdx.x;
    const size_t npart = (size_t)gridDim.x * nsplit;
    const float* pst = part + (size_t)2 * bh * nsplit;             // (max, sum) per split
    const float* pv = part + attn_vec_offset(npart) + (size_t)bh * nsplit * HD;  // per split
    // rounds of kR splits, every load of a round issued at once (indices clamped, entries past
    // the last split or of empty splits weighted 0): loads under a per-split branch ran one
    // round trip at a time
    constexpr int kR = 16;
    float M = -INFINITY;
    for (int s0 = 0; s0 < nsplit; s0 += kR) {
        float mv[kR];
#pragma unroll
        for (int j = 0; j < kR; ++j) mv[j] = pst[2 * min(s0 + j, nsplit - 1)];
#pragma unroll
        for (int j = 0; j < kR; ++j) M = fmaxf(M, mv[j]);
    }
    float num = 0.f, den = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += kR) {
        float ms[kR], ls[kR], vv[kR];
#pragma unroll
        for (int j = 0; j < kR; ++j) {
            const int sj = min(s0 + j, nsplit - 1);
            ms[j] = pst[2 * sj];
            ls[j] = pst[2 * sj + 1];
            vv[j] = pv[(size_t)sj * HD + threadIdx.x];
        }
#pragma unroll
        for (int j = 0; j < kR; ++j) {
            const bool live = s0 + j < nsplit && ms[j] != -INFINITY;
            const float w = live ? expf(ms[j] - M) : 0.f;
            den = fmaf(w, live ? ls[j] : 0.f, den);
            num = fmaf(w, live ? vv[j] : 0.f, num);
        }
    }
    out[(size_t)bh * HD + threadIdx.x] = den > 0.f ? num / den : 0.f;
}

// ---------------------------------------------------------------- token selection

// score = logit * ts (- penalty when repeated[i]); the best finite score wins, lowest index
// on ties. Stage 1: one (score, index) per workgroup; stage 2: one workgroup over those.
__device__ __forceinline__ void better(float& bs, int& bi, float s, int i) {
    if (s > bs || (s == bs && i < bi && i >= 0)) {
        bs = s;
        bi = i;
    }
}

// Row blockIdx.y of `rows` rows of n scores (one per sequence of a batch): logits, repeated
// and the workspace pairs are offset by the row.
__global__ __launch_bounds__(kThreads) void select1_kernel(const float* __restrict__ logits, int n,
                                                           const uint8_t* __restrict__ repeated,
                                                           float ts, float penalty,
                                                           float* __restrict__ ws_s,
                                                           int* __restrict__ ws_i) {
    logits += (size_t)blockIdx.y * n;
    if (repeated) repeated += (size_t)blockIdx.y * n;
    ws_s += (size_t)blockIdx.y * gridDim.x;
    ws_i += (size_t)blockIdx.y * gridDim.x;
    __shared__ float ss[kThreads];
    __shared__ int si[kThreads];
    float bs = -INFINITY;
    int bi = -1;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        float s = logits[i] * ts;
        if (!isfinite(s)) continue;
        if (repeated && repeated[i]) s -= penalty;
        if (bi < 0 || s > bs) {
            bs = s;
            bi = i;
        }
    }
    ss[threadIdx.x] = bs;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) {
            float s2 = ss[threadIdx.x + off];
            int i2 = si[threadIdx.x + off];
            if (i2 >= 0 && (si[threadIdx.x] < 0 || s2 > ss[threadIdx.x] ||
                            (s2 == ss[threadIdx.x] && i2 < si[threadIdx.x]))) {
                ss[threadIdx.x] = s2;
                si[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ws_s[blockIdx.x] = ss[0];
        ws_i[blockIdx.x] = si[0];
    }
}

// Row blockIdx.x: its nb stage-1 pairs, its token out[row], its generated-token set; the
// position advances once (row 0).
__global__ __launch_bounds__(kThreads) void select2_kernel(const float* __restrict__ ws_s,
                                                           const int* __restrict__ ws_i, int nb,
                                                           int* __restrict__ out,
                                                           int* __restrict__ pos_dev,
                                                           uint8_t* __restrict__ repeated, int n) {
    const int row = blockIdx.x;
    ws_s += (size_t)row * nb;
    ws_i += (size_t)row * nb;
    out += row;
    if (repeated) repeated += (size_t)row * n;
    __shared__ float ss[kThreads];
    __shared__ int si[kThreads];
    float bs = -INFINITY;
    int bi = -1;
    for (int i = threadIdx.x; i < nb; i += kThreads) {
        const float s = ws_s[i];
        const int ix = ws_i[i];
        if (ix >= 0 && (bi < 0 || s > bs || (s == bs && ix < bi))) {
            bs = s;
            bi = ix;
        }
    }
    ss[threadIdx.x] = bs;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) {
            float s2 = ss[threadIdx.x + off];
            int i2 = si[threadIdx.x + off];
            if (i2 >= 0 && (si[threadIdx.x] < 0 || s2 > ss[threadIdx.x] ||
                            (s2 == ss[threadIdx.x] && i2 < si[threadIdx.x]))) {
                ss[threadIdx.x] = s2;
                si[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        *out = si[0];
        if (pos_dev && row == 0) *pos_dev += 1;           // next decode position
        if (repeated && si[0] >= 0) repeated[si[0]] = 1;  // generated-token set
    }
}

constexpr int kSelectBlocks = 256;

// Positions per split: about T / 8 rounded up to a power of two in [64, 256], so a head has at
// most 8 splits up to 2048 positions (every split's K/V rows are loaded in one round trip, and
// the consumer's combine reads nsplit partials per feature; measured on cfg4, 640 positions:
// 128 ahead of 64 and 256).
int attn_split_len(int B, int Hkv, int zsplit, int T) {
    (void)B;
    (void)Hkv;
    (void)zsplit;
    int S = 64;
    while (S < 256 && 8LL * S < T) S *= 2;
    return S;
}

// Dynamic LDS above 64 KiB: a kernel's limit is raised once, to its largest shape (one
// instantiation per kernel: KIND tells the kernels of one HD and ROPE apart).
template <int KIND, int HD, bool ROPE>
void raise_lds_once(const void* fn, size_t bytes) {
    static const bool raised = [&] {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        return true;
    }();
    (void)raised;
}

// Whether grouped-query shapes take attn_mfma_kernel (CSDR_ATTN_MFMA=0 keeps the VALU kernels).
bool attn_mfma_enabled() {
    const char* e = std::getenv("CSDR_ATTN_MFMA");
    return !(e && e[0] == '0');
}

template <int HD, bool ROPE>
void launch_attn_mfma(dim3 grid, int G, const float* q, const _Float16* k16, const _Float16* v16,
                      const int* lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
                      float* part, float* out, int nsplit, const RopeArgs& ra, hipStream_t st) {
    raise_lds_once<0, HD, ROPE>(reinterpret_cast<const void*>(&attn_mfma_kernel<HD, ROPE>),
                   attn_mfma_lds_bytes(HD, kAttnMfmaMaxG, kAttnMaxS));
    attn_mfma_kernel<HD, ROPE><<<grid, kMThreads, attn_mfma_lds_bytes(HD, G, S), st>>>(
        q, k16, v16, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
}

template <int HD, bool ROPE>
void launch_attn(dim3 grid, int G, bool mfma, const float* q, const _Float16* k16,
                 const _Float16* v16, const int* lens, int len_host, int T, int Hq, int Hkv,
                 float scale, int S, float* part, float* out, int nsplit, const RopeArgs& ra,
                 hipStream_t st) {
    if (mfma) {
        launch_attn_mfma<HD, ROPE>(grid, G, q, k16, v16, lens, len_host, T, Hq, Hkv, scale, S,
                                   part, out, nsplit, ra, st);
        return;
    }
    // one query head per KV head: the lane-per-position kernel (measured at Llama-7B shape,
    // head_dim 128, 4096 positions: 20.5 vs 29.1 us; its small LDS footprint keeps several
    // workgroups per CU where the staged tile would allow one)
    if (G == 1)
        attn_split_kernel<HD, 1, ROPE><<<grid, kThreads, 0, st>>>(
            q, k16, v16, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
    else if (G <= 4) {
        raise_lds_once<1, HD, ROPE>(reinterpret_cast<const void*>(&attn_lds_kernel<HD, 4, ROPE>),
                                    attn_lds_bytes(HD, 4, kAttnMaxS));
        attn_lds_kernel<HD, 4, ROPE><<<grid, kThreads, attn_lds_bytes(HD, 4, S), st>>>(
            q, k16, v16, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
    } else {
        raise_lds_once<2, HD, ROPE>(reinterpret_cast<const void*>(&attn_lds_kernel<HD, 8, ROPE>),
                                    attn_lds_bytes(HD, 8, kAttnMaxS));
        attn_lds_kernel<HD, 8, ROPE><<<grid, kThreads, attn_lds_bytes(HD, 8, S), st>>>(
            q, k16, v16, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
    }
}

struct AttnShape {
    int G, GW, zsplit, S, nsplit;
    bool mfma;
};

AttnShape attn_shape(int B, int Hq, int Hkv, int hd, int T, bool kv32 = false) {
    AttnShape a;
    a.G = Hq / Hkv;
    if (kv32) {
        // fp32 cache: the lane-per-position kernel, up to 4 query heads per pass, splits of at
        // most kAttnMaxS32 positions
        a.mfma = false;
        a.GW = a.G == 1 ? 1 : 4;
        a.zsplit = (a.G + a.GW - 1) / a.GW;
        a.S = std::min(attn_split_len(B, Hkv, a.zsplit, T), kAttnMaxS32);
        // fewer than 256 workgroups at that length: 64-position splits (cfg4, 2 KV heads x 640
        // positions: 20 workgroups; 771 -> 784 decode tokens/s; 32 positions: 751)
        if ((long long)B * Hkv * a.zsplit * ((T + a.S - 1) / a.S) < 256) a.S = std::min(a.S, 64);
        a.nsplit = (T + a.S - 1) / a.S;
        return a;
    }
    a.mfma = a.G >= 2 && a.G <= kAttnMfmaMaxG && (hd == 64 || hd == 128) && attn_mfma_enabled();
    if (a.mfma) {
        a.GW = a.G;
        a.zsplit = 1;
        a.S = attn_split_len(B, Hkv, 1, T);
        a.nsplit = (T + a.S - 1) / a.S;
        return a;
    }
    a.GW = a.G == 1 ? 1 : (a.G <= 4 ? 4 : 8);
    a.zsplit = (a.G + a.GW - 1) / a.GW;
    a.S = attn_split_len(B, Hkv, a.zsplit, T);
    a.nsplit = (T + a.S - 1) / a.S;
    return a;
}

template <int HD, bool ROPE>
void launch_attn32(dim3 grid, int G, const float* q, const float* k32, const float* v32,
                   const int* lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
                   float* part, float* out, int nsplit, const RopeArgs& ra, hipStream_t st) {
    if (G == 1)
        attn_split_kernel<HD, 1, ROPE, float><<<grid, kThreads, 0, st>>>(
            q, k32, v32, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
    else
        attn_split_kernel<HD, 4, ROPE, float><<<grid, kThreads, 0, st>>>(
            q, k32, v32, lens, len_host, T, Hq, Hkv, scale, S, part, out, nsplit, ra);
}

int attn_run(const float* q, const void* kcache, const void* vcache, const int* lens_dev,
             int len_host, int B, int T, int Hq, int Hkv, int hd, float scale, float* out,
             void* workspace, size_t workspace_bytes, const RopeArgs* ra, hipStream_t st,
             bool kv32 = false) {
    const AttnShape sh = attn_shape(B, Hq, Hkv, hd, T, kv32);
    const bool partials = sh.nsplit > 1 || out == nullptr;
    if (partials &&
        (!workspace || workspace_bytes < csdr_attn_decode_workspace_bytes(B, Hq, hd, T)))
        return set_error(CSDR_E_WORKSPACE, "attn_decode: workspace too small");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)hd);
    float* part = static_cast<float*>(workspace);
    dim3 grid(B * Hkv, sh.nsplit, sh.zsplit);
    auto k16 = static_cast<const _Float16*>(kcache);
    auto v16 = static_cast<const _Float16*>(vcache);
    const RopeArgs none{};
    if (kv32) {
        auto k32 = static_cast<const float*>(kcache);
        auto v32 = static_cast<const float*>(vcache);
        if (hd == 64) {
            if (ra)
                launch_attn32<64, true>(grid, sh.G, q, k32, v32, lens_dev, len_host, T, Hq, Hkv,
                                        scale, sh.S, part, out, sh.nsplit, *ra, st);
            else
                launch_attn32<64, false>(grid, sh.G, q, k32, v32, lens_dev, len_host, T, Hq, Hkv,
                                         scale, sh.S, part, out, sh.nsplit, none, st);
            if (out && sh.nsplit > 1)
                attn_combine_kernel<64><<<B * Hq, 64, 0, st>>>(part, sh.nsplit, out);
        } else {
            if (ra)
                launch_attn32<128, true>(grid, sh.G, q, k32, v32, lens_dev, len_host, T, Hq, Hkv,
                                         scale, sh.S, part, out, sh.nsplit, *ra, st);
            else
                launch_attn32<128, false>(grid, sh.G, q, k32, v32, lens_dev, len_host, T, Hq,
                                          Hkv, scale, sh.S, part, out, sh.nsplit, none, st);
            if (out && sh.nsplit > 1)
                attn_combine_kernel<128><<<B * Hq, 128, 0, st>>>(part, sh.nsplit, out);
        }
        CSDR_LAUNCH_CHECK("attn_decode");
        return CSDR_OK;
    }
    if (hd == 64) {
        if (ra)
            launch_attn<64, true>(grid, sh.G, sh.mfma, q, k16, v16, lens_dev, len_host, T, Hq,
                                  Hkv, scale, sh.S, part, out, sh.nsplit, *ra, st);
        else
            launch_attn<64, false>(grid, sh.G, sh.mfma, q, k16, v16, lens_dev, len_host, T, Hq,
                                   Hkv, scale, sh.S, part, out, sh.nsplit, none, st);
        if (out && sh.nsplit > 1)
            attn_combine_kernel<64><<<B * Hq, 64, 0, st>>>(part, sh.nsplit, out);
    } else {
        if (ra)
            launch_attn<128, true>(grid, sh.G, sh.mfma, q, k16, v16, lens_dev, len_host, T, Hq,
                                   Hkv, scale, sh.S, part, out, sh.nsplit, *ra, st);
        else
            launch_attn<128, false>(grid, sh.G, sh.mfma, q, k16, v16, lens_dev, len_host, T, Hq,
                                    Hkv, scale, sh.S, part, out, sh.nsplit, none, st);
        if (out && sh.nsplit > 1)
            attn_combine_kernel<128><<<B * Hq, 128, 0, st>>>(part, sh.nsplit, out);
    }
    CSDR_LAUNCH_CHECK("attn_decode");
    return CSDR_OK;
}

}  // namespace

namespace csdr {

size_t select_workspace_rows(int rows) { return (size_t)kSelectBlocks * 8 * (size_t)rows; }

int select_best_rows(const float* logits, int n, int rows, const uint8_t* repeated,
                     float temperature, float penalty, int* out_tokens, int* pos_dev,
                     uint8_t* repeated_update, void* workspace, size_t workspace_bytes,
                     hipStream_t st) {
    if (!logits || n <= 0 || rows <= 0 || !out_tokens)
        return set_error(CSDR_E_INVALID, "select_best: bad argument");
    if (!workspace || workspace_bytes < select_workspace_rows(rows))
        return set_error(CSDR_E_WORKSPACE, "select_best: workspace too small");
    const float ts = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    const int nb = std::min(kSelectBlocks, (n + kThreads - 1) / kThreads);
    float* ws_s = static_cast<float*>(workspace);
    int* ws_i = reinterpret_cast<int*>(ws_s + (size_t)nb * rows);
    select1_kernel<<<dim3(nb, rows), kThreads, 0, st>>>(logits, n, repeated, ts, penalty, ws_s,
                                                        ws_i);
    select2_kernel<<<rows, kThreads, 0, st>>>(ws_s, ws_i, nb, out_tokens, pos_dev,
                                              repeated_update, n);
    CSDR_LAUNCH_CHECK("select_best");
    return CSDR_OK;
}

}  // namespace csdr

extern "C" {

CSDR_API int csdr_rms_norm(const float* x, const float* w, int ntok, int n, float eps, float* y,
                           void* hip_stream) {
    if (!x || !w || !y || ntok <= 0 || n <= 0)
        return set_error(CSDR_E_INVALID, "rms_norm: bad argument");
    const int nt = n > 2048 ? 1024 : 256;
    rms_norm_kernel<<<ntok, nt, 0, static_cast<hipStream_t>(hip_stream)>>>(x, w, n, eps, y);
    CSDR_LAUNCH_CHECK("rms_norm");
    return CSDR_OK;
}

CSDR_API int csdr_silu_mul(const float* g, const float* u, size_t n, float* y, void* hip_stream) {
    if (!g || !u || !y) return set_error(CSDR_E_INVALID, "silu_mul: bad argument");
    if (n == 0) return CSDR_OK;
    const int grid = (int)std::min<size_t>((n + kThreads - 1) / kThreads, 4096);
    silu_mul_kernel<<<grid, kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(g, u, n, y);
    CSDR_LAUNCH_CHECK("silu_mul");
    return CSDR_OK;
}

CSDR_API int csdr_rope_kv(float* q, float* k, const float* v, int ntok, int Hq, int Hkv, int hd,
                          const int* pos_dev, float theta, uint16_t* kcache, uint16_t* vcache,
                          int max_ctx, void* hip_stream) {
    if (!q || !k || !v || !pos_dev || !kcache || !vcache || ntok <= 0 || Hq <= 0 || Hkv <= 0 ||
        hd < 2 || Hq % Hkv)
        return set_error(CSDR_E_INVALID, "rope_kv: bad argument");
    rope_kv_kernel<<<ntok * (Hq + Hkv), 64, 0, static_cast<hipStream_t>(hip_stream)>>>(
        q, k, v, ntok, Hq, Hkv, hd, pos_dev, theta, reinterpret_cast<_Float16*>(kcache),
        reinterpret_cast<_Float16*>(vcache), max_ctx);
    CSDR_LAUNCH_CHECK("rope_kv");
    return CSDR_OK;
}

CSDR_API size_t csdr_attn_decode_workspace_bytes(int B, int Hq, int hd, int T) {
    const int nsplit = (T + 63) / 64;  // the shortest split bounds the count
    return (size_t)B * Hq * nsplit * (hd + 2) * 4 + 16;  // + the vectors' 16-byte alignment
}

CSDR_API int csdr_attn_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                              const int* lens_dev, int len_host, int B, int T, int Hq, int Hkv,
                              int hd, float scale, float* out, void* workspace,
                              size_t workspace_bytes, void* hip_stream) {
    if (!q || !kcache || !vcache || !out || B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 ||
        Hq % Hkv)
        return set_error(CSDR_E_INVALID, "attn_decode: bad argument");
    if (!lens_dev && (len_host < 0 || len_host > T))
        return set_error(CSDR_E_INVALID, "attn_decode: length out of range");
    if (hd != 64 && hd != 128)
        return set_error(CSDR_E_UNSUPPORTED, "attn_decode: head_dim must be 64 or 128");
    return attn_run(q, kcache, vcache, lens_dev, len_host, B, T, Hq, Hkv, hd, scale, out,
                    workspace, workspace_bytes, nullptr, static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_attn_decode_splits(int B, int Hq, int Hkv, int hd, int T) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0 || Hq % Hkv) return -1;
    return attn_shape(B, Hq, Hkv, hd, T).nsplit;
}

CSDR_API int csdr_attn_decode_rope(const float* q, const float* k_new, const float* v_new,
                                   uint16_t* kcache, uint16_t* vcache, const int* lens_dev, int B,
                                   int T, int Hq, int Hkv, int hd, float theta, float scale,
                                   float* out, void* workspace, size_t workspace_bytes,
                                   void* hip_stream) {
    if (!q || !k_new || !v_new || !kcache || !vcache || !lens_dev || B <= 0 || T <= 0 ||
        Hq <= 0 || Hkv <= 0 || Hq % Hkv)
        return set_error(CSDR_E_INVALID, "attn_decode_rope: bad argument");
    if (hd != 64 && hd != 128)
        return set_error(CSDR_E_UNSUPPORTED, "attn_decode_rope: head_dim must be 64 or 128");
    return csdr_attn_decode_rope_kv(q, k_new, v_new, kcache, vcache, CSDR_F16, lens_dev, B, T,
                                    Hq, Hkv, hd, theta, scale, out, workspace, workspace_bytes,
                                    hip_stream);
}

CSDR_API int csdr_attn_decode_rope_kv(const float* q, const float* k_new, const float* v_new,
                                      void* kcache, void* vcache, int kv_dtype,
                                      const int* lens_dev, int B, int T, int Hq, int Hkv, int hd,
                                      float theta, float scale, float* out, void* workspace,
                                      size_t workspace_bytes, void* hip_stream) {
    if (!q || !k_new || !v_new || !kcache || !vcache || !lens_dev || B <= 0 || T <= 0 ||
        Hq <= 0 || Hkv <= 0 || Hq % Hkv)
        return set_error(CSDR_E_INVALID, "attn_decode_rope: bad argument");
    if (hd != 64 && hd != 128)
        return set_error(CSDR_E_UNSUPPORTED, "attn_decode_rope: head_dim must be 64 or 128");
    if (kv_dtype != CSDR_F16 && kv_dtype != CSDR_F32)
        return set_error(CSDR_E_INVALID, "attn_decode_rope: kv_dtype must be CSDR_F16 or CSDR_F32");
    const bool kv32 = kv_dtype == CSDR_F32;
    RopeArgs ra{k_new, v_new, kv32 ? nullptr : static_cast<_Float16*>(kcache),
                kv32 ? nullptr : static_cast<_Float16*>(vcache), theta,
                kv32 ? static_cast<float*>(kcache) : nullptr,
                kv32 ? static_cast<float*>(vcache) : nullptr};
    return attn_run(q, kcache, vcache, lens_dev, 0, B, T, Hq, Hkv, hd, scale, out, workspace,
                    workspace_bytes, &ra, static_cast<hipStream_t>(hip_stream), kv32);
}

CSDR_API int csdr_attn_decode_splits_kv(int B, int Hq, int Hkv, int hd, int T, int kv_dtype) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0 || Hq % Hkv) return -1;
    return attn_shape(B, Hq, Hkv, hd, T, kv_dtype == CSDR_F32).nsplit;
}

CSDR_API size_t csdr_select_workspace_bytes(void) { return (size_t)kSelectBlocks * 8; }

CSDR_API int csdr_select_best(const float* logits, int n, const uint8_t* repeated,
                              float temperature, float penalty, int* out_token, int* pos_dev,
                              uint8_t* repeated_update, void* workspace, size_t workspace_bytes,
                              void* hip_stream) {
    return csdr::select_best_rows(logits, n, 1, repeated, temperature, penalty, out_token,
                                  pos_dev, repeated_update, workspace, workspace_bytes,
                                  static_cast<hipStream_t>(hip_stream));
}

}  // extern "C"
