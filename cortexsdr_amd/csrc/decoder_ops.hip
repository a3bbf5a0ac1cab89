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

#include <cmath>
#include <string>

#include "common.hpp"

namespace {

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

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w, int n,
                                                            float eps, float* __restrict__ y) {
    __shared__ float red[kThreads / 64];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kThreads) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) yr[i] = xr[i] * inv * w[i];
}

// ---------------------------------------------------------------- SiLU(g) * u

// Dense fp32 linear for uncoded (strategy 0) 2-D weights: one wave per output row, lanes
// stride over the input features, fp32 sums reduced across the wave.
__global__ __launch_bounds__(kThreads) void dense_linear_kernel(const float* __restrict__ W, int R,
                                                                int C, const float* __restrict__ x,
                                                                int M, float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (r >= R) return;
    const float* w = W + (size_t)r * C;
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (size_t)m * C;
        float acc = 0.0f;
        for (int c = lane; c < C; c += 64) acc = fmaf(w[c], xm[c], acc);
        acc = csdr::wave_sum(acc);
        if (lane == 0) y[(size_t)m * R + r] = acc;
    }
}

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
// out [position][kv head][hd] with row capacity max_ctx.
__global__ __launch_bounds__(kThreads) void rope_kv_kernel(float* __restrict__ q,
                                                           float* __restrict__ k,
                                                           const float* __restrict__ v, int ntok,
                                                           int Hq, int Hkv, int hd,
                                                           const int* __restrict__ pos_dev,
                                                           float theta, _Float16* kcache,
                                                           _Float16* vcache, int max_ctx) {
    const int t = blockIdx.x;
    const int pos = *pos_dev + t;
    const int half = hd / 2;
    const int rot = hd - (hd % 2);
    // pairs (2i, 2i+1) of every head: Hq heads of q, then Hkv heads of k
    for (int e = threadIdx.x; e < (Hq + Hkv) * half; e += kThreads) {
        const int head = e / half, i2 = 2 * (e % half);
        if (i2 >= rot) continue;
        float* base = head < Hq ? q + ((size_t)t * Hq + head) * hd
                                : k + ((size_t)t * Hkv + (head - Hq)) * hd;
        const float freq = powf(theta, -((float)i2 / (float)hd));
        const float ang = (float)pos * freq;
        const float c = cosf(ang), s = sinf(ang);
        const float x0 = base[i2], x1 = base[i2 + 1];
        base[i2] = x0 * c - x1 * s;
        base[i2 + 1] = x0 * s + x1 * c;
    }
    __syncthreads();
    if (pos >= max_ctx) return;
    for (int e = threadIdx.x; e < Hkv * hd; e += kThreads) {
        const size_t src = (size_t)t * Hkv * hd + e;
        const size_t dst = (size_t)pos * Hkv * hd + e;
        kcache[dst] = (_Float16)k[src];
        vcache[dst] = (_Float16)v[src];
    }
}

// ---------------------------------------------------------------- flash-decode attention

// Partial softmax-attention of one query head over positions [s*S, min(L, (s+1)*S)):
// part = (max score m, sum of exp l, o[hd] = sum exp * v). One thread per position for the
// scores; for P.V, thread t owns dimension t % hd and a 1/(256/hd) share of the positions.
template <int HD>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ kc, const _Float16* __restrict__ vc,
    const int* __restrict__ lens, int len_host, int T, int Hq, int Hkv, float scale, int S,
    float* __restrict__ part, float* __restrict__ out, int nsplit) {
    __shared__ float qs[HD];
    __shared__ float ps[kThreads];
    __shared__ float red[kThreads / 64];
    __shared__ float acc_s[kThreads];
    const int bh = blockIdx.x;  // batch * Hq + head
    const int b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const int s = blockIdx.y;
    const int L = lens ? lens[b] : len_host;
    const int p0 = s * S, p1 = min(L, p0 + S);
    for (int i = threadIdx.x; i < HD; i += kThreads) qs[i] = q[(size_t)bh * HD + i];
    __syncthreads();
    float* pp = part + ((size_t)bh * nsplit + s) * (HD + 2);
    if (p0 >= p1) {  // empty split (the length is below this split's range)
        if (nsplit > 1 && threadIdx.x == 0) {
            pp[0] = -INFINITY;
            pp[1] = 0.f;
        }
        if (nsplit > 1)
            for (int i = threadIdx.x; i < HD; i += kThreads) pp[2 + i] = 0.f;
        else
            for (int i = threadIdx.x; i < HD; i += kThreads) out[(size_t)bh * HD + i] = 0.f;
        return;
    }
    // scores: one position per thread (S <= kThreads)
    const int pos = p0 + threadIdx.x;
    float sc = -INFINITY;
    if (pos < p1) {
        // the key row: HD fp16 values as 16-byte vectors
        const h8* kr = reinterpret_cast<const h8*>(kc + (((size_t)b * T + pos) * Hkv + kvh) * HD);
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < HD / 8; ++j) {
            const h8 kv = kr[j];
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(qs[j * 8 + i], (float)kv[i], d);
        }
        sc = d * scale;
    }
    const float m = block_max(sc, red);
    const float e = (pos < p1) ? expf(sc - m) : 0.f;
    ps[threadIdx.x] = e;
    const float l = block_sum(e, red);
    // P.V: thread t -> dim t % HD, positions p0 + g, g = t / HD, t/HD + G, ...
    constexpr int G = kThreads / HD;
    const int dim = threadIdx.x % HD, grp = threadIdx.x / HD;
    float o = 0.f;
    for (int j = grp; j < p1 - p0; j += G)
        o = fmaf(ps[j], (float)vc[(((size_t)b * T + p0 + j) * Hkv + kvh) * HD + dim], o);
    acc_s[threadIdx.x] = o;
    __syncthreads();
    if (threadIdx.x < HD) {
        float sum = 0.f;
        for (int g2 = 0; g2 < G; ++g2) sum += acc_s[g2 * HD + threadIdx.x];
        if (nsplit == 1) {
            out[(size_t)bh * HD + threadIdx.x] = sum / l;
        } else {
            pp[2 + threadIdx.x] = sum;
            if (threadIdx.x == 0) {
                pp[0] = m;
                pp[1] = l;
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ part,
                                                          int nsplit, float* __restrict__ out) {
    const int bh = blockIdx.x;
    const float* pp = part + (size_t)bh * nsplit * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, pp[(size_t)s * (HD + 2)]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < nsplit; ++s) {
        const float ms = pp[(size_t)s * (HD + 2)];
        if (ms == -INFINITY) continue;
        const float w = expf(ms - M);
        den = fmaf(w, pp[(size_t)s * (HD + 2) + 1], den);
        num = fmaf(w, pp[(size_t)s * (HD + 2) + 2 + threadIdx.x], num);
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

__global__ __launch_bounds__(kThreads) void select1_kernel(const float* __restrict__ logits, int n,
                                                           const uint8_t* __restrict__ repeated,
                                                           float ts, float penalty,
                                                           float* __restrict__ ws_s,
                                                           int* __restrict__ ws_i) {
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

__global__ __launch_bounds__(kThreads) void select2_kernel(const float* __restrict__ ws_s,
                                                           const int* __restrict__ ws_i, int nb,
                                                           int* __restrict__ out,
                                                           int* __restrict__ pos_dev,
                                                           uint8_t* __restrict__ repeated) {
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
        if (pos_dev) *pos_dev += 1;                       // next decode position
        if (repeated && si[0] >= 0) repeated[si[0]] = 1;  // generated-token set
    }
}

constexpr int kSelectBlocks = 256;

}  // namespace

extern "C" {

CSDR_API int csdr_rms_norm(const float* x, const float* w, int ntok, int n, float eps, float* y,
                           void* hip_stream) {
    if (!x || !w || !y || ntok <= 0 || n <= 0)
        return set_error(CSDR_E_INVALID, "rms_norm: bad argument");
    rms_norm_kernel<<<ntok, kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(x, w, n, eps, y);
    CSDR_LAUNCH_CHECK("rms_norm");
    return CSDR_OK;
}

CSDR_API int csdr_dense_linear(const float* w, int R, int C, const float* x, int M, float* y,
                               void* hip_stream) {
    if (!w || !x || !y || R <= 0 || C <= 0 || M <= 0)
        return set_error(CSDR_E_INVALID, "dense_linear: bad argument");
    const int rows_per_block = kThreads / 64;
    dense_linear_kernel<<<(R + rows_per_block - 1) / rows_per_block, kThreads, 0,
                          static_cast<hipStream_t>(hip_stream)>>>(w, R, C, x, M, y);
    CSDR_LAUNCH_CHECK("dense_linear");
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
    rope_kv_kernel<<<ntok, kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(
        q, k, v, ntok, Hq, Hkv, hd, pos_dev, theta, reinterpret_cast<_Float16*>(kcache),
        reinterpret_cast<_Float16*>(vcache), max_ctx);
    CSDR_LAUNCH_CHECK("rope_kv");
    return CSDR_OK;
}

CSDR_API size_t csdr_attn_decode_workspace_bytes(int B, int Hq, int hd, int T) {
    const int nsplit = (T + kThreads - 1) / kThreads;
    return (size_t)B * Hq * nsplit * (hd + 2) * 4;
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
    const int nsplit = (T + kThreads - 1) / kThreads;
    if (nsplit > 1 && (!workspace || workspace_bytes < csdr_attn_decode_workspace_bytes(B, Hq, hd, T)))
        return set_error(CSDR_E_WORKSPACE, "attn_decode: workspace too small");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)hd);
    float* part = static_cast<float*>(workspace);
    dim3 grid(B * Hq, nsplit);
    auto k16 = reinterpret_cast<const _Float16*>(kcache);
    auto v16 = reinterpret_cast<const _Float16*>(vcache);
    if (hd == 64) {
        attn_split_kernel<64><<<grid, kThreads, 0, st>>>(q, k16, v16, lens_dev, len_host, T, Hq,
                                                        Hkv, scale, kThreads, part, out, nsplit);
        if (nsplit > 1) attn_combine_kernel<64><<<B * Hq, 64, 0, st>>>(part, nsplit, out);
    } else if (hd == 128) {
        attn_split_kernel<128><<<grid, kThreads, 0, st>>>(q, k16, v16, lens_dev, len_host, T, Hq,
                                                         Hkv, scale, kThreads, part, out, nsplit);
        if (nsplit > 1) attn_combine_kernel<128><<<B * Hq, 128, 0, st>>>(part, nsplit, out);
    } else {
        return set_error(CSDR_E_UNSUPPORTED, "attn_decode: head_dim must be 64 or 128");
    }
    CSDR_LAUNCH_CHECK("attn_decode");
    return CSDR_OK;
}

CSDR_API size_t csdr_select_workspace_bytes(void) { return (size_t)kSelectBlocks * 8; }

CSDR_API int csdr_select_best(const float* logits, int n, const uint8_t* repeated,
                              float temperature, float penalty, int* out_token, int* pos_dev,
                              uint8_t* repeated_update, void* workspace, size_t workspace_bytes,
                              void* hip_stream) {
    if (!logits || n <= 0 || !out_token) return set_error(CSDR_E_INVALID, "select_best: bad argument");
    if (!workspace || workspace_bytes < csdr_select_workspace_bytes())
        return set_error(CSDR_E_WORKSPACE, "select_best: workspace too small");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const float ts = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    float* ws_s = static_cast<float*>(workspace);
    int* ws_i = reinterpret_cast<int*>(ws_s + kSelectBlocks);
    const int nb = std::min(kSelectBlocks, (n + kThreads - 1) / kThreads);
    select1_kernel<<<nb, kThreads, 0, st>>>(logits, n, repeated, ts, penalty, ws_s, ws_i);
    select2_kernel<<<1, kThreads, 0, st>>>(ws_s, ws_i, nb, out_token, pos_dev, repeated_update);
    CSDR_LAUNCH_CHECK("select_best");
    return CSDR_OK;
}

}  // extern "C"
