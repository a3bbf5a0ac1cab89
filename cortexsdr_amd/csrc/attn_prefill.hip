// attn_prefill.hip — the prompt's multi-token causal attention and its RoPE / K-V append, for
// the decoder's batched prefill (gfx950).
//
// Reference: Kernels::multi_head_attention with the causal mask
// (kernels/attention_kernels.cpp:26-113; the tiled form kernels/flash_attention.cpp:17-163)
// as the SDK's whole-context forward runs it (api/cortex_sdk.cpp:1543-1696): q and k rotated
// on adjacent pairs at their positions (apply_rope_inplace :1395-1423), q head h reading kv
// head h / (Hq / Hkv) (repeat_kv_heads :1453-1478), scale 1 / sqrt(head_dim). Here the keys
// come from a K/V cache: the T new tokens of sequence b sit at positions p0 .. p0 + T - 1 (row
// b * T + t of q/k/v) and attend to every cached position up to their own.
//
// csdr_rope_kv_rows rotates q and k of those rows and appends k and v to the cache, with the
// decode step's rotation arithmetic (the same powf / cosf / sinf pair angles and fma forms),
// so a cache filled here holds what the token-at-a-time step would have written for the same
// projections.
//
// attn_prefill_kernel: one workgroup (4 waves) per (query block of 64 tokens, query head,
// sequence); wave w owns queries 16 w .. 16 w + 15 of the block. K/V tiles of KB positions
// are staged in LDS as fp32 (shared by the 4 waves), and each wave runs a flash-attention
// loop over 16-position sub-tiles up to its last query on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32):
//  * S^T = K Q^T: A = K rows (lane l: position l % 16), B = the scaled query (lane l: query
//    l % 16, held in registers), contraction over the head dims with lane group l / 16 taking
//    dims [HD / 4 (l / 16), + HD / 4); lane l ends with S[query l % 16][positions
//    4 (l / 16) + v], v = 0..3;
//  * causal mask and the online softmax per query column (row max and sum across the four
//    lane groups);
//  * O^T += V^T P^T: the sum over the 16 positions runs in the order step j takes position
//    4 g + j from lane group g, which is exactly the P value lane l already holds (v = j), so P
//    goes into the B operand without any exchange between lanes; A = V^T read from LDS.
// The output rows are normalised by the softmax sum at the end. Query blocks are issued
// latest first (they see the most positions).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
constexpr int kQB = 64;  // queries per workgroup

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <typename KT>
__device__ __forceinline__ void load8(const KT* p, floatx4& a, floatx4& b);
template <>
__device__ __forceinline__ void load8<float>(const float* p, floatx4& a, floatx4& b) {
    a = reinterpret_cast<const floatx4*>(p)[0];
    b = reinterpret_cast<const floatx4*>(p)[1];
}
template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16* p, floatx4& a, floatx4& b) {
    const h8 v = *reinterpret_cast<const h8*>(p);
    a = floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    b = floatx4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
}

// Row i = b * T + t at position p0 + t; one workgroup per (row, head): blocks [0, Hq) rotate a
// query head, [Hq, Hq + Hkv) rotate a key head and append it and the value head to sequence
// b's caches ([position][kv head][hd], capacity max_ctx positions).
template <typename KT>
__global__ __launch_bounds__(64) void rope_rows_kernel(float* __restrict__ q, float* __restrict__ k,
                                                       const float* __restrict__ v, int T, int p0,
                                                       int Hq, int Hkv, int hd, float theta,
                                                       KT* __restrict__ kc, KT* __restrict__ vc,
                                                       int max_ctx) {
    const int i = blockIdx.x / (Hq + Hkv);
    const int head = blockIdx.x % (Hq + Hkv);
    const int b = i / T, pos = p0 + i % T;
    float* base = head < Hq ? q + ((size_t)i * Hq + head) * hd
                            : k + ((size_t)i * Hkv + (head - Hq)) * hd;
    for (int e = threadIdx.x; e < hd / 2; e += 64) {
        const int i2 = 2 * e;
        const float freq = powf(theta, -((float)i2 / (float)hd));
        const float ang = (float)pos * freq;
        const float c = cosf(ang), sn = sinf(ang);
        const float x0 = base[i2], x1 = base[i2 + 1];
        base[i2] = fmaf(x0, c, -(x1 * sn));
        base[i2 + 1] = fmaf(x0, sn, x1 * c);
    }
    if (head < Hq) return;
    __syncthreads();
    const int kh = head - Hq;
    const size_t src = ((size_t)i * Hkv + kh) * hd;
    const size_t dst = (((size_t)b * max_ctx + pos) * Hkv + kh) * hd;
    for (int e = threadIdx.x; e < hd; e += 64) {
        kc[dst + e] = (KT)base[e];
        vc[dst + e] = (KT)v[src + e];
    }
}

template <int HD, typename KT>
__global__ __launch_bounds__(kThreads) void attn_prefill_kernel(
    const float* __restrict__ q, const KT* __restrict__ kc, const KT* __restrict__ vc, int T,
    int p0, int max_ctx, int Hq, int Hkv, float scale, float* __restrict__ out) {
    constexpr int KB = 4096 / HD;  // positions per LDS tile (64 at HD 64, 32 at HD 128)
    constexpr int LD = HD + 4;     // LDS row stride: the 16 rows of a K read and the 4 rows of
                                   // a V read fall on distinct banks
    constexpr int QS = HD / 4;     // head dims per lane group
    constexpr int NT = HD / 16;    // output dim tiles
    __shared__ __attribute__((aligned(16))) float Ks[KB * LD];
    __shared__ __attribute__((aligned(16))) float Vs[KB * LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int qb = (int)gridDim.x - 1 - (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int t0 = qb * kQB + wave * 16;
    const int tq = min(t0 + li, T - 1);  // this lane's query (rows past T compute row T - 1)
    const int qpos = p0 + tq;
    const int wave_last = p0 + min(t0 + 15, T - 1);
    const int wg_last = p0 + min(qb * kQB + kQB - 1, T - 1);

    float qf[QS];
    {
        const float* qr = q + ((size_t)(b * T + tq) * Hq + h) * HD + lg * QS;
#pragma unroll
        for (int s = 0; s < QS; s += 4) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(qr + s);
#pragma unroll
            for (int u = 0; u < 4; ++u) qf[s + u] = v[u] * scale;
        }
    }
    floatx4 o[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;
    const size_t rstride = (size_t)Hkv * HD;
    const KT* kbase = kc + ((size_t)b * max_ctx * Hkv + kvh) * HD;
    const KT* vbase = vc + ((size_t)b * max_ctx * Hkv + kvh) * HD;

    for (int k0 = 0; k0 <= wg_last; k0 += KB) {
        __syncthreads();  // the previous tile's reads are done
        for (int e = tid; e < KB * (HD / 8); e += kThreads) {
            const int row = e / (HD / 8), c8 = (e % (HD / 8)) * 8;
            const int p = k0 + row;
            floatx4 ka{0.f, 0.f, 0.f, 0.f}, kb2 = ka, va = ka, vb2 = ka;
            if (p <= wg_last) {
                load8<KT>(kbase + (size_t)p * rstride + c8, ka, kb2);
                load8<KT>(vbase + (size_t)p * rstride + c8, va, vb2);
            }
            *reinterpret_cast<floatx4*>(Ks + row * LD + c8) = ka;
            *reinterpret_cast<floatx4*>(Ks + row * LD + c8 + 4) = kb2;
            *reinterpret_cast<floatx4*>(Vs + row * LD + c8) = va;
            *reinterpret_cast<floatx4*>(Vs + row * LD + c8 + 4) = vb2;
        }
        __syncthreads();
        for (int j0 = 0; j0 < KB; j0 += 16) {
            const int kp0 = k0 + j0;
            if (kp0 > wave_last) break;  // wave-uniform: past every query of this wave
            floatx4 sacc{0.f, 0.f, 0.f, 0.f};
            const float* kr = Ks + (j0 + li) * LD + lg * QS;
#pragma unroll
            for (int s = 0; s < QS; s += 4) {
                const floatx4 kv = *reinterpret_cast<const floatx4*>(kr + s);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[u], qf[s + u], sacc, 0, 0, 0);
            }
            // sacc[v] = S[query tq][position kp0 + 4 lg + v]
            float sv[4];
            float tmax = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int kp = kp0 + 4 * lg + v;
                sv[v] = kp <= qpos ? sacc[v] : -INFINITY;
                tmax = fmaxf(tmax, sv[v]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            // position 0 is in the first sub-tile and under every query, so m_new is finite
            const float m_new = fmaxf(m_run, tmax);
            const float alpha = expf(m_run - m_new);
            float p[4];
            float ps = 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                p[v] = expf(sv[v] - m_new);
                ps += p[v];
            }
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            l_run = l_run * alpha + ps;
            m_run = m_new;
#pragma unroll
            for (int j = 0; j < NT; ++j) o[j] *= alpha;
            const float* vr = Vs + (j0 + 4 * lg) * LD + li;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int dt = 0; dt < NT; ++dt)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[j * LD + dt * 16], p[j], o[dt],
                                                                0, 0, 0);
        }
    }
    // lane holds O[query t0 + li][dims 16 dt + 4 lg + v]
    if (t0 + li < T) {
        const float inv = 1.0f / l_run;
        float* orow = out + ((size_t)(b * T + t0 + li) * Hq + h) * HD + 4 * lg;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt)
            *reinterpret_cast<floatx4*>(orow + dt * 16) = o[dt] * inv;
    }
}

template <int HD, typename KT>
void launch_prefill(const float* q, const void* kc, const void* vc, int B, int T, int p0,
                    int max_ctx, int Hq, int Hkv, float scale, float* out, hipStream_t st) {
    dim3 grid((T + kQB - 1) / kQB, Hq, B);
    attn_prefill_kernel<HD, KT><<<grid, kThreads, 0, st>>>(
        q, static_cast<const KT*>(kc), static_cast<const KT*>(vc), T, p0, max_ctx, Hq, Hkv, scale,
        out);
}

}  // namespace

extern "C" {

CSDR_API int csdr_rope_kv_rows(float* q, float* k, const float* v, int B, int T, int p0, int Hq,
                               int Hkv, int hd, float theta, void* kcache, void* vcache,
                               int kv_dtype, int max_ctx, void* hip_stream) {
    if (!q || !k || !v || !kcache || !vcache || B <= 0 || T <= 0 || p0 < 0 || Hq <= 0 ||
        Hkv <= 0 || Hq % Hkv || hd < 2 || hd % 2 || !(theta > 0.0f))
        return set_error(CSDR_E_INVALID, "rope_kv_rows: bad argument");
    if ((long long)p0 + T > max_ctx)
        return set_error(CSDR_E_INVALID, "rope_kv_rows: positions beyond the cache capacity");
    if (kv_dtype != CSDR_F32 && kv_dtype != CSDR_F16)
        return set_error(CSDR_E_INVALID, "rope_kv_rows: kv_dtype must be CSDR_F32 or CSDR_F16");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const long long blocks = (long long)B * T * (Hq + Hkv);
    if (blocks > 0x7fffffffLL) return set_error(CSDR_E_INVALID, "rope_kv_rows: too many rows");
    if (kv_dtype == CSDR_F32)
        rope_rows_kernel<float><<<(unsigned)blocks, 64, 0, st>>>(
            q, k, v, T, p0, Hq, Hkv, hd, theta, static_cast<float*>(kcache),
            static_cast<float*>(vcache), max_ctx);
    else
        rope_rows_kernel<_Float16><<<(unsigned)blocks, 64, 0, st>>>(
            q, k, v, T, p0, Hq, Hkv, hd, theta, static_cast<_Float16*>(kcache),
            static_cast<_Float16*>(vcache), max_ctx);
    CSDR_LAUNCH_CHECK("rope_kv_rows");
    return CSDR_OK;
}

CSDR_API int csdr_attn_prefill(const float* q, const void* kcache, const void* vcache,
                               int kv_dtype, int B, int T, int p0, int max_ctx, int Hq, int Hkv,
                               int hd, float scale, float* out, void* hip_stream) {
    if (!q || !kcache || !vcache || !out || B <= 0 || T <= 0 || p0 < 0 || Hq <= 0 || Hkv <= 0 ||
        Hq % Hkv)
        return set_error(CSDR_E_INVALID, "attn_prefill: bad argument");
    if ((long long)p0 + T > max_ctx)
        return set_error(CSDR_E_INVALID, "attn_prefill: positions beyond the cache capacity");
    if (hd != 64 && hd != 128)
        return set_error(CSDR_E_UNSUPPORTED, "attn_prefill: head_dim must be 64 or 128");
    if (kv_dtype != CSDR_F32 && kv_dtype != CSDR_F16)
        return set_error(CSDR_E_INVALID, "attn_prefill: kv_dtype must be CSDR_F32 or CSDR_F16");
    if (Hq > 65535 || B > 65535) return set_error(CSDR_E_INVALID, "attn_prefill: grid too large");
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                         reinterpret_cast<uintptr_t>(kcache) | reinterpret_cast<uintptr_t>(vcache);
    if (al % 16) return set_error(CSDR_E_INVALID, "attn_prefill: buffers must be 16-byte aligned");
    const float s = scale == 0.0f ? 1.0f / sqrtf((float)hd) : scale;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const bool f32 = kv_dtype == CSDR_F32;
    if (hd == 64) {
        if (f32) launch_prefill<64, float>(q, kcache, vcache, B, T, p0, max_ctx, Hq, Hkv, s, out, st);
        else launch_prefill<64, _Float16>(q, kcache, vcache, B, T, p0, max_ctx, Hq, Hkv, s, out, st);
    } else {
        if (f32) launch_prefill<128, float>(q, kcache, vcache, B, T, p0, max_ctx, Hq, Hkv, s, out, st);
        else launch_prefill<128, _Float16>(q, kcache, vcache, B, T, p0, max_ctx, Hq, Hkv, s, out, st);
    }
    CSDR_LAUNCH_CHECK("attn_prefill");
    return CSDR_OK;
}

}  // extern "C"
