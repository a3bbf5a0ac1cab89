// hsdr_encode.hip — the HSDR encoder on the GPU (gfx950): hierarchical binary matching pursuit
// over many tiles at once, and the strategy's compress around it.
//
// Reference (cortexSDR tree, src/ai_compression/strategies/HierarchicalSDRStrategy.cpp):
// hierarchicalBinaryCode :219-262 (per tile, per stage l with scale gamma_l, k greedy picks of
// argmax |<D_j, r>| with a strict '>' scan from (0, 0.0f), atoms picked earlier in the stage
// scoring 0, sign = +1 when the projection is >= 0, then r -= gamma_l * sign * D_best),
// dot_product_simd :157-190 and axpy_subtract_simd :193-216 (its AVX2 arithmetic),
// fitHierarchicalKSVD :495-602 (dictionary initialisation, hsdr_init.cpp), compress
// :1064-1237 (tiling, edge strips, serialisation), packIndexSign :76-80.
//
// mp_kernel: a workgroup of 256 threads encodes up to 8 tiles together, their residuals in
// LDS. Per pick: every 16-lane group takes atoms g, g + 16, ...; lane l accumulates the
// elements l, l + 16, ... of the dot product with one FMA chain per tile (the 16 lanes of the
// reference's two 8-wide accumulators), lanes 0..7 add the 8-element chunk, and xor-shuffles
// over 8, 4, 1, 2 lanes combine them in the reference's order (acc0 + acc1, low + high half,
// two horizontal adds): the projections are the reference's to the bit, so are the picks.
// Each D element loaded is used for every tile of the workgroup. Then one wave per tile scans
// the scores (first maximum), and the residuals are updated with one fused multiply-add per
// element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace csdr {
// fitHierarchicalKSVD's dictionary initialisation, in the reference build's arithmetic, the
// mean tile norm and atomUpdateStep's re-seed of an atom (hsdr_init.cpp).
void hsdr_init_dictionary(const float* tiles, uint32_t n, uint32_t C, uint16_t K, uint32_t slots,
                          float* D, std::mt19937* rng);
double hsdr_mean_tile_norm(const float* tiles, uint32_t n, uint32_t C);
void hsdr_reseed_atom(const float* tiles, uint32_t n, uint32_t C, uint64_t base_seed, uint32_t j,
                      uint32_t mul, double target_norm, float* atom);
}  // namespace csdr

namespace {

using csdr::set_error;

constexpr int kEThreads = 256;
constexpr int kEGroups = kEThreads / 16;
constexpr int kMaxTT = 8;        // tiles per workgroup, at most
constexpr int kMaxStages = 32;
constexpr size_t kLdsSoft = 64 * 1024;    // several workgroups per CU below this
constexpr size_t kLdsHard = 160 * 1024;

struct MpArgs {
    const float* tiles;  // n x C
    const float* D;      // K x C
    uint16_t* codes;     // n x S*k, packIndexSign
    long long n;
    int C, K, S, k, tt;
    float gamma[kMaxStages];
};

// The TT tiles' residual values of one element (TT * 4 bytes, aligned to that size) in one
// or two wide LDS reads.
template <int TT>
__device__ __forceinline__ void load_tiles(const float* rc, float* rv) {
    if constexpr (TT % 4 == 0) {
#pragma unroll
        for (int t4 = 0; t4 < TT / 4; ++t4) {
            const float4 v = reinterpret_cast<const float4*>(rc)[t4];
            rv[4 * t4] = v.x;
            rv[4 * t4 + 1] = v.y;
            rv[4 * t4 + 2] = v.z;
            rv[4 * t4 + 3] = v.w;
        }
    } else if constexpr (TT == 2) {
        const float2 v = *reinterpret_cast<const float2*>(rc);
        rv[0] = v.x;
        rv[1] = v.y;
    } else {
        rv[0] = rc[0];
    }
}

template <int TT>
__global__ __launch_bounds__(kEThreads) void mp_kernel(MpArgs a) {
    extern __shared__ float smem[];
    const int tt = TT, C = a.C, K = a.K;
    const long long t0 = (long long)blockIdx.x * tt;
    const int nt = (int)min((long long)tt, a.n - t0);
    float* r = smem;                                                    // C x TT residuals
    float* proj = r + (size_t)tt * C;                                   // nt x K scores
    uint8_t* used = reinterpret_cast<uint8_t*>(proj + (size_t)tt * K);  // nt x K
    __shared__ int best_s[TT];
    __shared__ float scale_s[TT];
    const int tid = threadIdx.x, l16 = tid & 15, grp = tid >> 4;
    const int lane = tid & 63, wave = tid >> 6;
    // residuals tile-minor, r[c * TT + t] (one 16-byte LDS read gives four tiles' values of an
    // element); slots past nt hold zeros
    for (int i = tid; i < TT * C; i += kEThreads) {
        const int c = i / TT, t = i - c * TT;
        r[i] = t < nt ? a.tiles[(t0 + t) * C + c] : 0.f;
    }
    // atoms per 16-lane group at a time: 8 with up to 2 tiles (D blocks of 4 chunks), 2 with
    // more (registers; measured 896 x 896 at 2 tiles: 0.60 ms with 2, 0.51 with 4, 0.45 with 8;
    // 4864 x 896 at 4 tiles: 3.48 ms with 2, 4.01 with 4)
    constexpr int kNA = TT <= 2 ? 8 : 2;
    constexpr int kDB = kNA >= 8 ? 4 : 8;  // chunks of an atom loaded per block
    const int C16 = C & ~15, C8 = C & ~7;  // end of the 16-element chunks, of the 8-element one
    const int nch = C16 / 16;  // full 16-element chunks (block loads clamp into them)
    const int slots = a.S * a.k;
    for (int l = 0; l < a.S; ++l) {
        for (int i = tid; i < nt * K; i += kEThreads) used[i] = 0;
        __syncthreads();
        for (int st = 0; st < a.k; ++st) {
            // 1. projections of every tile onto every atom: the atom's values 16 chunks at
            // a time, the next block in flight while this one is used (loads clamp into the
            // row's full chunks: in bounds, uniform, so the waits stay per block); tile slots
            // past nt hold zeros and are computed too (no per-tile branches)
            // kNA atoms per group at a time (j, j + 16, ...): each residual read feeds all
            for (int j = grp; j < K; j += kNA * kEGroups) {
                const float* dj[kNA];
#pragma unroll
                for (int u = 0; u < kNA; ++u) {
                    const int ju = j + u * kEGroups;
                    dj[u] = a.D + (size_t)(ju < K ? ju : j) * C + l16;
                }
                float p[kNA][TT];
#pragma unroll
                for (int u = 0; u < kNA; ++u)
#pragma unroll
                    for (int t = 0; t < TT; ++t) p[u][t] = 0.f;
                float cv[kNA][kDB], nv[kNA][kDB];
#pragma unroll
                for (int u = 0; u < kNA; ++u)
#pragma unroll
                    for (int q = 0; q < kDB; ++q) cv[u][q] = nch ? dj[u][min(q, nch - 1) * 16] : 0.f;
                for (int b0 = 0; b0 < nch; b0 += kDB) {
#pragma unroll
                    for (int u = 0; u < kNA; ++u)
#pragma unroll
                        for (int q = 0; q < kDB; ++q)
                            nv[u][q] = dj[u][min(b0 + kDB + q, nch - 1) * 16];
#pragma unroll
                    for (int q = 0; q < kDB; ++q) {
                        if (b0 + q >= nch) break;
                        float rv[TT];
                        load_tiles<TT>(r + ((b0 + q) * 16 + l16) * TT, rv);
#pragma unroll
                        for (int u = 0; u < kNA; ++u)
#pragma unroll
                            for (int t = 0; t < TT; ++t) p[u][t] = fmaf(cv[u][q], rv[t], p[u][t]);
                    }
#pragma unroll
                    for (int u = 0; u < kNA; ++u)
#pragma unroll
                        for (int q = 0; q < kDB; ++q) cv[u][q] = nv[u][q];
                }
                if (C8 > C16 && l16 < 8) {
                    const float* rc = r + (C16 + l16) * TT;
#pragma unroll
                    for (int u = 0; u < kNA; ++u) {
                        const float dv = dj[u][C16];
#pragma unroll
                        for (int t = 0; t < TT; ++t) p[u][t] = fmaf(dv, rc[t], p[u][t]);
                    }
                }
#pragma unroll
                for (int u = 0; u < kNA; ++u) {
                    const int ju = j + u * kEGroups;
                    const float* dt = dj[u] - l16;  // the atom's row
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        float v = p[u][t];
                        v += __shfl_xor(v, 8, 16);  // acc0 + acc1
                        v += __shfl_xor(v, 4, 16);  // low + high 128 bits
                        v += __shfl_xor(v, 1, 16);  // horizontal add
                        v += __shfl_xor(v, 2, 16);  // horizontal add
                        // the last C % 8 elements: the scalar tail, in element order
                        for (int c = C8; c < C; ++c) v = fmaf(dt[c], r[c * TT + t], v);
                        if (l16 == 0 && t < nt && ju < K)
                            proj[t * K + ju] = used[t * K + ju] ? 0.0f : v;
                    }
                }
            }
            __syncthreads();
            // 2. the pick per tile: first maximum of |score|, as the reference's scan
            for (int t = wave; t < nt; t += kEThreads / 64) {
                float bv = 0.f;
                int bi = 0;
                for (int j = lane; j < K; j += 64) {
                    const float av = fabsf(proj[t * K + j]);
                    if (av > bv) {
                        bv = av;
                        bi = j;
                    }
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) {
                    const float ov = __shfl_xor(bv, off, 64);
                    const int oi = __shfl_xor(bi, off, 64);
                    if (ov > bv || (ov == bv && oi < bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                if (lane == 0) {
                    const int sg = proj[t * K + bi] >= 0.0f ? 1 : -1;
                    a.codes[(size_t)(t0 + t) * slots + l * a.k + st] =
                        (uint16_t)((bi & 0x7FFF) | (sg < 0 ? 0x8000 : 0));
                    used[t * K + bi] = 1;
                    best_s[t] = bi;
                    scale_s[t] = a.gamma[l] * (float)sg;
                }
            }
            __syncthreads();
            // 3. r -= scale * D[best], fused
            for (int i = tid; i < nt * C; i += kEThreads) {
                const int t = i / C, c = i - t * C;
                float& rv = r[c * TT + t];
                rv = fmaf(-a.D[(size_t)best_s[t] * C + c], scale_s[t], rv);
            }
            __syncthreads();
        }
    }
}

size_t mp_lds_bytes(int tt, int C, int K) {
    return (size_t)tt * ((size_t)C + K) * 4 + csdr::align_up((size_t)tt * K, 16);
}

// Tiles per workgroup: about n / 1024, at least 2 (measured on the Qwen2-0.5B shapes, 1-row
// tiles: 896 x 896 best at 2 (0.93 ms vs 1.00 at 4, 1.31 at 8), 4864 x 896 at 4 (4.5 ms vs 5.0
// at 8, 7.3 at 2): enough workgroups per CU to hide latency, and every workgroup reads all of
// D once per pick, so more tiles each is less D traffic), a power of two, at most 8 and what
// fits under the soft LDS size; else one tile under the hard size; else 0 (too large).
int mp_tiles_per_wg(long long n, int C, int K) {
    const char* ev = std::getenv("CSDR_HSDR_TILES_PER_WG");  // tuning override: 1, 2, 4 or 8
    long long want = std::min<long long>(kMaxTT, std::max<long long>(2, n / 1024));
    if (ev && std::atoi(ev) >= 1) want = std::min(kMaxTT, std::atoi(ev));
    for (int tt = kMaxTT; tt >= 1; tt >>= 1)  // a power of two (the kernel's template)
        if (tt <= want && mp_lds_bytes(tt, C, K) <= kLdsSoft) return tt;
    return mp_lds_bytes(1, C, K) <= kLdsHard ? 1 : 0;
}

int check_mp_shape(long long n, int C, int K, int S, int k) {
    if (n < 0 || C <= 0 || K <= 0 || S <= 0 || k <= 0)
        return set_error(CSDR_E_INVALID, "hsdr_encode: bad shape");
    if (K > 32768) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: at most 32768 atoms");
    if (S > kMaxStages) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: at most 32 stages");
    if (k > K) return set_error(CSDR_E_INVALID, "hsdr_encode: more picks per stage than atoms");
    if (mp_tiles_per_wg(n, C, K) == 0)
        return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: tile and dictionary exceed LDS");
    return CSDR_OK;
}

int launch_mp(const float* tiles, long long n, int C, const float* D, int K, int S, int k,
              const float* gamma, uint16_t* codes, hipStream_t st) {
    if (n == 0) return CSDR_OK;
    MpArgs a{};
    a.tiles = tiles;
    a.D = D;
    a.codes = codes;
    a.n = n;
    a.C = C;
    a.K = K;
    a.S = S;
    a.k = k;
    a.tt = mp_tiles_per_wg(n, C, K);
    for (int l = 0; l < S; ++l) a.gamma[l] = gamma[l];
    const size_t lds = mp_lds_bytes(a.tt, C, K);
    const long long grid = (n + a.tt - 1) / a.tt;
    if (grid > 0x7fffffffLL) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: too many tiles");
    auto go = [&](auto kern) {
        if (lds > 64 * 1024)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        kern<<<(unsigned)grid, kEThreads, lds, st>>>(a);
    };
    switch (a.tt) {
        case 8: go(&mp_kernel<8>); break;
        case 4: go(&mp_kernel<4>); break;
        case 2: go(&mp_kernel<2>); break;
        default: go(&mp_kernel<1>); break;
    }
    CSDR_LAUNCH_CHECK("hsdr_encode");
    return CSDR_OK;
}

// ---------------------------------------------------------------- K-SVD atom update

// atomUpdateStep (HierarchicalSDRStrategy.cpp:281-490) on the device, per refinement pass:
//  residual_kernel: residual = tile - sum over slots of gamma_l * sign * D[idx], one thread
//    per element, slots in order, each term fused (the reference's r[c] += scale * atom[c],
//    :300-311), then tile - recon (:316-320);
//  atom_update_kernel: one workgroup per atom with users; correction[c] = sum over the atom's
//    users, in (tile, slot) order, of sign * gamma * residual (double, fused: :428-437), the
//    new value atom + correction * (0.5 / sum gamma^2) rounded to float (:448-458), a
//    non-finite value flags the atom for the host's re-seed (:461), the squared norm summed
//    in element order as the reference's loop does (:456), and atoms longer than the cap
//    scaled back to the target norm (:482-487). Atoms without users are re-seeded by the
//    host (:411-425).
struct ResArgs {
    const float* tiles;
    const float* D;
    const uint16_t* codes;
    float* res;
    long long n;
    int C, S, k;
    float gamma[kMaxStages];
};

__global__ __launch_bounds__(kEThreads) void residual_kernel(ResArgs a) {
    const long long total = a.n * a.C;
    const int slots = a.S * a.k;
    for (long long e = (long long)blockIdx.x * kEThreads + threadIdx.x; e < total;
         e += (long long)gridDim.x * kEThreads) {
        const long long i = e / a.C;
        const int c = (int)(e - i * a.C);
        const uint16_t* cd = a.codes + i * slots;
        float rec = 0.0f;
        for (int sl = 0; sl < slots; ++sl) {
            const uint16_t v = cd[sl];
            const float scale = a.gamma[sl / a.k] * ((v & 0x8000) ? -1.0f : 1.0f);
            rec = fmaf(scale, a.D[(size_t)(v & 0x7FFF) * a.C + c], rec);
        }
        a.res[e] = a.tiles[e] - rec;
    }
}

constexpr uint8_t kAtomKept = 0, kAtomNonFinite = 1, kAtomDead = 2;

__global__ __launch_bounds__(kEThreads) void atom_update_kernel(
    const float* __restrict__ res, int C, float* __restrict__ D, const int* __restrict__ off,
    const uint32_t* __restrict__ utile, const double* __restrict__ ucoef,
    const double* __restrict__ inv_w, double cap, double target, uint8_t* __restrict__ flag) {
    extern __shared__ float nv[];  // C: the atom's new values
    __shared__ double nsq_s;
    const int j = blockIdx.x, tid = threadIdx.x;
    const int u0 = off[j], u1 = off[j + 1];
    if (u0 == u1) {
        if (tid == 0) flag[j] = kAtomDead;
        return;
    }
    const double iw = inv_w[j];
    if (iw == 0.0) {  // sum of gamma^2 <= 1e-12: the atom stays
        if (tid == 0) flag[j] = kAtomKept;
        return;
    }
    float* atom = D + (size_t)j * C;
    int bad = 0;
    for (int c = tid; c < C; c += kEThreads) {
        double corr = 0.0;
        for (int u = u0; u < u1; ++u)
            corr = fma(ucoef[u], (double)res[(size_t)utile[u] * C + c], corr);
        const double v = fma(corr, iw, (double)atom[c]);
        const float vf = (float)v;
        if (!isfinite(v) || !isfinite(vf)) bad = 1;
        nv[c] = vf;
    }
    if (__syncthreads_or(bad)) {
        if (tid == 0) flag[j] = kAtomNonFinite;
        return;
    }
    if (tid == 0) {
        double sq = 0.0;
        for (int c = 0; c < C; ++c) sq = fma((double)nv[c], (double)nv[c], sq);
        nsq_s = sq;
        flag[j] = isfinite(sq) ? kAtomKept : kAtomNonFinite;
    }
    __syncthreads();
    const double nsq = nsq_s;
    if (!isfinite(nsq)) return;
    const double nn = sqrt(nsq);
    if (nn > cap) {
        const double sc = target / nn;
        for (int c = tid; c < C; c += kEThreads) atom[c] = (float)((double)nv[c] * sc);
    } else {
        for (int c = tid; c < C; c += kEThreads) atom[c] = nv[c];
    }
}

// ---------------------------------------------------------------- compress (host side)

struct Geometry {
    uint32_t R, C, tr, tc, R_full, C_full, n_tiles, tile_dim, edge_floats;
    uint16_t K;
    uint8_t S, k;
};

// The strategy's geometry (compress :1130-1160; configFor :1024-1046 widens 1-row tiles to
// the whole row).
int geometry(uint32_t R, uint32_t C, uint16_t tile_rows, uint16_t tile_cols, uint16_t K,
             uint8_t S, uint8_t k, Geometry* g) {
    if (R == 0 || C == 0 || tile_rows == 0 || tile_cols == 0 || K == 0 || S == 0 || k == 0)
        return set_error(CSDR_E_INVALID, "hsdr_compress: bad shape or config");
    g->R = R;
    g->C = C;
    g->tr = tile_rows;
    g->tc = (tile_rows == 1 && C <= 0xFFFFu) ? C : tile_cols;
    g->R_full = R / g->tr * g->tr;
    g->C_full = C / g->tc * g->tc;
    if (g->R_full == 0 || g->C_full == 0)
        return set_error(CSDR_E_FORMAT, "HSDR: tensor too small to hold even one full tile");
    g->n_tiles = (g->R_full / g->tr) * (g->C_full / g->tc);
    g->tile_dim = g->tr * g->tc;
    if (g->n_tiles < K)
        return set_error(CSDR_E_FORMAT,
                         "HSDR: not enough tiles to fit the requested dictionary size");
    g->edge_floats = g->R_full * (C - g->C_full) + (R - g->R_full) * C;
    g->K = K;
    g->S = S;
    g->k = k;
    return CSDR_OK;
}

size_t stream_bytes(const Geometry& g) {
    return 36 + (size_t)g.S * 4 + (size_t)g.K * g.tile_dim * 4 +
           (size_t)g.n_tiles * g.S * g.k * 2 + (size_t)g.edge_floats * 4;
}

// A device allocation freed with its scope.
struct DevBuf {
    void* p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    float* f() const { return static_cast<float*>(p); }
    uint16_t* u16() const { return static_cast<uint16_t*>(p); }
};

// One atomUpdateStep per pass (HierarchicalSDRStrategy.cpp:281-490): the users of every atom
// gathered on the host from the current codes in (tile, slot) order (:325-339) with their
// sign * gamma and the sum of gamma^2 (fused, :428-437), the residuals and the updates on the
// device, the re-seeds on the host from the fit's generator (base seed :403).
struct Refine {
    DevBuf res, off, utile, ucoef, invw, flag;
    double target = 0.0, cap = 0.0;

    int init(const Geometry& g, const std::vector<float>& tiles, hipStream_t) {
        const size_t slots = (size_t)g.S * g.k, ncodes = (size_t)g.n_tiles * slots;
        target = std::max(1e-6, csdr::hsdr_mean_tile_norm(tiles.data(), g.n_tiles, g.tile_dim) /
                                    std::sqrt((double)slots));  // :390-392
        cap = 1.5 * target;
        CSDR_HIP_CHECK(hipMalloc(&res.p, tiles.size() * 4));
        CSDR_HIP_CHECK(hipMalloc(&off.p, ((size_t)g.K + 1) * 4));
        CSDR_HIP_CHECK(hipMalloc(&utile.p, std::max<size_t>(ncodes, 1) * 4));
        CSDR_HIP_CHECK(hipMalloc(&ucoef.p, std::max<size_t>(ncodes, 1) * 8));
        CSDR_HIP_CHECK(hipMalloc(&invw.p, (size_t)g.K * 8));
        CSDR_HIP_CHECK(hipMalloc(&flag.p, (size_t)g.K));
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&atom_update_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)(g.tile_dim * 4));
        return CSDR_OK;
    }

    int pass(const Geometry& g, const std::vector<float>& tiles, const std::vector<float>& gamma,
             const float* d_tiles, float* d_D, const uint16_t* d_codes, std::mt19937& rng,
             hipStream_t st) {
        const size_t slots = (size_t)g.S * g.k, ncodes = (size_t)g.n_tiles * slots;
        const uint32_t C = g.tile_dim;
        std::vector<uint16_t> codes(ncodes);
        CSDR_HIP_CHECK(
            hipMemcpyAsync(codes.data(), d_codes, ncodes * 2, hipMemcpyDeviceToHost, st));
        CSDR_HIP_CHECK(hipStreamSynchronize(st));
        std::vector<int> offs((size_t)g.K + 1, 0);
        for (uint16_t v : codes) {
            if ((v & 0x7FFF) >= g.K) return set_error(CSDR_E_INVALID, "hsdr_compress: bad code");
            ++offs[(v & 0x7FFF) + 1];
        }
        for (uint32_t j = 0; j < g.K; ++j) offs[j + 1] += offs[j];
        std::vector<int> pos(offs.begin(), offs.end() - 1);
        std::vector<uint32_t> ut(ncodes);
        std::vector<double> uc(ncodes), wsum(g.K, 0.0), iw(g.K, 0.0);
        for (size_t i = 0; i < g.n_tiles; ++i)
            for (size_t sl = 0; sl < slots; ++sl) {
                const uint16_t v = codes[i * slots + sl];
                const uint32_t j = v & 0x7FFF;
                const double gm = (double)gamma[sl / g.k];
                const int p = pos[j]++;
                ut[p] = (uint32_t)i;
                uc[p] = ((v & 0x8000) ? -1.0 : 1.0) * gm;
                wsum[j] = std::fma(gm, gm, wsum[j]);
            }
        for (uint32_t j = 0; j < g.K; ++j) iw[j] = wsum[j] <= 1e-12 ? 0.0 : 0.5 / wsum[j];
        CSDR_HIP_CHECK(
            hipMemcpyAsync(off.p, offs.data(), offs.size() * 4, hipMemcpyHostToDevice, st));
        CSDR_HIP_CHECK(hipMemcpyAsync(utile.p, ut.data(), ncodes * 4, hipMemcpyHostToDevice, st));
        CSDR_HIP_CHECK(hipMemcpyAsync(ucoef.p, uc.data(), ncodes * 8, hipMemcpyHostToDevice, st));
        CSDR_HIP_CHECK(hipMemcpyAsync(invw.p, iw.data(), iw.size() * 8, hipMemcpyHostToDevice, st));
        const uint64_t base_seed = static_cast<uint64_t>(rng()) ^ 0xA0B1C2D3u;

        ResArgs ra{};
        ra.tiles = d_tiles;
        ra.D = d_D;
        ra.codes = d_codes;
        ra.res = res.f();
        ra.n = g.n_tiles;
        ra.C = (int)C;
        ra.S = g.S;
        ra.k = g.k;
        for (uint32_t l = 0; l < g.S; ++l) ra.gamma[l] = gamma[l];
        const long long total = (long long)g.n_tiles * C;
        const int rgrid = (int)std::min<long long>((total + kEThreads - 1) / kEThreads, 16384);
        residual_kernel<<<rgrid, kEThreads, 0, st>>>(ra);
        CSDR_LAUNCH_CHECK("hsdr_compress residual");
        atom_update_kernel<<<g.K, kEThreads, (size_t)C * 4, st>>>(
            res.f(), (int)C, d_D, static_cast<const int*>(off.p),
            static_cast<const uint32_t*>(utile.p), static_cast<const double*>(ucoef.p),
            static_cast<const double*>(invw.p), cap, target, static_cast<uint8_t*>(flag.p));
        CSDR_LAUNCH_CHECK("hsdr_compress atom update");
        std::vector<uint8_t> fl(g.K);
        CSDR_HIP_CHECK(hipMemcpyAsync(fl.data(), flag.p, g.K, hipMemcpyDeviceToHost, st));
        CSDR_HIP_CHECK(hipStreamSynchronize(st));
        std::vector<float> atom(C);
        for (uint32_t j = 0; j < g.K; ++j) {
            if (fl[j] == kAtomKept) continue;
            csdr::hsdr_reseed_atom(tiles.data(), g.n_tiles, C, base_seed, j,
                                   fl[j] == kAtomDead ? 0x9E3779B1u : 0xB7E15163u, target,
                                   atom.data());
            CSDR_HIP_CHECK(hipMemcpy(d_D + (size_t)j * C, atom.data(), (size_t)C * 4,
                                     hipMemcpyHostToDevice));
        }
        return CSDR_OK;
    }
};

template <class T>
void put(std::vector<uint8_t>& out, const T& v) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
    out.insert(out.end(), p, p + sizeof(T));
}

// fitHierarchicalKSVD (HierarchicalSDRStrategy.cpp:494-607) over host tiles (n x tile_dim):
// the dictionary initialisation on the host from the fit's generator (mt19937(0xC0DE), :513),
// matching pursuit on the GPU, then ksvd_iters atom-update passes each followed by matching
// pursuit again (:570-573); D (K x tile_dim, non-finite values zeroed as :592-601) and, when
// codes is not null, the final codes.
int fit_tiles(const std::vector<float>& tiles, uint32_t n_tiles, uint32_t tile_dim, uint16_t K,
              uint8_t S, uint8_t k, uint8_t ksvd_iters, const std::vector<float>& gamma,
              std::vector<float>& D, std::vector<uint16_t>* codes_out, hipStream_t st) {
    Geometry g{};
    g.n_tiles = n_tiles;
    g.tile_dim = tile_dim;
    g.K = K;
    g.S = S;
    g.k = k;
    if (ksvd_iters != 0 && tile_dim > 32768)
        return set_error(CSDR_E_UNSUPPORTED,
                         "hsdr_compress: K-SVD refinement takes tiles of at most 32768 values");
    int rc = check_mp_shape(n_tiles, (int)tile_dim, K, S, k);
    if (rc != CSDR_OK) return rc;
    D.assign((size_t)K * tile_dim, 0.0f);
    std::mt19937 rng(0xC0DE);  // the fit's generator (:513), through init and every pass
    csdr::hsdr_init_dictionary(tiles.data(), n_tiles, tile_dim, K, (uint32_t)S * k, D.data(),
                               &rng);
    const size_t ncodes = (size_t)n_tiles * S * k;
    DevBuf d_tiles, d_D, d_codes;
    CSDR_HIP_CHECK(hipMalloc(&d_tiles.p, std::max<size_t>(tiles.size(), 1) * 4));
    CSDR_HIP_CHECK(hipMalloc(&d_D.p, D.size() * 4));
    CSDR_HIP_CHECK(hipMalloc(&d_codes.p, std::max<size_t>(ncodes * 2, 2)));
    CSDR_HIP_CHECK(hipMemcpyAsync(d_tiles.p, tiles.data(), tiles.size() * 4,
                                  hipMemcpyHostToDevice, st));
    CSDR_HIP_CHECK(hipMemcpyAsync(d_D.p, D.data(), D.size() * 4, hipMemcpyHostToDevice, st));
    rc = launch_mp(d_tiles.f(), n_tiles, (int)tile_dim, d_D.f(), K, S, k, gamma.data(),
                   d_codes.u16(), st);
    if (rc != CSDR_OK) return rc;
    if (ksvd_iters) {
        Refine rf;
        rc = rf.init(g, tiles, st);
        if (rc != CSDR_OK) return rc;
        for (int it = 0; it < ksvd_iters; ++it) {  // atom update, then encode again (:570-573)
            rc = rf.pass(g, tiles, gamma, d_tiles.f(), d_D.f(), d_codes.u16(), rng, st);
            if (rc != CSDR_OK) return rc;
            rc = launch_mp(d_tiles.f(), n_tiles, (int)tile_dim, d_D.f(), K, S, k, gamma.data(),
                           d_codes.u16(), st);
            if (rc != CSDR_OK) return rc;
        }
        CSDR_HIP_CHECK(hipMemcpyAsync(D.data(), d_D.p, D.size() * 4, hipMemcpyDeviceToHost, st));
    }
    if (codes_out) {
        codes_out->resize(ncodes);
        CSDR_HIP_CHECK(hipMemcpyAsync(codes_out->data(), d_codes.p, ncodes * 2,
                                      hipMemcpyDeviceToHost, st));
    }
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    for (float& x : D)  // the fit's final sanitisation (:592-601)
        if (!std::isfinite(x)) x = 0.0f;
    return CSDR_OK;
}

// Matching pursuit of host tiles against a fixed dictionary (encodeAllTilesAgainstDictionary,
// the encode of compressFP32WithExternalDictionary :1690-1754).
int encode_tiles(const float* tiles, uint32_t n_tiles, uint32_t tile_dim, const std::vector<float>& D,
                 uint16_t K, uint8_t S, uint8_t k, const std::vector<float>& gamma,
                 std::vector<uint16_t>& codes, hipStream_t st) {
    int rc = check_mp_shape(n_tiles, (int)tile_dim, K, S, k);
    if (rc != CSDR_OK) return rc;
    const size_t ncodes = (size_t)n_tiles * S * k;
    DevBuf d_tiles, d_D, d_codes;
    CSDR_HIP_CHECK(hipMalloc(&d_tiles.p, std::max<size_t>((size_t)n_tiles * tile_dim, 1) * 4));
    CSDR_HIP_CHECK(hipMalloc(&d_D.p, D.size() * 4));
    CSDR_HIP_CHECK(hipMalloc(&d_codes.p, std::max<size_t>(ncodes * 2, 2)));
    CSDR_HIP_CHECK(hipMemcpyAsync(d_tiles.p, tiles, (size_t)n_tiles * tile_dim * 4,
                                  hipMemcpyHostToDevice, st));
    CSDR_HIP_CHECK(hipMemcpyAsync(d_D.p, D.data(), D.size() * 4, hipMemcpyHostToDevice, st));
    rc = launch_mp(d_tiles.f(), n_tiles, (int)tile_dim, d_D.f(), K, S, k, gamma.data(),
                   d_codes.u16(), st);
    if (rc != CSDR_OK) return rc;
    codes.resize(ncodes);
    CSDR_HIP_CHECK(hipMemcpyAsync(codes.data(), d_codes.p, ncodes * 2, hipMemcpyDeviceToHost, st));
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    return CSDR_OK;
}

// Tiles of an R x C matrix in row-major tile order (extractTiles :94-116), of its aligned
// top-left block.
std::vector<float> extract_tiles(const float* w, uint32_t R, uint32_t C, uint32_t tr,
                                 uint32_t tc) {
    const uint32_t nrt = R / tr, nct = C / tc;
    std::vector<float> tiles((size_t)nrt * nct * tr * tc);
    for (uint32_t br = 0; br < nrt; ++br)
        for (uint32_t bc = 0; bc < nct; ++bc) {
            float* dst = tiles.data() + (size_t)(br * nct + bc) * tr * tc;
            for (uint32_t r = 0; r < tr; ++r)
                std::memcpy(dst + (size_t)r * tc, w + (size_t)(br * tr + r) * C + (size_t)bc * tc,
                            sizeof(float) * tc);
        }
    return tiles;
}

// compressGroupedSegments' bucket key and its hash (HierarchicalSDRStrategy.cpp:2088-2120),
// so that the buckets come out of the same std::unordered_map in the same order.
struct GroupKey {
    uint16_t tile_rows, tile_cols, n_atoms;
    uint8_t n_stages, k;
    float decay;
    bool operator==(const GroupKey& o) const {
        return tile_rows == o.tile_rows && tile_cols == o.tile_cols && n_atoms == o.n_atoms &&
               n_stages == o.n_stages && k == o.k && decay == o.decay;
    }
};
struct GroupKeyHash {
    size_t operator()(const GroupKey& g) const {
        size_t h = std::hash<uint32_t>{}(((uint32_t)g.tile_rows << 16) | g.tile_cols);
        h ^= std::hash<uint32_t>{}(((uint32_t)g.n_atoms << 16) | ((uint32_t)g.n_stages << 8) | g.k) +
             0x9e3779b9 + (h << 6) + (h >> 2);
        h ^= std::hash<float>{}(g.decay) + 0x9e3779b9 + (h << 6) + (h >> 2);
        return h;
    }
};

}  // namespace

extern "C" {

CSDR_API int csdr_hsdr_encode(const float* tiles, size_t n_tiles, int tile_dim, const float* D,
                              int n_atoms, int n_stages, int k_per_stage,
                              const float* stage_scales, uint16_t* codes, void* hip_stream) {
    if ((n_tiles && (!tiles || !codes)) || !D || !stage_scales)
        return set_error(CSDR_E_INVALID, "hsdr_encode: null pointer");
    const int rc = check_mp_shape((long long)n_tiles, tile_dim, n_atoms, n_stages, k_per_stage);
    if (rc != CSDR_OK) return rc;
    return launch_mp(tiles, (long long)n_tiles, tile_dim, D, n_atoms, n_stages, k_per_stage,
                     stage_scales, codes, static_cast<hipStream_t>(hip_stream));
}

CSDR_API int csdr_hsdr_init_dictionary(const float* tiles, uint32_t n_tiles, uint32_t tile_dim,
                                       uint16_t n_atoms, uint8_t n_stages, uint8_t k_per_stage,
                                       float* D) {
    if (!tiles || !D || n_tiles == 0 || tile_dim == 0 || n_atoms == 0 || n_stages == 0 ||
        k_per_stage == 0)
        return set_error(CSDR_E_INVALID, "hsdr_init_dictionary: bad argument");
    csdr::hsdr_init_dictionary(tiles, n_tiles, tile_dim, n_atoms,
                               (uint32_t)n_stages * k_per_stage, D, nullptr);
    return CSDR_OK;
}

CSDR_API size_t csdr_hsdr_compress_bytes(uint32_t rows, uint32_t cols, uint16_t tile_rows,
                                         uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                                         uint8_t k_per_stage) {
    Geometry g;
    if (geometry(rows, cols, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage, &g) !=
        CSDR_OK)
        return 0;
    return stream_bytes(g);
}

CSDR_API int csdr_hsdr_compress(const float* w, uint32_t rows, uint32_t cols, uint16_t tile_rows,
                                uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                                uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay,
                                uint8_t* out, size_t out_bytes, void* hip_stream) {
    if (!w || !out) return set_error(CSDR_E_INVALID, "hsdr_compress: null pointer");
    Geometry g;
    int rc = geometry(rows, cols, tile_rows, tile_cols, n_atoms, n_stages, k_per_stage, &g);
    if (rc != CSDR_OK) return rc;
    if (out_bytes < stream_bytes(g))
        return set_error(CSDR_E_INVALID, "hsdr_compress: output buffer too small");
    if (ksvd_iters != 0 && g.tile_dim > 32768)
        return set_error(CSDR_E_UNSUPPORTED,
                         "hsdr_compress: K-SVD refinement takes tiles of at most 32768 values");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    // tiles in row-major tile order (extractTiles :94-116) of the aligned block
    std::vector<float> tiles = extract_tiles(w, g.R_full, g.C, g.tr, g.tc);
    tiles.resize((size_t)g.n_tiles * g.tile_dim);
    std::vector<float> gamma(g.S), D;
    for (uint32_t l = 0; l < g.S; ++l) gamma[l] = std::pow(stage_decay, (float)l);
    std::vector<uint16_t> codes;
    rc = fit_tiles(tiles, g.n_tiles, g.tile_dim, g.K, g.S, g.k, ksvd_iters, gamma, D, &codes, st);
    if (rc != CSDR_OK) return rc;

    // serialisation (:1197-1237): header, stage scales, D, packed codes, edge strips
    std::vector<uint8_t> s;
    s.reserve(stream_bytes(g));
    s.insert(s.end(), {'H', 'S', 'D', 'R'});
    put<uint32_t>(s, 2);
    put<uint32_t>(s, g.R);
    put<uint32_t>(s, g.C);
    put<uint32_t>(s, g.n_tiles);
    put<uint16_t>(s, (uint16_t)g.tr);
    put<uint16_t>(s, (uint16_t)g.tc);
    put<uint16_t>(s, g.K);
    put<uint8_t>(s, g.S);
    put<uint8_t>(s, g.k);
    put<float>(s, stage_decay);
    put<uint32_t>(s, g.edge_floats * 4);
    for (float x : gamma) put<float>(s, x);
    for (float x : D) put<float>(s, x);
    for (uint16_t c : codes) put<uint16_t>(s, c);
    for (uint32_t r = 0; r < g.R_full; ++r)
        for (uint32_t c = g.C_full; c < g.C; ++c) put<float>(s, w[(size_t)r * g.C + c]);
    for (uint32_t r = g.R_full; r < g.R; ++r)
        for (uint32_t c = 0; c < g.C; ++c) put<float>(s, w[(size_t)r * g.C + c]);
    std::memcpy(out, s.data(), s.size());
    return CSDR_OK;
}

CSDR_API int csdr_hsda_build(int n, const char* const* names, const float* const* w,
                             const uint32_t* rows, const uint32_t* cols,
                             const uint8_t* original_types, uint16_t tile_rows,
                             uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                             uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay,
                             uint32_t max_tiles_for_fit, uint8_t** out, size_t* out_size,
                             uint8_t* skipped, void* hip_stream) {
    if (n <= 0 || !names || !w || !rows || !cols || !out || !out_size)
        return set_error(CSDR_E_INVALID, "hsda_build: bad argument");
    if (tile_rows == 0 || tile_cols == 0 || n_atoms == 0 || n_stages == 0 || k_per_stage == 0)
        return set_error(CSDR_E_INVALID, "hsda_build: bad config");
    *out = nullptr;
    *out_size = 0;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    try {
        // configFor per segment (1-row tiles widen to the row), suitability (:2147-2190:
        // shape divisible by the tile; the caller's matrices are fp32), buckets by config
        std::vector<GroupKey> keys(n);
        std::unordered_map<GroupKey, std::vector<size_t>, GroupKeyHash> buckets;
        std::vector<uint8_t> skip(n, 0);
        for (int i = 0; i < n; ++i) {
            if (!names[i] || !w[i]) return set_error(CSDR_E_INVALID, "hsda_build: null entry");
            GroupKey key{tile_rows, (tile_rows == 1 && cols[i] <= 0xFFFFu) ? (uint16_t)cols[i]
                                                                          : tile_cols,
                         n_atoms, n_stages, k_per_stage, stage_decay};
            keys[i] = key;
            if (rows[i] == 0 || cols[i] == 0 || rows[i] % key.tile_rows ||
                cols[i] % key.tile_cols) {
                skip[i] = 1;
                continue;
            }
            buckets[key].push_back((size_t)i);
        }
        std::vector<float> gamma(n_stages);
        for (uint32_t l = 0; l < n_stages; ++l) gamma[l] = std::pow(stage_decay, (float)l);
        struct Dict {
            GroupKey key;
            std::vector<float> atoms;
        };
        struct Entry {
            size_t seg, dict;
            std::vector<uint16_t> codes;
            uint32_t n_tiles;
        };
        std::vector<Dict> dicts;
        std::vector<Entry> entries;
        for (auto& kv : buckets) {
            const GroupKey& key = kv.first;
            const uint32_t tr = key.tile_rows, tc = key.tile_cols, tile_dim = tr * tc;
            uint64_t total = 0;
            for (size_t i : kv.second) total += (uint64_t)(rows[i] / tr) * (cols[i] / tc);
            const uint32_t pooled_count = total > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)total;
            const uint32_t cap = (max_tiles_for_fit > 0 && total > max_tiles_for_fit)
                                     ? max_tiles_for_fit
                                     : pooled_count;
            const bool reservoir = cap < pooled_count;
            std::vector<float> pool((size_t)cap * tile_dim);
            std::mt19937 res_rng(0xC0DECAFEu ^ cap);  // :2277
            uint64_t seen = 0;
            uint32_t fill = 0;
            std::vector<size_t> pooled_segs;
            std::vector<std::vector<float>> seg_tiles;
            for (size_t i : kv.second) {
                // per-segment non-finite gate (:2324-2358): probe 1 in 256, then sanitise and
                // skip the segment when more than 1e-3 of it is bad. The sanitised values are
                // also what the segment is encoded from, in every tile mode; the reference
                // re-encodes 2-D segments from the raw values (:2373, :2474-2475), letting
                // NaN / Inf into matching pursuit (a deliberate difference)
                std::vector<float> m(w[i], w[i] + (size_t)rows[i] * cols[i]);
                bool any_bad = false;
                for (size_t j = 0; j < m.size(); j += 256)
                    if (!std::isfinite(m[j])) {
                        any_bad = true;
                        break;
                    }
                if (any_bad) {
                    size_t bad = 0;
                    for (float& v : m)
                        if (!std::isfinite(v)) {
                            v = 0.0f;
                            ++bad;
                        }
                    if ((double)bad / std::max<size_t>(1, m.size()) > 1e-3) {
                        skip[i] = 1;
                        continue;
                    }
                }
                std::vector<float> t = (tr == 1 && tc == cols[i])
                                           ? std::move(m)
                                           : extract_tiles(m.data(), rows[i], cols[i], tr, tc);
                const uint32_t nt = (rows[i] / tr) * (cols[i] / tc);
                for (uint32_t j = 0; j < nt; ++j) {
                    const float* src = t.data() + (size_t)j * tile_dim;
                    if (!reservoir || fill < cap) {
                        std::memcpy(pool.data() + (size_t)fill * tile_dim, src, tile_dim * 4);
                        ++fill;
                    } else {
                        std::uniform_int_distribution<uint64_t> dist(0, seen);
                        const uint64_t r = dist(res_rng);
                        if (r < cap) std::memcpy(pool.data() + r * tile_dim, src, tile_dim * 4);
                    }
                    ++seen;
                }
                pooled_segs.push_back(i);
                seg_tiles.push_back(std::move(t));
            }
            pool.resize((size_t)fill * tile_dim);
            for (float& v : pool)  // pool integrity (:2403-2419)
                if (!std::isfinite(v)) v = 0.0f;
            if (fill < key.n_atoms) {  // too small to fit the dictionary: the bucket is skipped
                for (size_t i : pooled_segs) skip[i] = 1;
                continue;
            }
            Dict d;
            d.key = key;
            int rc = fit_tiles(pool, fill, tile_dim, key.n_atoms, key.n_stages, key.k, ksvd_iters,
                               gamma, d.atoms, nullptr, st);
            if (rc != CSDR_OK) return rc;
            const size_t di = dicts.size();
            dicts.push_back(std::move(d));
            for (size_t q = 0; q < pooled_segs.size(); ++q) {
                const size_t i = pooled_segs[q];
                Entry e;
                e.seg = i;
                e.dict = di;
                e.n_tiles = (rows[i] / tr) * (cols[i] / tc);
                rc = encode_tiles(seg_tiles[q].data(), e.n_tiles, tile_dim, dicts[di].atoms,
                                  key.n_atoms, key.n_stages, key.k, gamma, e.codes, st);
                if (rc != CSDR_OK) return rc;
                std::vector<float>().swap(seg_tiles[q]);
                entries.push_back(std::move(e));
            }
        }
        // SharedDictArchive::writeToStream (:1967-2002)
        std::vector<uint8_t> s;
        s.insert(s.end(), {'H', 'S', 'D', 'A'});
        put<uint32_t>(s, 1);
        put<uint32_t>(s, (uint32_t)dicts.size());
        put<uint32_t>(s, (uint32_t)entries.size());
        for (const Dict& d : dicts) {
            // the 20-byte HierarchicalSDRConfig (HierarchicalSDRStrategy.hpp:43-58); its two
            // padding bytes (10-11) written as zeros
            put<uint16_t>(s, d.key.tile_rows);
            put<uint16_t>(s, d.key.tile_cols);
            put<uint16_t>(s, d.key.n_atoms);
            put<uint8_t>(s, d.key.n_stages);
            put<uint8_t>(s, d.key.k);
            put<uint8_t>(s, ksvd_iters);
            put<uint8_t>(s, 0);  // reserved_pad
            put<uint16_t>(s, 0);
            put<float>(s, d.key.decay);
            put<uint32_t>(s, max_tiles_for_fit);
            put<uint32_t>(s, (uint32_t)gamma.size());
            for (float x : gamma) put<float>(s, x);
            put<uint32_t>(s, (uint32_t)d.atoms.size());
            for (float x : d.atoms) put<float>(s, x);
        }
        for (const Entry& e : entries) {
            const size_t i = e.seg;
            const std::string name = names[i];
            const GroupKey& key = dicts[e.dict].key;
            put<uint32_t>(s, (uint32_t)name.size());
            s.insert(s.end(), name.begin(), name.end());
            put<uint32_t>(s, (uint32_t)e.dict);
            put<uint64_t>(s, (uint64_t)rows[i] * cols[i] * 4);
            put<uint8_t>(s, original_types ? original_types[i] : (uint8_t)1);
            // compressFP32WithExternalDictionary's HSDC stream (:1732-1754): 32-byte header,
            // packed codes
            put<uint32_t>(s, (uint32_t)(32 + e.codes.size() * 2));
            s.insert(s.end(), {'H', 'S', 'D', 'C'});
            put<uint32_t>(s, 1);
            put<uint32_t>(s, rows[i]);
            put<uint32_t>(s, cols[i]);
            put<uint32_t>(s, e.n_tiles);
            put<uint16_t>(s, key.tile_rows);
            put<uint16_t>(s, key.tile_cols);
            put<uint16_t>(s, key.n_atoms);
            put<uint8_t>(s, key.n_stages);
            put<uint8_t>(s, key.k);
            put<float>(s, key.decay);
            for (uint16_t c : e.codes) put<uint16_t>(s, c);
        }
        uint8_t* buf = static_cast<uint8_t*>(std::malloc(std::max<size_t>(s.size(), 1)));
        if (!buf) return set_error(CSDR_E_INVALID, "hsda_build: out of host memory");
        std::memcpy(buf, s.data(), s.size());
        *out = buf;
        *out_size = s.size();
        if (skipped) std::memcpy(skipped, skip.data(), skip.size());
    } catch (const std::exception& ex) {
        return set_error(CSDR_E_INVALID, std::string("hsda_build: ") + ex.what());
    }
    return CSDR_OK;
}

CSDR_API void csdr_free_buffer(void* p) { std::free(p); }

}  // extern "C"
