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
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "common.hpp"

namespace csdr {
// fitHierarchicalKSVD's dictionary initialisation, in the reference build's arithmetic
// (hsdr_init.cpp).
void hsdr_init_dictionary(const float* tiles, uint32_t n, uint32_t C, uint16_t K, uint32_t slots,
                          float* D);
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

__global__ __launch_bounds__(kEThreads) void mp_kernel(MpArgs a) {
    extern __shared__ float smem[];
    const int tt = a.tt, C = a.C, K = a.K;
    const long long t0 = (long long)blockIdx.x * tt;
    const int nt = (int)min((long long)tt, a.n - t0);
    float* r = smem;                                                    // nt x C residuals
    float* proj = r + (size_t)tt * C;                                   // nt x K scores
    uint8_t* used = reinterpret_cast<uint8_t*>(proj + (size_t)tt * K);  // nt x K
    __shared__ int best_s[kMaxTT];
    __shared__ float scale_s[kMaxTT];
    const int tid = threadIdx.x, l16 = tid & 15, grp = tid >> 4;
    const int lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < nt * C; i += kEThreads) r[i] = a.tiles[t0 * C + i];
    const int C16 = C & ~15, C8 = C & ~7;  // end of the 16-element chunks, of the 8-element one
    const int slots = a.S * a.k;
    for (int l = 0; l < a.S; ++l) {
        for (int i = tid; i < nt * K; i += kEThreads) used[i] = 0;
        __syncthreads();
        for (int st = 0; st < a.k; ++st) {
            // 1. projections of every tile onto every atom
            for (int j = grp; j < K; j += kEGroups) {
                const float* dj = a.D + (size_t)j * C;
                float p[kMaxTT];
#pragma unroll
                for (int t = 0; t < kMaxTT; ++t) p[t] = 0.f;
                for (int c = l16; c < C16; c += 16) {
                    const float dv = dj[c];
#pragma unroll
                    for (int t = 0; t < kMaxTT; ++t)
                        if (t < nt) p[t] = fmaf(dv, r[t * C + c], p[t]);
                }
                if (C8 > C16 && l16 < 8) {
                    const int c = C16 + l16;
                    const float dv = dj[c];
#pragma unroll
                    for (int t = 0; t < kMaxTT; ++t)
                        if (t < nt) p[t] = fmaf(dv, r[t * C + c], p[t]);
                }
#pragma unroll
                for (int t = 0; t < kMaxTT; ++t) {
                    float v = p[t];
                    v += __shfl_xor(v, 8, 16);  // acc0 + acc1
                    v += __shfl_xor(v, 4, 16);  // low + high 128 bits
                    v += __shfl_xor(v, 1, 16);  // horizontal add
                    v += __shfl_xor(v, 2, 16);  // horizontal add
                    p[t] = v;
                }
                if (l16 == 0) {
#pragma unroll
                    for (int t = 0; t < kMaxTT; ++t)
                        if (t < nt) proj[t * K + j] = used[t * K + j] ? 0.0f : p[t];
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
                r[i] = fmaf(-a.D[(size_t)best_s[t] * C + c], scale_s[t], r[i]);
            }
            __syncthreads();
        }
    }
}

size_t mp_lds_bytes(int tt, int C, int K) {
    return (size_t)tt * ((size_t)C + K) * 4 + csdr::align_up((size_t)tt * K, 16);
}

// Tiles per workgroup: as many as fit (up to 8) under the soft LDS size, else one tile under
// the hard one, else 0 (too large).
int mp_tiles_per_wg(int C, int K) {
    for (int tt = kMaxTT; tt >= 1; --tt)
        if (mp_lds_bytes(tt, C, K) <= kLdsSoft) return tt;
    return mp_lds_bytes(1, C, K) <= kLdsHard ? 1 : 0;
}

int check_mp_shape(long long n, int C, int K, int S, int k) {
    if (n < 0 || C <= 0 || K <= 0 || S <= 0 || k <= 0)
        return set_error(CSDR_E_INVALID, "hsdr_encode: bad shape");
    if (C % 8)
        return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: tile size must be a multiple of 8");
    if (K > 32768) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: at most 32768 atoms");
    if (S > kMaxStages) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: at most 32 stages");
    if (k > K) return set_error(CSDR_E_INVALID, "hsdr_encode: more picks per stage than atoms");
    if (mp_tiles_per_wg(C, K) == 0)
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
    a.tt = mp_tiles_per_wg(C, K);
    for (int l = 0; l < S; ++l) a.gamma[l] = gamma[l];
    const size_t lds = mp_lds_bytes(a.tt, C, K);
    if (lds > 64 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&mp_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    const long long grid = (n + a.tt - 1) / a.tt;
    if (grid > 0x7fffffffLL) return set_error(CSDR_E_UNSUPPORTED, "hsdr_encode: too many tiles");
    mp_kernel<<<(unsigned)grid, kEThreads, lds, st>>>(a);
    CSDR_LAUNCH_CHECK("hsdr_encode");
    return CSDR_OK;
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

template <class T>
void put(std::vector<uint8_t>& out, const T& v) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
    out.insert(out.end(), p, p + sizeof(T));
}

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
                               (uint32_t)n_stages * k_per_stage, D);
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
    if (ksvd_iters != 0)
        return set_error(CSDR_E_UNSUPPORTED, "hsdr_compress: K-SVD refinement not built");
    rc = check_mp_shape(g.n_tiles, (int)g.tile_dim, g.K, g.S, g.k);
    if (rc != CSDR_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);

    // tiles in row-major tile order (extractTiles :94-116) of the aligned block
    const uint32_t nrt = g.R_full / g.tr, nct = g.C_full / g.tc;
    std::vector<float> tiles((size_t)g.n_tiles * g.tile_dim);
    for (uint32_t br = 0; br < nrt; ++br)
        for (uint32_t bc = 0; bc < nct; ++bc) {
            float* dst = tiles.data() + (size_t)(br * nct + bc) * g.tile_dim;
            for (uint32_t r = 0; r < g.tr; ++r)
                std::memcpy(dst + (size_t)r * g.tc,
                            w + (size_t)(br * g.tr + r) * g.C + (size_t)bc * g.tc,
                            sizeof(float) * g.tc);
        }
    std::vector<float> gamma(g.S), D;
    for (uint32_t l = 0; l < g.S; ++l) gamma[l] = std::pow(stage_decay, (float)l);
    D.assign((size_t)g.K * g.tile_dim, 0.0f);
    csdr::hsdr_init_dictionary(tiles.data(), g.n_tiles, g.tile_dim, g.K, (uint32_t)g.S * g.k,
                               D.data());

    const size_t slots = (size_t)g.S * g.k, ncodes = (size_t)g.n_tiles * slots;
    std::vector<uint16_t> codes(ncodes);
    float *d_tiles = nullptr, *d_D = nullptr;
    uint16_t* d_codes = nullptr;
    auto cleanup = [&] {
        if (d_tiles) (void)hipFree(d_tiles);
        if (d_D) (void)hipFree(d_D);
        if (d_codes) (void)hipFree(d_codes);
    };
    auto hip_fail = [&](hipError_t e, const char* what) {
        cleanup();
        return set_error(CSDR_E_HIP, std::string("hsdr_compress: ") + what + ": " +
                                         hipGetErrorString(e));
    };
    hipError_t e;
    if ((e = hipMalloc(&d_tiles, tiles.size() * 4)) != hipSuccess) return hip_fail(e, "malloc");
    if ((e = hipMalloc(&d_D, D.size() * 4)) != hipSuccess) return hip_fail(e, "malloc");
    if ((e = hipMalloc(&d_codes, std::max<size_t>(ncodes * 2, 2))) != hipSuccess)
        return hip_fail(e, "malloc");
    if ((e = hipMemcpyAsync(d_tiles, tiles.data(), tiles.size() * 4, hipMemcpyHostToDevice,
                            st)) != hipSuccess)
        return hip_fail(e, "upload");
    if ((e = hipMemcpyAsync(d_D, D.data(), D.size() * 4, hipMemcpyHostToDevice, st)) !=
        hipSuccess)
        return hip_fail(e, "upload");
    rc = launch_mp(d_tiles, g.n_tiles, (int)g.tile_dim, d_D, g.K, g.S, g.k, gamma.data(),
                   d_codes, st);
    if (rc != CSDR_OK) {
        cleanup();
        return rc;
    }
    if ((e = hipMemcpyAsync(codes.data(), d_codes, ncodes * 2, hipMemcpyDeviceToHost, st)) !=
        hipSuccess)
        return hip_fail(e, "download");
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(e, "synchronize");
    cleanup();
    for (float& x : D)  // the fit's final sanitisation (:592-601)
        if (!std::isfinite(x)) x = 0.0f;

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

}  // extern "C"
