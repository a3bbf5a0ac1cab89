// hsdr_init.cpp — the HSDR encoder's dictionary initialisation (host code, x86-64).
//
// Reference: fitHierarchicalKSVD (cortexSDR tree, src/ai_compression/strategies/
// HierarchicalSDRStrategy.cpp:507-541): atom j is the tile picked by
// std::uniform_int_distribution<uint32_t>(0, n - 1) over std::mt19937(0xC0DE), scaled to unit
// length; then every atom is scaled by mean_i ||tile_i|| / max(1, sqrt(S * k)).
//
// The reference is built with -O3 -ffast-math -mavx2 -mfma (its CMakeLists.txt), and its
// arithmetic here is what that build executes, restated operation by operation so that the
// dictionary is the reference's bit for bit on the same CPU:
//   * the squared norm of an atom: 8 FMA lanes over 8-element chunks, then the upper four
//     lanes added onto the lower, then lanes 2, 3 onto 0, 1, then lane 1 onto lane 0; a
//     4-element remainder as plain products summed (1 + 3) + (0 + 2) and added on; FMAs for
//     the last elements;
//   * x / sqrt(s) as x * r with r = (y0 * (y0 * s) - 3) * (y0 * -0.5), y0 the CPU's approximate
//     reciprocal square root (rsqrtss) and the inner product-sum fused: one Newton step.
//     rsqrtss differs between CPU models, and so does the reference's dictionary; this code
//     reproduces the reference on the CPU it runs on;
//   * the mean tile norm in double (FMA sums), divided by n, rounded to float.
// The atom re-seeding of atomUpdateStep (:411-425, :461-474) is here too: a tile picked by a
// per-atom generator, scaled to the target norm in double.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>

#pragma clang fp contract(off)

namespace csdr {

namespace {

float rsqrt_newton(float s) {
    const float y0 = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(s)));
    const float ys = y0 * s;
    const float t = std::fma(y0, ys, -3.0f);
    const float h = y0 * -0.5f;
    return t * h;
}

float squared_norm(const float* d, uint32_t C) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    uint32_t c = 0;
    for (; c + 8 <= C; c += 8)
        for (int l = 0; l < 8; ++l) v[l] = std::fma(d[c + l], d[c + l], v[l]);
    float h[4];
    for (int i = 0; i < 4; ++i) h[i] = v[i + 4] + v[i];
    const float a0 = h[2] + h[0], a1 = h[3] + h[1];
    float sq = a1 + a0;
    if (c + 4 <= C) {
        float p[4];
        for (int i = 0; i < 4; ++i) p[i] = d[c + i] * d[c + i];
        const float b0 = p[2] + p[0], b1 = p[3] + p[1];
        const float b = b1 + b0;
        sq = sq + b;
        c += 4;
    }
    for (; c < C; ++c) sq = std::fma(d[c], d[c], sq);
    return sq;
}

}  // namespace

// Mean of the tiles' Euclidean norms, in double (fitHierarchicalKSVD :529-536, atomUpdateStep
// :374-383, whose OpenMP reduction sums per-thread partials: its last bits follow the thread
// count).
double hsdr_mean_tile_norm(const float* tiles, uint32_t n, uint32_t C) {
    double norm_sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) {
        const float* t = tiles + (size_t)i * C;
        double sq = 0.0;
        for (uint32_t c = 0; c < C; ++c) sq = std::fma((double)t[c], (double)t[c], sq);
        norm_sum += std::sqrt(sq);
    }
    return norm_sum / (double)std::max<uint32_t>(1u, n);
}

void hsdr_init_dictionary(const float* tiles, uint32_t n, uint32_t C, uint16_t K,
                          uint32_t slots, float* D, std::mt19937* rng_io) {
    std::mt19937 local(0xC0DE);
    std::mt19937& rng = rng_io ? *rng_io : local;  // the fit's generator, seeded 0xC0DE
    std::uniform_int_distribution<uint32_t> pick(0, n - 1);
    for (uint32_t j = 0; j < K; ++j) {
        const uint32_t src = pick(rng);
        float* d = D + (size_t)j * C;
        std::memcpy(d, tiles + (size_t)src * C, sizeof(float) * C);
        const float r = rsqrt_newton(std::max(squared_norm(d, C), 1e-24f));
        for (uint32_t c = 0; c < C; ++c) d[c] = d[c] * r;
    }
    float scale = (float)(hsdr_mean_tile_norm(tiles, n, C));
    const float s = (float)slots;
    if (s > 1.0f) scale = scale * rsqrt_newton(s);
    for (size_t i = 0; i < (size_t)K * C; ++i) D[i] = D[i] * scale;
}

// atomUpdateStep's re-seed of atom j (:411-425 for an atom nobody uses, seed constant
// 0x9E3779B1; :461-474 for one whose update was not finite, 0xB7E15163; base_seed :403): the
// tile picked by
// std::mt19937((uint32_t)(base_seed ^ (j * mul))) over [0, n - 1], scaled to target_norm.
void hsdr_reseed_atom(const float* tiles, uint32_t n, uint32_t C, uint64_t base_seed, uint32_t j,
                      uint32_t mul, double target_norm, float* atom) {
    std::mt19937 local(static_cast<uint32_t>(base_seed ^ (uint64_t)(j * mul)));
    std::uniform_int_distribution<uint32_t> pick(0, n - 1);
    const float* src = tiles + (size_t)pick(local) * C;
    double sq = 0.0;
    for (uint32_t c = 0; c < C; ++c) sq = std::fma((double)src[c], (double)src[c], sq);
    const double s = target_norm / std::sqrt(std::max(sq, 1e-30));
    for (uint32_t c = 0; c < C; ++c) atom[c] = (float)((double)src[c] * s);
}

}  // namespace csdr
