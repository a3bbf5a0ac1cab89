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
//   * x / sqrt(s) as x * r with r = (y0 * (y0 * s) - 3) * (y0 * -0.5), y0 the approximate
//     reciprocal square root (x86 rsqrtss) and the inner product-sum fused: one Newton step.
//     rsqrtss differs between CPU models, and so does the reference's dictionary. y0 here is
//     that of the CPU the golden vectors were written on (an Intel Xeon: a function of the
//     exponent's parity and the top 10 mantissa bits, scaling by 2^-k for 4^k s; the table
//     comes from rsqrt_table_gen.c run there), so the dictionary is the same on every host;
//   * each tile's squared norm in double as the -O3 -ffast-math AVX2 build sums
//     `sq += (double)t[c] * t[c]` (gcc 11): four lanes taking 8 values per step, lane j adding
//     fma(t[c + j], t[c + j], t[c + 4 + j]^2), then (lane 0 + lane 2) + (lane 1 + lane 3); a
//     remaining group of 4 as fma(t0, t0, t2^2) + fma(t1, t1, t3^2); FMAs for the last values;
//   * the mean tile norm: those norms summed in tile order, divided by n (rounded to float
//     for the initialisation).
// The atom re-seeding of atomUpdateStep (:411-425, :461-474) is here too: a tile picked by a
// per-atom generator, its squared norm summed as above, scaled to the target norm in double.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>

#pragma clang fp contract(off)

namespace csdr {

namespace {

#include "hsdr_rsqrt_table.inc"

// The golden vectors' CPU's rsqrtss of a normal positive s
float rsqrt_approx(float s) {
    uint32_t b;
    std::memcpy(&b, &s, 4);
    const int e = (int)(b >> 23) - 127;
    const int p = e & 1;          // s = 4^k 2^p (1 + m / 2^23)
    const int k = (e - p) / 2;
    float y;
    std::memcpy(&y, &kRsqrtTable[p * 1024 + ((b >> 13) & 1023u)], 4);
    return std::ldexp(y, -k);
}

float rsqrt_newton(float s) {
    const float y0 = rsqrt_approx(s);
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

// sum_c (double)t[c]^2 in the order of the reference's vectorised loop (header)
double squared_norm_d(const float* t, uint32_t C) {
    double total = 0.0;
    uint32_t c = 0;
    if (C >= 8) {
        double a[4] = {0.0, 0.0, 0.0, 0.0};
        for (; c + 8 <= C; c += 8)
            for (int j = 0; j < 4; ++j) {
                const double lo = t[c + j], hi = t[c + 4 + j];
                a[j] = a[j] + std::fma(lo, lo, hi * hi);
            }
        total = (a[0] + a[2]) + (a[1] + a[3]);
    }
    if (C - c >= 4) {
        const double t0 = t[c], t1 = t[c + 1], t2 = t[c + 2], t3 = t[c + 3];
        const double e0 = std::fma(t0, t0, t2 * t2), e1 = std::fma(t1, t1, t3 * t3);
        total = total + (e0 + e1);
        c += 4;
    }
    for (; c < C; ++c) total = std::fma((double)t[c], (double)t[c], total);
    return total;
}

}  // namespace

// Mean of the tiles' Euclidean norms, in double (fitHierarchicalKSVD :529-536, atomUpdateStep
// :374-383): the norms summed in tile order, as the reference's OpenMP reduction does with
// one thread (with more, its per-thread partials change the last bits).
double hsdr_mean_tile_norm(const float* tiles, uint32_t n, uint32_t C) {
    double norm_sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) norm_sum += std::sqrt(squared_norm_d(tiles + (size_t)i * C, C));
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
    const double sq = squared_norm_d(src, C);
    const double s = target_norm / std::sqrt(std::max(sq, 1e-30));
    for (uint32_t c = 0; c < C; ++c) atom[c] = (float)((double)src[c] * s);
}

}  // namespace csdr
