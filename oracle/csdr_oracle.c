/*
 * csdr_oracle.c — CPU restatement of cortexSDR's compressed-weight inference path.
 *
 * TEST INFRASTRUCTURE ONLY (see csdr_oracle.h): the checker for tests/, smoke() and
 * bench.py's cpu_baseline leg. Never linked into the product.
 *
 * Arithmetic: built with -ffp-contract=off; every multiply-add that the reference
 * performs as `acc += a * b` inside a loop is written here as fmaf(a, b, acc) in the
 * reference's loop order, so that dense decodes can be compared bit-exactly with the
 * reference built by oracle/Makefile (its -O3 -mfma build contracts the same
 * expressions into FMAs).
 */
#include "csdr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

float orc_f16_to_f32(uint16_t h) {
    /* utils/fp16_convert.hpp:33-60 (bit-level decode incl. subnormals, inf, nan) */
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = sign << 31;
        } else {
            int ex = 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                ex--;
            }
            m &= 0x3FFu;
            f = (sign << 31) | ((uint32_t)(ex + 112) << 23) | (m << 13);
        }
    } else if (e == 0x1F) {
        f = (sign << 31) | 0x7F800000u | (m << 13);
    } else {
        f = (sign << 31) | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

uint16_t orc_f32_to_f16(float fv) {
    /* IEEE-754 binary16, round to nearest, ties to even (the F16C path of
     * utils/fp16_convert.hpp:68-71). Subnormals are produced, not flushed. */
    uint32_t x;
    memcpy(&x, &fv, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) { /* inf or nan */
        if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (absx < 0x38800000u) {                                   /* below 2^-14: subnormal */
        if (absx < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); unit = 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u;
    uint32_t m = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

/* ---------------------------------------------------------- stream parse */

static uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

int orc_hsdr_parse(const uint8_t* buf, size_t n, orc_hsdr_view* v) {
    /* Header layout: HierarchicalSDRStrategy.cpp:49-66 (packed, 36 bytes). */
    if (!buf || !v) return ORC_E_ARG;
    memset(v, 0, sizeof(*v));
    if (n < 36) return ORC_E_TRUNCATED;
    if (memcmp(buf, "HSDR", 4) == 0) {
        v->is_hsdb = 0;
    } else if (memcmp(buf, "HSDB", 4) == 0) {
        v->is_hsdb = 1;
    } else {
        return ORC_E_MAGIC; /* :1266-1268 */
    }
    v->version = rd32(buf + 4);
    if ((!v->is_hsdb && v->version != 2) || (v->is_hsdb && v->version != 1))
        return ORC_E_VERSION; /* :1269-1271 */
    v->rows = rd32(buf + 8);
    v->cols = rd32(buf + 12);
    v->n_tiles = rd32(buf + 16);
    v->tile_rows = rd16(buf + 20);
    v->tile_cols = rd16(buf + 22);
    v->n_atoms = rd16(buf + 24);
    v->n_stages = buf[26];
    v->k_per_stage = buf[27];
    memcpy(&v->stage_decay, buf + 28, 4);
    v->edge_bytes = rd32(buf + 32);
    if (v->tile_rows == 0 || v->tile_cols == 0) return ORC_E_GEOMETRY;
    if (v->is_hsdb && v->tile_rows != 1) return ORC_E_GEOMETRY;
    {
        uint64_t rf = (uint64_t)(v->rows / v->tile_rows) * v->tile_rows;
        uint64_t cf = (uint64_t)(v->cols / v->tile_cols) * v->tile_cols;
        uint64_t expect_tiles = (rf / v->tile_rows) * (cf / v->tile_cols);
        if (expect_tiles != v->n_tiles) return ORC_E_GEOMETRY;
        uint64_t expect_edge = (rf * (v->cols - cf) + (v->rows - rf) * (uint64_t)v->cols) * 4u;
        if (expect_edge != v->edge_bytes) return ORC_E_GEOMETRY;
    }
    v->slots_per_tile = (size_t)v->n_stages * v->k_per_stage;
    v->n_codes = (size_t)v->n_tiles * v->slots_per_tile;
    size_t tile_dim = (size_t)v->tile_rows * v->tile_cols;
    size_t off = 36;
    v->off_gamma = off;
    off += 4u * v->n_stages;
    v->off_dict = off;
    off += 4u * (size_t)v->n_atoms * tile_dim;
    v->off_packed = off;
    off += 2u * v->n_codes;
    v->off_coef = off;
    if (v->is_hsdb) off += 2u * v->n_codes;
    v->off_edge = off;
    off += v->edge_bytes;
    v->end = off;
    if (off > n) return ORC_E_TRUNCATED; /* readBuffer, :218-225 */
    return ORC_OK;
}

int orc_hsdr_unpack(const uint8_t* buf, size_t n, uint16_t* idx, int8_t* sign, float* coef) {
    orc_hsdr_view v;
    int rc = orc_hsdr_parse(buf, n, &v);
    if (rc) return rc;
    for (size_t i = 0; i < v.n_codes; ++i) {
        uint16_t p = rd16(buf + v.off_packed + 2 * i);
        size_t slot = i % v.slots_per_tile;
        size_t l = slot / v.k_per_stage;
        float g;
        memcpy(&g, buf + v.off_gamma + 4 * l, 4);
        int8_t s = (p & 0x8000u) ? -1 : 1; /* :81-84 */
        if (idx) idx[i] = (uint16_t)(p & 0x7FFFu);
        if (sign) sign[i] = s;
        if (coef) {
            float mag = v.is_hsdb ? orc_f16_to_f32(rd16(buf + v.off_coef + 2 * i)) : 1.0f;
            coef[i] = g * ((float)s * mag); /* scale = gamma * sign, :627 */
        }
    }
    return ORC_OK;
}

/* Copies the dictionary (n_atoms x tile_dim fp32) out of the stream. */
static float* copy_dict(const uint8_t* buf, const orc_hsdr_view* v) {
    size_t nf = (size_t)v->n_atoms * v->tile_rows * v->tile_cols;
    float* D = (float*)malloc(nf * 4 + 4);
    if (D) memcpy(D, buf + v->off_dict, nf * 4);
    return D;
}

int orc_hsdr_decompress(const uint8_t* buf, size_t n, float* out, size_t out_floats) {
    orc_hsdr_view v;
    int rc = orc_hsdr_parse(buf, n, &v);
    if (rc) return rc;
    const size_t R = v.rows, C = v.cols;
    if (out_floats < R * C) return ORC_E_ARG; /* originalSize check, :1371-1374 */
    const size_t tr = v.tile_rows, tc = v.tile_cols, tile_dim = tr * tc;
    const size_t R_full = (R / tr) * tr, C_full = (C / tc) * tc;
    const size_t n_col_tiles = C_full / tc;
    float* D = copy_dict(buf, &v);
    float* coef = (float*)malloc(v.n_codes * 4 + 4);
    uint16_t* idx = (uint16_t*)malloc(v.n_codes * 2 + 2);
    if (!D || !coef || !idx) {
        free(D), free(coef), free(idx);
        return ORC_E_ARG;
    }
    orc_hsdr_unpack(buf, n, idx, NULL, coef);
    /* tiles are decoded independently (each element's slot order is the reference's), so
     * they run in parallel */
#pragma omp parallel
    {
        float* tile = (float*)malloc(tile_dim * 4);
#pragma omp for schedule(static)
        for (long long tt = 0; tt < (long long)v.n_tiles; ++tt) {
            const size_t t = (size_t)tt;
            /* decodeAllTiles, :612-634: zero tile, then stage-major slot accumulation */
            for (size_t c = 0; c < tile_dim; ++c) tile[c] = 0.0f;
            for (size_t s = 0; s < v.slots_per_tile; ++s) {
                size_t slot = t * v.slots_per_tile + s;
                const float scale = coef[slot];
                /* the reference's sign-0 skip (:626) never fires: unpacked signs are +-1 */
                if (idx[slot] >= v.n_atoms) continue; /* out of range: reference reads past D */
                const float* atom = D + (size_t)idx[slot] * tile_dim;
                for (size_t c = 0; c < tile_dim; ++c) tile[c] = fmaf(scale, atom[c], tile[c]);
            }
            /* reassembleTiles, :119-135: tile (br, bc) -> rows br*tr.., cols bc*tc.. */
            size_t br = t / n_col_tiles, bc = t % n_col_tiles;
            for (size_t r = 0; r < tr; ++r)
                memcpy(out + (br * tr + r) * C + bc * tc, tile + r * tc, tc * 4);
        }
        free(tile);
    }
    /* edge splice: top-right strip then bottom strip, :1401-1438 */
    size_t e = 0;
    const uint8_t* eb = buf + v.off_edge;
    for (size_t r = 0; r < R_full; ++r)
        for (size_t c = C_full; c < C; ++c, ++e) memcpy(out + r * C + c, eb + 4 * e, 4);
    for (size_t r = R_full; r < R; ++r)
        for (size_t c = 0; c < C; ++c, ++e) memcpy(out + r * C + c, eb + 4 * e, 4);
    free(D), free(coef), free(idx);
    return ORC_OK;
}

int orc_hsdr_matmul_row_major(const uint8_t* buf, size_t n, const float* x, size_t batch,
                              float* y) {
    orc_hsdr_view v;
    int rc = orc_hsdr_parse(buf, n, &v);
    if (rc) return rc;
    if (v.is_hsdb) return ORC_E_MAGIC;
    /* :1273-1289 geometry checks */
    if (v.tile_rows != 1 || v.tile_cols != v.cols || v.n_tiles != v.rows) return ORC_E_GEOMETRY;
    const size_t R = v.rows, C = v.cols, K = v.n_atoms;
    float* D = copy_dict(buf, &v);
    float* Dx = (float*)calloc(K * batch + 1, 4);
    float* coef = (float*)malloc(v.n_codes * 4 + 4);
    uint16_t* idx = (uint16_t*)malloc(v.n_codes * 2 + 2);
    if (!D || !Dx || !coef || !idx) {
        free(D), free(Dx), free(coef), free(idx);
        return ORC_E_ARG;
    }
    orc_hsdr_unpack(buf, n, idx, NULL, coef);
    /* hot loop 1, :1304-1315: Dx[a, b] = sum_c D[a, c] * x[c, b] */
    for (size_t a = 0; a < K; ++a)
        for (size_t c = 0; c < C; ++c) {
            const float av = D[a * C + c];
            for (size_t b = 0; b < batch; ++b)
                Dx[a * batch + b] = fmaf(av, x[c * batch + b], Dx[a * batch + b]);
        }
    /* hot loop 2, :1318-1336: per-row signed gather */
    for (size_t r = 0; r < R; ++r) {
        float* yr = y + r * batch;
        for (size_t b = 0; b < batch; ++b) yr[b] = 0.0f;
        for (size_t s = 0; s < v.slots_per_tile; ++s) {
            size_t slot = r * v.slots_per_tile + s;
            if (idx[slot] >= K) continue;
            const float scale = coef[slot];
            const float* dx = Dx + (size_t)idx[slot] * batch;
            for (size_t b = 0; b < batch; ++b) yr[b] = fmaf(scale, dx[b], yr[b]);
        }
    }
    free(D), free(Dx), free(coef), free(idx);
    return ORC_OK;
}

int orc_hsdb_matmul(const uint8_t* buf, size_t n, const float* x, size_t M, float* y) {
    orc_hsdr_view v;
    int rc = orc_hsdr_parse(buf, n, &v);
    if (rc) return rc;
    if (v.tile_rows != 1) return ORC_E_GEOMETRY;
    const size_t R = v.rows, C = v.cols, K = v.n_atoms, B = v.tile_cols;
    const size_t NB = C / B, C_full = NB * B, S = v.slots_per_tile;
    float* D = copy_dict(buf, &v);
    float* coef = (float*)malloc(v.n_codes * 4 + 4);
    uint16_t* idx = (uint16_t*)malloc(v.n_codes * 2 + 2);
    float* Dx = (float*)malloc(NB * K * M * 4 + 4);
    if (!D || !coef || !idx || !Dx) {
        free(D), free(coef), free(idx), free(Dx);
        return ORC_E_ARG;
    }
    orc_hsdr_unpack(buf, n, idx, NULL, coef);
    /* impl_fused_real, benchmark.py:117-118: Dx_b = D @ x_block, per block column b */
#pragma omp parallel for schedule(static)
    for (long long ba = 0; ba < (long long)(NB * K); ++ba) {
        size_t b = (size_t)ba / K, a = (size_t)ba % K;
        float* o = Dx + (b * K + a) * M;
        for (size_t m = 0; m < M; ++m) o[m] = 0.0f;
        for (size_t t = 0; t < B; ++t) {
            const float dv = D[a * B + t];
            const float* xr = x + (b * B + t) * M;
            for (size_t m = 0; m < M; ++m) o[m] = fmaf(dv, xr[m], o[m]);
        }
    }
    /* benchmark.py:122-127: tile (r, b) contributes its code row times Dx_b to row r;
     * tile (r, b) sits at index r*NB + b (HierarchicalSDRStrategy.cpp:101-104). */
#pragma omp parallel for schedule(static)
    for (long long rr = 0; rr < (long long)R; ++rr) {
        size_t r = (size_t)rr;
        float* yr = y + r * M;
        for (size_t m = 0; m < M; ++m) yr[m] = 0.0f;
        for (size_t b = 0; b < NB; ++b) {
            const size_t t = r * NB + b;
            for (size_t s = 0; s < S; ++s) {
                const size_t slot = t * S + s;
                if (idx[slot] >= K) continue;
                const float cf = coef[slot];
                const float* dx = Dx + (b * K + idx[slot]) * M;
                for (size_t m = 0; m < M; ++m) yr[m] = fmaf(cf, dx[m], yr[m]);
            }
        }
        /* edge strip (cols C_full..C of row r), fp32 verbatim */
        const size_t ce = C - C_full;
        for (size_t c = 0; c < ce; ++c) {
            float ev;
            memcpy(&ev, buf + v.off_edge + 4 * (r * ce + c), 4);
            const float* xr = x + (C_full + c) * M;
            for (size_t m = 0; m < M; ++m) yr[m] = fmaf(ev, xr[m], yr[m]);
        }
    }
    free(D), free(coef), free(idx), free(Dx);
    return ORC_OK;
}

/* --------------------------------------------------------------- K-quants */

/* ggufGetScaleMinQ4K, SparseInferenceEngine.cpp:266-274 (identical bit layout to
 * unpack_k_scales_mins, HierarchicalSDRStrategy.cpp:802-814). */
static void q4k_scale_min(const uint8_t* sc12, int j, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = sc12[j] & 0x3Fu;
        *mn = sc12[j + 4] & 0x3Fu;
    } else {
        *sc = (uint8_t)((sc12[j + 4] & 0x0Fu) | ((sc12[j - 4] >> 6) << 4));
        *mn = (uint8_t)((sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4));
    }
}

void orc_q4k_dequant(const uint8_t* blocks, size_t n_blocks, int order, float* out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* p = blocks + b * 144;
        const float d = orc_f16_to_f32(rd16(p));
        const float dmin = orc_f16_to_f32(rd16(p + 2));
        const uint8_t* sc12 = p + 4;
        const uint8_t* qs = p + 16;
        float* o = out + b * 256;
        for (int is = 0; is < 8; ++is) {
            uint8_t sc, mn;
            q4k_scale_min(sc12, is, &sc, &mn);
            const float ds = d * (float)sc;
            const float dm = dmin * (float)mn;
            for (int j = 0; j < 32; ++j) {
                uint8_t q;
                if (order == ORC_Q4K_GGML) {
                    /* SparseInferenceEngine.cpp:375-382: group g = is/2 holds 32 bytes;
                     * even sub-block = low nibbles, odd = high nibbles */
                    const uint8_t byte = qs[(is / 2) * 32 + j];
                    q = (is & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0Fu);
                } else {
                    /* HierarchicalSDRStrategy.cpp:840-845 */
                    const int idx = is * 32 + j;
                    const uint8_t byte = qs[idx / 2];
                    q = (idx & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0Fu);
                }
                o[is * 32 + j] = (float)q * ds - dm;
            }
        }
    }
}

void orc_q5k_dequant(const uint8_t* blocks, size_t n_blocks, float* out) {
    /* HierarchicalSDRStrategy.cpp:851-885 */
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* p = blocks + b * 176;
        const float d = orc_f16_to_f32(rd16(p));
        const float dmin = orc_f16_to_f32(rd16(p + 2));
        const uint8_t* sc12 = p + 4;
        const uint8_t* qh = p + 16;
        const uint8_t* qs = qh + 32;
        for (int is = 0; is < 8; ++is) {
            uint8_t sc, mn;
            q4k_scale_min(sc12, is, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            for (int j = 0; j < 32; ++j) {
                const int idx = is * 32 + j;
                const uint8_t byte = qs[idx / 2];
                const uint8_t lo = (idx & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0Fu);
                const uint8_t hi = (uint8_t)((qh[idx / 8] >> (idx % 8)) & 1u);
                out[b * 256 + idx] = (float)((hi << 4) | lo) * ds - dm;
            }
        }
    }
}

void orc_q6k_dequant(const uint8_t* blocks, size_t n_blocks, float* out) {
    /* HierarchicalSDRStrategy.cpp:888-933 (interleaved nibble / 2-bit order) */
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* p = blocks + b * 210;
        const uint8_t* ql = p;
        const uint8_t* qh = p + 128;
        const int8_t* scales = (const int8_t*)(p + 192);
        const float d = orc_f16_to_f32(rd16(p + 208));
        for (int half = 0; half < 2; ++half) {
            for (int sub = 0; sub < 8; ++sub) {
                const float ds = d * (float)scales[half * 8 + sub];
                for (int j = 0; j < 16; ++j) {
                    const int e = sub * 16 + j;
                    const uint8_t qb = ql[half * 64 + e / 2];
                    const uint8_t lo = (e & 1) ? (uint8_t)(qb >> 4) : (uint8_t)(qb & 0x0Fu);
                    const uint8_t hi = (uint8_t)((qh[half * 32 + e / 4] >> ((e % 4) * 2)) & 3u);
                    out[b * 256 + half * 128 + e] = (float)(((hi << 4) | lo) - 32) * ds;
                }
            }
        }
    }
}

int orc_q4k_linear(const uint8_t* w, size_t R, size_t C, int order, const float* x, size_t M,
                   float* y) {
    if (C % 256) return ORC_E_GEOMETRY;
    const size_t nb = C / 256;
    /* decode (SparseInferenceEngine.cpp:362-384), then out[m, r] = sum_c in[m, c] * W[r, c]
     * (blas_kernels.cpp:264-293 / BLAS-less row loop :101-143) */
#pragma omp parallel
    {
        float* row = (float*)malloc(C * 4);
#pragma omp for schedule(static)
        for (long long rr = 0; rr < (long long)R; ++rr) {
            size_t r = (size_t)rr;
            orc_q4k_dequant(w + r * nb * 144, nb, order, row);
            for (size_t m = 0; m < M; ++m) {
                float acc = 0.0f;
                const float* xm = x + m * C;
                for (size_t c = 0; c < C; ++c) acc = fmaf(xm[c], row[c], acc);
                y[m * R + r] = acc;
            }
        }
        free(row);
    }
    return ORC_OK;
}

/* --------------------------------------------------------------- engine GGUF formats */

/* decodeSupportedGGUFQuantized (SparseInferenceEngine.cpp:276-469) with the block sizes of
 * ggufBlockBytesForFormat / ggufBlockElementsForFormat / ggufQuantBitsForFormat (:181-252).
 * Format ids are ggml's type numbers (as include/cortexsdr_hip.h CSDR_GGUF_*). bits > 0 marks
 * a format decoded by the reference's generic rule (:439-465). */
static int gguf_table(int fmt, int* bb, int* be, int* bits) {
    static const int T[][4] = {
        {2, 18, 32, 0},    {3, 20, 32, 0},    {6, 22, 32, 0},    {7, 24, 32, 0},
        {8, 34, 32, 0},    {9, 40, 32, 0},    {10, 84, 256, 2},  {11, 110, 256, 3},
        {12, 144, 256, 0}, {13, 176, 256, 5}, {14, 210, 256, 0}, {15, 292, 256, 0},
        {16, 66, 256, 2},  {17, 74, 256, 2},  {18, 98, 256, 3},  {19, 50, 256, 1},
        {20, 18, 32, 4},   {21, 110, 256, 3}, {22, 82, 256, 2},  {23, 136, 256, 4},
        {29, 56, 256, 1},  {31, 72, 128, 4},  {32, 144, 256, 4}, {33, 144, 256, 4},
        {34, 54, 256, 1},  {35, 66, 256, 2}};
    for (size_t i = 0; i < sizeof(T) / sizeof(T[0]); ++i)
        if (T[i][0] == fmt) {
            *bb = T[i][1];
            *be = T[i][2];
            *bits = T[i][3];
            return 0;
        }
    return -1;
}

int orc_gguf_block(int fmt, int* block_bytes, int* block_elems) {
    int bits;
    return gguf_table(fmt, block_bytes, block_elems, &bits) ? ORC_E_GEOMETRY : ORC_OK;
}

static uint32_t packed_bits_lsb(const uint8_t* bytes, size_t bit_offset, size_t count) {
    /* readPackedBitsLSB, SparseInferenceEngine.cpp:254-264 */
    uint32_t v = 0;
    for (size_t b = 0; b < count; ++b) {
        const size_t a = bit_offset + b;
        v |= (uint32_t)((bytes[a / 8] >> (a % 8)) & 1u) << b;
    }
    return v;
}

int orc_gguf_dequant(const uint8_t* blocks, int fmt, size_t n_blocks, float* out) {
    int bb, be, bits;
    if (gguf_table(fmt, &bb, &be, &bits)) return ORC_E_GEOMETRY;
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* p = blocks + b * (size_t)bb;
        float* o = out + b * (size_t)be;
        if (bits) { /* :439-465 */
            const size_t packed = ((size_t)be * bits + 7) / 8;
            const uint8_t* data = p + (bb - packed);
            float d = orc_f16_to_f32(rd16(p));
            if (!isfinite(d) || fabsf(d) < 1e-12f) d = 1.0f;
            const int32_t centre = (int32_t)(1u << (bits - 1));
            for (int i = 0; i < be; ++i)
                o[i] = (float)((int32_t)packed_bits_lsb(data, (size_t)i * bits, bits) - centre) * d;
            continue;
        }
        switch (fmt) {
            case 8: { /* q8_0, :310-316 */
                const float d = orc_f16_to_f32(rd16(p));
                for (int i = 0; i < 32; ++i) o[i] = (float)(int8_t)p[2 + i] * d;
                break;
            }
            case 9: { /* q8_1, :319-326: the scale read as fp32 */
                float d;
                memcpy(&d, p, 4);
                for (int i = 0; i < 32; ++i) o[i] = (float)(int8_t)p[8 + i] * d;
                break;
            }
            case 14: { /* q6_k, :329-359 */
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = (const int8_t*)(p + 192);
                const float d = orc_f16_to_f32(rd16(p + 208));
                int k = 0;
                for (int half = 0; half < 2; ++half) {
                    const uint8_t* qlh = ql + half * 64;
                    const uint8_t* qhh = qh + half * 32;
                    const int8_t* sh = sc + half * 8;
                    for (int l = 0; l < 32; ++l)
                        o[k++] = d * (float)(sh[0] * ((int)((qlh[l] & 0x0F) | (((qhh[l] >> 0) & 3) << 4)) - 32));
                    for (int l = 0; l < 32; ++l)
                        o[k++] = d * (float)(sh[2] * ((int)((qlh[l + 32] & 0x0F) | (((qhh[l] >> 2) & 3) << 4)) - 32));
                    for (int l = 0; l < 32; ++l)
                        o[k++] = d * (float)(sh[4] * ((int)(((qlh[l] >> 4) & 0x0F) | (((qhh[l] >> 4) & 3) << 4)) - 32));
                    for (int l = 0; l < 32; ++l)
                        o[k++] = d * (float)(sh[6] * ((int)(((qlh[l + 32] >> 4) & 0x0F) | (((qhh[l] >> 6) & 3) << 4)) - 32));
                }
                break;
            }
            case 12: /* q4_k, :362-384 (ggml order) */
                orc_q4k_dequant(p, 1, ORC_Q4K_GGML, o);
                break;
            case 15: { /* q8_k, :387-395: fp16 scale, quants at byte 4 */
                const float d = orc_f16_to_f32(rd16(p));
                for (int i = 0; i < 256; ++i) o[i] = (float)(int8_t)p[4 + i] * d;
                break;
            }
            case 2: { /* q4_0, :398-406 */
                const float d = orc_f16_to_f32(rd16(p));
                for (int i = 0; i < 32; ++i) {
                    const uint8_t nb = (i & 1) == 0 ? (p[2 + i / 2] & 0x0F) : (p[2 + i / 2] >> 4);
                    o[i] = ((float)nb - 8.0f) * d;
                }
                break;
            }
            case 3: { /* q4_1, :408-417 (x * d + m as one fused multiply-add) */
                const float d = orc_f16_to_f32(rd16(p)), m = orc_f16_to_f32(rd16(p + 2));
                for (int i = 0; i < 32; ++i) {
                    const uint8_t nb = (i & 1) == 0 ? (p[4 + i / 2] & 0x0F) : (p[4 + i / 2] >> 4);
                    o[i] = fmaf((float)nb, d, m);
                }
                break;
            }
            case 6:
            case 7: { /* q5_0 / q5_1, :419-436 */
                const int has_m = fmt == 7;
                const float d = orc_f16_to_f32(rd16(p));
                const float m = has_m ? orc_f16_to_f32(rd16(p + 2)) : 0.0f;
                const uint8_t* qh = p + (has_m ? 4 : 2);
                const uint8_t* qs = p + (has_m ? 8 : 6);
                const uint32_t hb = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) |
                                    ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
                for (int i = 0; i < 32; ++i) {
                    uint8_t q = (i & 1) == 0 ? (qs[i / 2] & 0x0F) : (qs[i / 2] >> 4);
                    q |= (uint8_t)(((hb >> i) & 1u) << 4);
                    o[i] = has_m ? fmaf((float)q, d, m) : ((float)q - 16.0f) * d;
                }
                break;
            }
            default:
                return ORC_E_GEOMETRY;
        }
    }
    return ORC_OK;
}

int orc_gguf_linear(const uint8_t* w, int fmt, size_t R, size_t C, const float* x, size_t M,
                    float* y) {
    int bb, be, bits;
    if (gguf_table(fmt, &bb, &be, &bits) || C % (size_t)be) return ORC_E_GEOMETRY;
    const size_t nb = C / (size_t)be;
    /* decode, then out[m, r] = sum_c in[m, c] * W[r, c] (blas_kernels.cpp:264-293) */
    int rc = ORC_OK;
#pragma omp parallel
    {
        float* row = (float*)malloc(C * 4);
#pragma omp for schedule(static)
        for (long long rr = 0; rr < (long long)R; ++rr) {
            const size_t r = (size_t)rr;
            if (orc_gguf_dequant(w + r * nb * (size_t)bb, fmt, nb, row)) rc = ORC_E_GEOMETRY;
            for (size_t m = 0; m < M; ++m) {
                float acc = 0.0f;
                const float* xm = x + m * C;
                for (size_t c = 0; c < C; ++c) acc = fmaf(xm[c], row[c], acc);
                y[m * R + r] = acc;
            }
        }
        free(row);
    }
    return rc;
}

/* --------------------------------------------------------------- attention */

static void softmax_row(float* s, size_t n) {
    /* simd_kernels.cpp softmax: subtract max, exp, normalise */
    float mx = -INFINITY;
    for (size_t i = 0; i < n; ++i)
        if (s[i] > mx) mx = s[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        s[i] = expf(s[i] - mx);
        sum += s[i];
    }
    for (size_t i = 0; i < n; ++i) s[i] /= sum;
}

void orc_mha_causal(const float* q, const float* k, const float* v, float* out, size_t B,
                    size_t T, size_t hidden, size_t heads) {
    /* attention_kernels.cpp:26-113. Each output element sums over positions j in ascending
     * order with fmaf (the V loop runs j-outer over a row of accumulators: the same order per
     * element); queries are independent, so they run in parallel. */
    const size_t d = hidden / heads;
    const float scale = 1.0f / sqrtf((float)d);
    const long long n = (long long)(B * heads * T);
#pragma omp parallel
    {
        float* sc = (float*)malloc(T * 4 + 4);
        float* acc = (float*)malloc(d * 4 + 4);
#pragma omp for schedule(static)
        for (long long it = 0; it < n; ++it) {
            const size_t i = (size_t)it % T, h = ((size_t)it / T) % heads,
                         b = (size_t)it / (T * heads);
            const float* qi = q + (b * T + i) * hidden + h * d;
            for (size_t j = 0; j < T; ++j) {
                const float* kj = k + (b * T + j) * hidden + h * d;
                float a = 0.0f;
                for (size_t t = 0; t < d; ++t) a = fmaf(qi[t], kj[t], a);
                sc[j] = (j > i) ? -INFINITY : a * scale; /* apply_causal_mask */
            }
            softmax_row(sc, T);
            for (size_t t = 0; t < d; ++t) acc[t] = 0.0f;
            for (size_t j = 0; j < T; ++j) {
                const float* vj = v + (b * T + j) * hidden + h * d;
                for (size_t t = 0; t < d; ++t) acc[t] = fmaf(sc[j], vj[t], acc[t]);
            }
            float* o = out + (b * T + i) * hidden + h * d;
            for (size_t t = 0; t < d; ++t) o[t] = acc[t];
        }
        free(acc);
        free(sc);
    }
}

void orc_attn_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                     const int32_t* lens, size_t B, size_t T, size_t Hq, size_t Hkv, size_t d,
                     float scale, float* out) {
    /* per (sequence, query head): scores over the cached positions, softmax, then the V sum
     * per element in ascending position order with fmaf (j-outer over a row of accumulators);
     * the (sequence, head) pairs are independent and run in parallel */
    const size_t rep = Hq / Hkv;
    const long long n = (long long)(B * Hq);
#pragma omp parallel
    {
        float* sc = (float*)malloc(T * 4 + 4);
        float* acc = (float*)malloc(d * 4 + 4);
#pragma omp for schedule(static)
        for (long long it = 0; it < n; ++it) {
            const size_t b = (size_t)it / Hq, h = (size_t)it % Hq;
            const size_t L = lens ? (size_t)lens[b] : T;
            const size_t kvh = h / rep;
            const float* qh = q + (b * Hq + h) * d;
            float* o = out + (b * Hq + h) * d;
            if (L == 0) {
                for (size_t t = 0; t < d; ++t) o[t] = 0.0f;
                continue;
            }
            for (size_t j = 0; j < L; ++j) {
                const uint16_t* kj = kcache + ((b * T + j) * Hkv + kvh) * d;
                float a = 0.0f;
                for (size_t t = 0; t < d; ++t) a = fmaf(qh[t], orc_f16_to_f32(kj[t]), a);
                sc[j] = a * scale;
            }
            softmax_row(sc, L);
            for (size_t t = 0; t < d; ++t) acc[t] = 0.0f;
            for (size_t j = 0; j < L; ++j) {
                const uint16_t* vj = vcache + ((b * T + j) * Hkv + kvh) * d;
                for (size_t t = 0; t < d; ++t) acc[t] = fmaf(sc[j], orc_f16_to_f32(vj[t]), acc[t]);
            }
            for (size_t t = 0; t < d; ++t) o[t] = acc[t];
        }
        free(acc);
        free(sc);
    }
}

/* ---------------------------------------------------------- decoder ops */

void orc_rms_norm(const float* x, const float* w, size_t ntok, size_t n, float eps, float* y) {
    /* cortex_sdk.cpp:1208-1232 */
    for (size_t t = 0; t < ntok; ++t) {
        const float* s = x + t * n;
        float ms = 0.0f;
        for (size_t i = 0; i < n; ++i) ms += s[i] * s[i];
        ms /= (float)n;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < n; ++i) y[t * n + i] = s[i] * inv * w[i];
    }
}

void orc_silu_mul(const float* gate, const float* up, size_t n, float* y) {
    /* cortex_sdk.cpp:1245-1256 */
    for (size_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float sig = 1.0f / (1.0f + expf(-g));
        y[i] = (g * sig) * up[i];
    }
}

void orc_rope(float* x, size_t ntok, size_t heads, size_t head_dim, float theta, size_t pos0) {
    /* get_rope_cache / apply_rope_inplace, cortex_sdk.cpp:1363-1423: freq for pair
     * (i, i+1) = theta^(-i/head_dim), angle = pos * freq, adjacent-pair rotation. */
    const size_t rot = head_dim - (head_dim % 2);
    for (size_t t = 0; t < ntok; ++t) {
        const float pos = (float)(pos0 + t);
        for (size_t h = 0; h < heads; ++h) {
            float* base = x + (t * heads + h) * head_dim;
            for (size_t i = 0; i < rot; i += 2) {
                const float freq = powf(theta, -((float)i / (float)head_dim));
                const float ang = pos * freq;
                const float c = cosf(ang), s = sinf(ang);
                const float x0 = base[i], x1 = base[i + 1];
                base[i] = x0 * c - x1 * s;
                base[i + 1] = x0 * s + x1 * c;
            }
        }
    }
}

int orc_select_best(const float* logits, size_t n, const uint8_t* repeated, float temperature,
                    float penalty) {
    /* cortex_sdk.cpp:1005-1030 */
    const float ts = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    float best = -INFINITY;
    int tok = -1;
    for (size_t i = 0; i < n; ++i) {
        float s = logits[i] * ts;
        if (!isfinite(s)) continue;
        if (repeated && repeated[i]) s -= penalty;
        if (s > best) {
            best = s;
            tok = (int)i;
        }
    }
    return tok;
}

/* ------------------------------------------------------------------ HSDR encoder */

/* dot_product_simd (HierarchicalSDRStrategy.cpp:157-190) in its AVX2 lane order */
static float dot_avx2_order(const float* a, const float* b, size_t n) {
    float acc[16] = {0};  /* acc0 = lanes 0..7, acc1 = lanes 8..15 */
    size_t c = 0;
    for (; c + 16 <= n; c += 16)
        for (int l = 0; l < 16; ++l) acc[l] = fmaf(a[c + l], b[c + l], acc[l]);
    for (; c + 8 <= n; c += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[c + l], b[c + l], acc[l]);
    float v[8], h[4];
    for (int l = 0; l < 8; ++l) v[l] = acc[l] + acc[8 + l];   /* acc0 + acc1 */
    for (int i = 0; i < 4; ++i) h[i] = v[i] + v[i + 4];        /* low + high 128 */
    float s = (h[0] + h[1]) + (h[2] + h[3]);                   /* two horizontal adds */
    for (; c < n; ++c) s = fmaf(a[c], b[c], s);                /* scalar tail, contracted */
    return s;
}

void orc_hsdr_mp(const float* tiles, size_t n_tiles, size_t C, const float* D, size_t K,
                 size_t S, size_t k, const float* gamma, uint16_t* codes) {
    /* hierarchicalBinaryCode :219-262, one tile per iteration (the reference's encode_all
     * loop, :556-567) */
    long i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < (long)n_tiles; ++i) {
        float* r = (float*)malloc(C * sizeof(float));
        float* proj = (float*)malloc(K * sizeof(float));
        uint8_t* used = (uint8_t*)malloc(K);
        memcpy(r, tiles + (size_t)i * C, C * sizeof(float));
        for (size_t l = 0; l < S; ++l) {
            memset(used, 0, K);
            for (size_t st = 0; st < k; ++st) {
                for (size_t j = 0; j < K; ++j) {
                    const float sj = dot_avx2_order(D + j * C, r, C);
                    proj[j] = used[j] ? 0.0f : sj;
                }
                size_t best = 0;
                float best_abs = 0.0f;
                for (size_t j = 0; j < K; ++j) {
                    const float a = fabsf(proj[j]);
                    if (a > best_abs) {
                        best_abs = a;
                        best = j;
                    }
                }
                const int sign = proj[best] >= 0.0f ? 1 : -1;
                codes[(size_t)i * S * k + l * k + st] =
                    (uint16_t)((best & 0x7FFFu) | (sign < 0 ? 0x8000u : 0u));
                used[best] = 1;
                const float scale = gamma[l] * (float)sign;
                const float* atom = D + best * C;
                for (size_t c = 0; c < C; ++c) r[c] = fmaf(-atom[c], scale, r[c]);
            }
        }
        free(r);
        free(proj);
        free(used);
    }
}

int orc_set_threads(int n) {
    const int prev = omp_get_max_threads();
    if (n > 0) omp_set_num_threads(n);
    return prev;
}

/* ---------------------------------------------------------------- A14 lazy HSDR (CLI) */

typedef struct {
    uint32_t R, C, K, S, k;
    size_t off_gamma, off_atoms, off_packed;
} lazy_view;

/* parse_hsdr_codes_for_embedding, cortexsdr_cli.cpp:488-534 */
static int lazy_parse(const uint8_t* buf, size_t n, lazy_view* v) {
    if (!buf || !v) return ORC_E_ARG;
    if (n < 36) return ORC_E_TRUNCATED;
    if (memcmp(buf, "HSDR", 4) != 0) return ORC_E_MAGIC;
    if (rd16(buf + 20) != 1) return ORC_E_GEOMETRY; /* 1-row tiles only, :520 */
    v->R = rd32(buf + 16);
    v->C = rd16(buf + 22);
    v->K = rd16(buf + 24);
    v->S = buf[26];
    v->k = buf[27];
    v->off_gamma = 36;
    v->off_atoms = v->off_gamma + 4u * v->S;
    v->off_packed = v->off_atoms + 4u * (size_t)v->K * v->C;
    if (v->off_packed + 2u * (size_t)v->R * v->S * v->k > n) return ORC_E_TRUNCATED;
    return ORC_OK;
}

static void lazy_code(uint16_t pk, int unpack, uint32_t* idx, float* sgn) {
    if (unpack == ORC_LAZY_CLI) { /* :545-546, :716-717 */
        *idx = pk >> 1;
        *sgn = (pk & 1u) ? -1.0f : 1.0f;
    } else { /* HierarchicalSDRStrategy.cpp:81-84 */
        *idx = pk & 0x7FFFu;
        *sgn = (pk & 0x8000u) ? -1.0f : 1.0f;
    }
}

int orc_lazy_hsdr_info(const uint8_t* buf, size_t n, uint32_t* rows, uint32_t* cols) {
    lazy_view v;
    int rc = lazy_parse(buf, n, &v);
    if (rc) return rc;
    if (rows) *rows = v.R;
    if (cols) *cols = v.C;
    return ORC_OK;
}

int orc_lazy_hsdr_decode_row(const uint8_t* buf, size_t n, int unpack, uint32_t row, float* out) {
    /* hsdr_decode_row, cortexsdr_cli.cpp:536-554 */
    lazy_view v;
    int rc = lazy_parse(buf, n, &v);
    if (rc) return rc;
    if (row >= v.R || !out) return ORC_E_ARG;
    for (uint32_t c = 0; c < v.C; ++c) out[c] = 0.0f;
    const size_t slots = (size_t)v.S * v.k;
    for (uint32_t l = 0; l < v.S; ++l) {
        float gamma;
        memcpy(&gamma, buf + v.off_gamma + 4u * l, 4);
        for (uint32_t b = 0; b < v.k; ++b) {
            uint32_t idx;
            float sgn;
            lazy_code(rd16(buf + v.off_packed + 2u * ((size_t)row * slots + (size_t)l * v.k + b)),
                      unpack, &idx, &sgn);
            if (idx >= v.K) continue;
            const float scale = gamma * sgn;
            for (uint32_t c = 0; c < v.C; ++c) {
                float a;
                memcpy(&a, buf + v.off_atoms + 4u * ((size_t)idx * v.C + c), 4);
                out[c] += scale * a;
            }
        }
    }
    return ORC_OK;
}

int orc_lazy_hsdr_select(const uint8_t* buf, size_t n, int unpack, const float* hidden,
                         const uint8_t* repeated, float temperature, float penalty,
                         float* scores, int* token) {
    /* select_next_token_from_lazy_hsdr, cortexsdr_cli.cpp:687-732 */
    lazy_view v;
    int rc = lazy_parse(buf, n, &v);
    if (rc) return rc;
    if (!hidden || !token) return ORC_E_ARG;
    float* ah = (float*)malloc(((size_t)v.K + 1) * 4);
    float* gam = (float*)malloc(((size_t)v.S + 1) * 4);
    if (!ah || !gam) {
        free(ah);
        free(gam);
        return ORC_E_ARG;
    }
    memcpy(gam, buf + v.off_gamma, 4u * v.S);
    for (uint32_t a = 0; a < v.K; ++a) {
        double s = 0.0;
        for (uint32_t c = 0; c < v.C; ++c) {
            float x;
            memcpy(&x, buf + v.off_atoms + 4u * ((size_t)a * v.C + c), 4);
            s += (double)x * hidden[c];
        }
        ah[a] = (float)s;
    }
    const float temp_scale = temperature > 0.0f ? (1.0f / temperature) : 1.0f;
    const size_t slots = (size_t)v.S * v.k;
    int best = -1;
    float best_score = -INFINITY;
    for (uint32_t tok = 0; tok < v.R; ++tok) {
        float score = 0.0f;
        for (uint32_t l = 0; l < v.S; ++l) {
            for (uint32_t b = 0; b < v.k; ++b) {
                uint32_t idx;
                float sgn;
                lazy_code(rd16(buf + v.off_packed + 2u * ((size_t)tok * slots + (size_t)l * v.k + b)),
                          unpack, &idx, &sgn);
                if (idx >= v.K) continue;
                score += gam[l] * sgn * ah[idx];
            }
        }
        if (scores) scores[tok] = score;
        score *= temp_scale;
        if (repeated && repeated[tok]) score -= penalty;
        if (score > best_score) {
            best_score = score;
            best = (int)tok;
        }
    }
    free(ah);
    free(gam);
    *token = best;
    return ORC_OK;
}
