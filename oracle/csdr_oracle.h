/*
 * csdr_oracle.h — CPU restatement of cortexSDR's compressed-weight inference path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker. The product
 * (cortexsdr_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * cortexSDR source tree). Pinning: each function is checked in tests/ against
 * reference golden vectors (known-answer tests, fixtures emitted by the compiled
 * reference in oracle/_ref) or against closed forms / brute force. Functions with
 * no such check are marked "parity unpinned" below (none at present).
 *
 * Conventions
 *   - status codes: 0 ok, negative = error (ORC_E_*).
 *   - HSDR weight W is R x C row-major fp32 (segment dims {R, C}).
 *   - matmul_row_major x is (C x batch) row-major, Y is (R x batch) row-major
 *     (HierarchicalSDRStrategy.hpp:179-181 convention).
 *   - linear x is (M x C) row-major, y is (M x R) row-major
 *     (kernels/blas_kernels.cpp:264-293 linear_forward convention).
 */
#ifndef CSDR_ORACLE_H
#define CSDR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_OK 0
#define ORC_E_MAGIC (-1)
#define ORC_E_VERSION (-2)
#define ORC_E_TRUNCATED (-3)
#define ORC_E_GEOMETRY (-4)
#define ORC_E_ARG (-5)

/* ---- fp16 (utils/fp16_convert.hpp:26-62 decode; encode = IEEE round-to-nearest-even,
 *      the F16C branch at :68-71, not the truncating scalar branch at :73-93) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);
void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);

/* ---- HSDR-family stream view (HierarchicalSDRStrategy.cpp:46-66 header, :1197-1237 order).
 * Magic "HSDR" (version 2): binary codes, coefficient = gamma_l * sign.
 * Magic "HSDB" (version 1): block-coded extension, tile 1 x B; after the packed
 * u16 codes it carries one fp16 |c| per slot; coefficient = gamma_l * sign * |c|.
 * Arrays are copied out (the stream gives no alignment guarantee). */
typedef struct {
    int is_hsdb;
    uint32_t version, rows, cols, n_tiles;
    uint32_t tile_rows, tile_cols, n_atoms, n_stages, k_per_stage;
    float stage_decay;
    uint32_t edge_bytes;
    size_t slots_per_tile;  /* n_stages * k_per_stage */
    size_t n_codes;         /* n_tiles * slots_per_tile */
    size_t off_gamma, off_dict, off_packed, off_coef, off_edge, end;
} orc_hsdr_view;

int orc_hsdr_parse(const uint8_t* buf, size_t n, orc_hsdr_view* v);

/* Unpacked codes in stream (tile-major, stage-major slot) order:
 * idx = packed & 0x7FFF, sign = +1/-1 from bit 15 (HierarchicalSDRStrategy.cpp:81-84).
 * coef = gamma_l * sign (HSDR) or gamma_l * sign * f16(|c|) (HSDB), fp32. */
int orc_hsdr_unpack(const uint8_t* buf, size_t n, uint16_t* idx, int8_t* sign, float* coef);

/* Dense decode, A2: decodeAllTiles + reassembleTiles + edge splice
 * (HierarchicalSDRStrategy.cpp:612-634, 119-135, 1340-1440). out: R*C fp32. */
int orc_hsdr_decompress(const uint8_t* buf, size_t n, float* out, size_t out_floats);

/* Fused 1D-row matmul, A3 (HierarchicalSDRStrategy.cpp:1257-1338). HSDR only;
 * requires tile_rows == 1, tile_cols == C, n_tiles == R (same checks as :1273-1289). */
int orc_hsdr_matmul_row_major(const uint8_t* buf, size_t n, const float* x, size_t batch,
                              float* y);

/* Block-coded fused matmul, A0 (research exp_c_kernel/benchmark.py:106-130 impl_fused_real,
 * with the 1 x B tile order of HierarchicalSDRStrategy.cpp:95-116): per block column b,
 * Dx_b = D . x_b (K x M), then Y[r] += sum_j coef_j * Dx_b[idx_j]; plus the fp32 edge strip
 * times x[C_full:]. x is (C x M) row-major, y (R x M). Accepts HSDR streams with
 * tile_rows == 1 as well (binary codes). */
int orc_hsdb_matmul(const uint8_t* buf, size_t n, const float* x, size_t M, float* y);
/* OpenMP threads of the parallel loops from now on (the CPU baseline's single-thread time);
 * returns the previous setting. */
int orc_set_threads(int n);

/* ---- GGUF K-quant dequant ----
 * ggml order (engine path, A7): SparseInferenceEngine.cpp:266-274 (scale/min unpack),
 * :362-384 (per 32-byte group g: 32 low nibbles -> sub-block 2g, 32 high -> 2g+1).
 * interleaved order (HSDR compress side, A6): HierarchicalSDRStrategy.cpp:802-849
 * (element i of the super-block reads byte i/2, low nibble when i is even).
 * value = (d*sc) * q - (dmin*m). One super-block = 144 bytes = 256 values. */
#define ORC_Q4K_GGML 0
#define ORC_Q4K_INTERLEAVED 1
void orc_q4k_dequant(const uint8_t* blocks, size_t n_blocks, int order, float* out);
/* Q5_K (176 B) and Q6_K (210 B) dequant as HierarchicalSDRStrategy.cpp:851-989. */
void orc_q5k_dequant(const uint8_t* blocks, size_t n_blocks, float* out);
void orc_q6k_dequant(const uint8_t* blocks, size_t n_blocks, float* out);

/* Q4_K linear: y (M x R) = x (M x C) . dequant(W)^T, W = R rows of C/256 super-blocks
 * (GGUF row-major). Dequant then linear_forward semantics (blas_kernels.cpp:264-293,
 * BLAS-less row loop :101-143), fp32 accumulation in column order. */
/* Engine GGUF formats (ids = ggml type numbers, include/cortexsdr_hip.h CSDR_GGUF_*):
 * decodeSupportedGGUFQuantized (SparseInferenceEngine.cpp:276-469), then linear_forward. */
int orc_gguf_block(int fmt, int* block_bytes, int* block_elems);
int orc_gguf_dequant(const uint8_t* blocks, int fmt, size_t n_blocks, float* out);
int orc_gguf_linear(const uint8_t* w, int fmt, size_t R, size_t C, const float* x, size_t M,
                    float* y);
int orc_q4k_linear(const uint8_t* w, size_t R, size_t C, int order, const float* x,
                   size_t M, float* y);

/* ---- Attention ----
 * Causal multi-head attention as kernels/attention_kernels.cpp:26-113: per head,
 * scores = Q K^T / sqrt(d), causal mask, row softmax, times V. q,k,v,out: (B, T, H*d). */
void orc_mha_causal(const float* q, const float* k, const float* v, float* out, size_t B,
                    size_t T, size_t hidden, size_t heads);

/* Decode attention against a cache (the behaviour flash_attention_with_kv_cache,
 * kernels/flash_attention.cpp:165-247, intends, with GQA as repeat_kv_heads,
 * api/cortex_sdk.cpp:1453-1478: q head h reads kv head h / (Hq/Hkv)).
 * q: (B, Hq, d) fp32; kcache/vcache: (B, T, Hkv, d) fp16 bits; out (B, Hq, d).
 * Attends to positions [0, len_b) where len_b = lens[b] (or T when lens == NULL). */
void orc_attn_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                     const int32_t* lens, size_t B, size_t T, size_t Hq, size_t Hkv, size_t d,
                     float scale, float* out);

/* ---- Decoder elementwise (api/cortex_sdk.cpp) ---- */
/* rms_norm :1208-1232 (eps default 1e-5) over ntok rows of width n. */
void orc_rms_norm(const float* x, const float* w, size_t ntok, size_t n, float eps, float* y);
/* silu_mul :1245-1256 */
void orc_silu_mul(const float* gate, const float* up, size_t n, float* y);
/* RoPE on adjacent pairs, get_rope_cache/apply_rope_inplace :1363-1423, positions
 * pos0..pos0+ntok-1; x is (ntok, heads, head_dim) in place. */
void orc_rope(float* x, size_t ntok, size_t heads, size_t head_dim, float theta, size_t pos0);
/* select_best_from_logits :1005-1030: score = logit * (1/temperature when > 0), minus
 * penalty when the token was generated before; strict '>' keeps the first maximum;
 * non-finite scores skipped. Returns -1 when nothing is finite. */
int orc_select_best(const float* logits, size_t n, const uint8_t* repeated, float temperature,
                    float penalty);

/* ---- HSDR encoder (HierarchicalSDRStrategy.cpp) ----
 * Hierarchical binary matching pursuit, hierarchicalBinaryCode :219-262, over n_tiles tiles
 * of C floats against D (K x C): per stage l (gamma[l]) k greedy picks of argmax |<D_j, r>|
 * (first maximum, strict '>', atoms picked earlier in the stage score 0), sign = +1 when the
 * projection is >= 0, r -= gamma_l * sign * D_best. Projections in dot_product_simd's
 * (:157-190) AVX2 order: 16 lane sums over 16-element chunks (two 8-lane FMA accumulators),
 * an 8-element chunk into the first, then (acc0 + acc1), low + high halves, two horizontal
 * adds, then a contracted scalar tail. The update as axpy_subtract_simd (:193-216): fused
 * r - atom * scale. codes: packIndexSign (:76-80), tile-major, stage-major slots. */
void orc_hsdr_mp(const float* tiles, size_t n_tiles, size_t C, const float* D, size_t K,
                 size_t S, size_t k, const float* gamma, uint16_t* codes);

/* ---- A14: the text CLI's lazy HSDR embedding (cortexsdr_cli.cpp:488-554, 687-732).
 * The stream is read as parse_hsdr_codes_for_embedding does (:488-534): the 36-byte HSDR
 * header (magic "HSDR", version not checked), 1-row tiles only, vocabulary R = n_tiles,
 * width C = tile_cols, then stage scales, atoms (K x C), packed codes (R x S*k u16); a stream
 * shorter than that is ORC_E_TRUNCATED (the CLI reads past it). unpack: ORC_LAZY_PACKED
 * reads codes as packIndexSign wrote them (bit 15 sign, bits 0-14 index,
 * HierarchicalSDRStrategy.cpp:76-84); ORC_LAZY_CLI as the CLI reads them (index = v >> 1,
 * sign = v & 1, :545-546, :716-717). Indices >= K are skipped (:547, :718).
 * decode_row: hsdr_decode_row (:536-554), out[c] += (gamma_l * sign) * atom[c] in float, slot
 * order. select: select_next_token_from_lazy_hsdr (:687-732): ah[a] = float(sum over c of
 * double(atom[a][c]) * hidden[c], c ascending); score = sum over the slots in order of
 * (gamma_l * sign) * ah[idx] in float, times 1 / temperature when temperature > 0, minus
 * penalty (1.0 in the CLI) when repeated[token] != 0 (repeated may be NULL); the first token
 * with a strictly larger score wins (*token = -1 when none beats -infinity). scores (may be NULL)
 * receives the sums before temperature and penalty. Evaluated in ISO order without
 * contraction (the CLI's -ffast-math build may fuse or reorder, changing last bits). */
#define ORC_LAZY_PACKED 0
#define ORC_LAZY_CLI 1
int orc_lazy_hsdr_info(const uint8_t* buf, size_t n, uint32_t* rows, uint32_t* cols);
int orc_lazy_hsdr_decode_row(const uint8_t* buf, size_t n, int unpack, uint32_t row, float* out);
int orc_lazy_hsdr_select(const uint8_t* buf, size_t n, int unpack, const float* hidden,
                         const uint8_t* repeated, float temperature, float penalty,
                         float* scores, int* token);

#ifdef __cplusplus
}
#endif
#endif
