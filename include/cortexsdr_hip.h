/*
 * cortexsdr_hip.h — C-ABI of the MI355X (gfx950) compressed-weight inference path.
 *
 * The library (cortexsdr_amd/libcortexsdr_amd.so) is the device layer that the
 * reference's CPU inference path binds to. Every entry point takes plain pointers,
 * sizes and an explicit HIP stream (`void*` = hipStream_t, NULL = the null stream),
 * returns an int status (0 = CSDR_OK, negative = error; the message is available from
 * csdr_last_error() on the calling thread), throws nothing, and allocates nothing on the
 * compute path: loads allocate the device-resident segment once, compute calls take a
 * caller-owned workspace. Calls on different streams are reentrant as long as they use
 * different workspaces.
 *
 * Reference interfaces replaced (paths relative to the cortexSDR tree):
 *   csdr_hsdb_load / csdr_hsdb_free
 *       the per-call parse of an HSDR stream in HierarchicalSDRStrategy::matmulRowMajor
 *       (strategies/HierarchicalSDRStrategy.cpp:1265-1299) and
 *       SDRModelLoader::loadCompressedBytesByName (SparseInferenceEngine.cpp:1055-1064),
 *       here done once into a device-resident segment.
 *   csdr_hsdb_matmul
 *       HierarchicalSDRStrategy::matmulRowMajor (HierarchicalSDRStrategy.hpp:179-181,
 *       .cpp:1257-1338) for 1-row-tile HSDR streams, generalised to the block-coded
 *       1 x 64 "HSDB" streams (research exp_c_kernel/benchmark.py:106-130), and the
 *       engine's SDRModelLoader::matmulHSDR / SDRInferenceEngine::matmulForLayer routing
 *       target (SparseInferenceEngine.hpp:190-192, :305-307).
 *   csdr_hsdb_decompress
 *       HierarchicalSDRStrategy::decompress (HierarchicalSDRStrategy.cpp:1340-1440).
 *   csdr_hsdb_export_codes
 *       the unpacked (index, sign) view of decodeAllTiles' inputs
 *       (HierarchicalSDRStrategy.cpp:81-84, 612-634), for bit-exact layout checks.
 *   csdr_q4k_linear / csdr_q4k_dequant
 *       decodeSupportedGGUFQuantized q4_k (SparseInferenceEngine.cpp:266-274, 362-384) followed
 *       by Kernels::linear_forward (kernels/blas_kernels.cpp:264-293).
 *   csdr_gguf_format / csdr_gguf_block / csdr_gguf_linear / csdr_gguf_dequant
 *       decodeSupportedGGUFQuantized for every format it decodes (SparseInferenceEngine.cpp:
 *       181-231 block sizes, 276-469 decode) followed by Kernels::linear_forward.
 *   csdr_hsdr_encode / csdr_hsdr_init_dictionary / csdr_hsdr_compress(_bytes)
 *       the encode side: hierarchicalBinaryCode (HierarchicalSDRStrategy.cpp:219-262) over
 *       many tiles, fitHierarchicalKSVD's initialisation (:507-541), and
 *       HierarchicalSDRStrategy::compress (:1064-1237) around them.
 */
#ifndef CORTEXSDR_HIP_H
#define CORTEXSDR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define CSDR_API __attribute__((visibility("default")))
#else
#define CSDR_API
#endif

/* ---- status codes (0 = success, as CortexError.code in api/c_api.hpp:18-29) ---- */
#define CSDR_OK 0
#define CSDR_E_INVALID (-1)   /* bad argument / shape mismatch                         */
#define CSDR_E_FORMAT (-2)    /* bad magic, version or geometry (CompressionError)     */
#define CSDR_E_TRUNCATED (-3) /* stream shorter than its header says                   */
#define CSDR_E_HIP (-4)       /* a HIP runtime call failed                             */
#define CSDR_E_WORKSPACE (-5) /* workspace missing or too small                        */
#define CSDR_E_UNSUPPORTED (-6)

/* ---- element types of activation buffers ---- */
#define CSDR_F32 0
#define CSDR_F16 1

/* Last error message of the calling thread ("" when none). */
CSDR_API const char* csdr_last_error(void);
/* Library version string. */
CSDR_API const char* csdr_version(void);

/* ======================================================================
 * HSDR / HSDB device segments (strategy id 5 payloads)
 * ==================================================================== */

/* Opaque device-resident coded matrix. */
typedef struct csdr_hsdb csdr_hsdb;

typedef struct csdr_hsdb_info {
    uint32_t rows;          /* R: output features                                   */
    uint32_t cols;          /* C: input features                                    */
    uint32_t tile_rows;     /* 1 for matmul-capable streams                          */
    uint32_t tile_cols;     /* block length B (64 for HSDB; C for 1-row HSDR)        */
    uint32_t n_atoms;       /* K                                                    */
    uint32_t n_stages;      /* S                                                    */
    uint32_t k_per_stage;   /* k                                                    */
    uint32_t slots;         /* S * k coded atoms per tile                           */
    uint32_t n_block_cols;  /* C_full / B                                           */
    uint32_t chunk_blocks;  /* block columns per device code chunk                  */
    uint32_t edge_cols;     /* C - C_full (fp32 edge strip width)                   */
    uint32_t is_hsdb;       /* 1 = real fp16 coefficients, 0 = binary HSDR          */
    uint64_t code_bytes;    /* compressed code bytes on device (4 per slot)         */
    uint64_t device_bytes;  /* total device bytes held by the segment               */
} csdr_hsdb_info;

/* Parse an HSDR v2 ("HSDR") or HSDB v1 ("HSDB") stream from host memory and upload it to
 * the current device in the kernel layout. Validation follows matmulRowMajor/decompress:
 * magic, version, tile geometry vs shape, edge byte count, truncation, and every atom index
 * < n_atoms (the reference would read outside D). */
CSDR_API int csdr_hsdb_load(const void* stream, size_t nbytes, void* hip_stream,
                            csdr_hsdb** out);
/* csdr_hsdb_load with the code words kept in pinned host memory instead of device memory
 * (the dictionary, stage gammas and edge strips are uploaded): the unit of the on-demand
 * layer loading of SDRInferenceEngine::runLayersOnDemand / loadLayerByNameAsync
 * (SparseInferenceEngine.cpp:2911-3027, 1101-1224), whose layers are read when they run.
 * A decoder streams such a layer's codes to the device when the layer runs
 * (csdr_decoder_set_layer_prefetch); products, decodes and exports on the segment itself
 * return CSDR_E_UNSUPPORTED. device_bytes in csdr_hsdb_get_info excludes the host codes. */
CSDR_API int csdr_hsdb_load_host(const void* stream, size_t nbytes, void* hip_stream,
                                 csdr_hsdb** out);
CSDR_API int csdr_hsdb_free(csdr_hsdb* seg);
CSDR_API int csdr_hsdb_get_info(const csdr_hsdb* seg, csdr_hsdb_info* info);

/* Device workspace bytes csdr_hsdb_matmul needs for batch M (P = D . X on the P path, the
 * transposed fp16 X on the matrix-core path); enough for every batch <= M too.
 * Calls that share a workspace must be ordered (same stream); concurrent calls need their
 * own. */
CSDR_API size_t csdr_hsdb_workspace_bytes(const csdr_hsdb* seg, int M);

/* Y = W . X with W never materialised. X: device, (C x M) row-major (feature-major, the
 * matmulRowMajor convention), element type x_dtype; Y: device fp32 (R x M) row-major.
 * tile_rows must be 1. fp32 accumulation throughout. */
CSDR_API int csdr_hsdb_matmul(const csdr_hsdb* seg, const void* x, int x_dtype, int M,
                              float* y, void* workspace, size_t workspace_bytes,
                              void* hip_stream);

/* csdr_hsdb_matmul without a workspace argument and without any allocation: the product's
 * scratch memory (the P slices, or the transposed X of the matrix-core path) is a
 * file-scope device array of 8 MiB per device, held until the process ends. No counterpart
 * in the reference: for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Products whose csdr_hsdb_workspace_bytes(seg, M)
 * exceeds 8 MiB are rejected with CSDR_E_WORKSPACE. Every call on a device shares that
 * device's scratch, so calls that overlap on one device (other streams, other threads) race;
 * serialise them. The segment must live on the current device. */
CSDR_API int csdr_hsdb_matmul_noalloc(const csdr_hsdb* seg, const void* x, int x_dtype, int M,
                                      float* y, void* hip_stream);

/* Grouped form: n (1..8) independent products Y_i = W_i . X_i (all with the same M and
 * x_dtype), e.g. the q/k/v or gate/up projections of a decoder layer, in two launches.
 * The P path, all fp32: a dx launch (P = D . X per block column into the workspace, Y = 0 or
 * bias; on the fp32 matrix cores for 64-column blocks) and a gather launch (Y += the coded
 * rows gathered from P). It serves M == 1 (4, 8 or 16 slots: two 1024-thread workgroups per
 * CU stream the codes), 2 <= M <= 8 with 1-row tiles of 4/8/16 slots (the codes streamed once
 * for all M columns), and matrices the matrix-core path does not take. Other M >= 2 with
 * 64-column blocks, K <= 1024 atoms and 4/8/16 slots: an init launch and a matrix-core launch that
 * decodes 64-column tiles (dictionary and decoded weights rounded to fp16, fp32 X split into
 * fp16 hi + lo, fp32 accumulation: about 3e-4 relative L2 from the fp32 product); setting the
 * environment variable CSDR_HSDB_MFMA=0 keeps such calls on the fp32 P path. At M <= 16 with
 * fp16 X and 4 or 8 slots the matrix-core launch forms Q = D . X per block column instead
 * and gathers each row's slots from it. Q is stored in fp16, so each 64-value block of an X
 * column needs a norm below 65504, the fp16 maximum (|Q| <= ||x_block|| for unit-norm atoms).
 * CSDR_HSDB_QROUTE=0 keeps those calls on the decoding launch. The workspace
 * is csdr_hsdb_group_workspace_bytes(n, segs, M) bytes, enough for every path and phase at
 * that M (x-op calls and the separate dx / gather phases take the P path). csdr_hsdb_matmul
 * is the n = 1 case. Y rows are accumulated over block-column ranges with device-scope float
 * atomics, so repeated calls agree to fp32 rounding, not bit for bit. */
CSDR_API size_t csdr_hsdb_group_workspace_bytes(int n, const csdr_hsdb* const* segs, int M);
CSDR_API int csdr_hsdb_matmul_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream);
/* The two launches of the P path of csdr_hsdb_matmul_group, separately, at any M (same
 * arguments; dx must precede gather on the stream, with the same workspace and X; the
 * workspace is csdr_hsdb_group_workspace_bytes(n, segs, M) bytes). */
CSDR_API int csdr_hsdb_dx_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                int x_dtype, int M, float* const* y, void* workspace,
                                size_t workspace_bytes, void* hip_stream);
CSDR_API int csdr_hsdb_gather_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream);

/* As csdr_hsdb_matmul_group with per-matrix bias (bias[i] = NULL or R_i floats added to every
 * column; bias itself may be NULL) and flags: CSDR_HSDB_ACCUMULATE makes Y += W.X (+ bias)
 * instead of Y = W.X (+ bias), which folds a residual add into the product;
 * CSDR_HSDB_TOKEN_MAJOR takes X as M x C and writes Y as M x R (token-major, the layout of
 * Kernels::linear_forward, blas_kernels.cpp:264-293, and of the SDK's run_layer) instead of
 * C x M and R x M (identical at M == 1). 2 <= M <= 8 (1-row tiles of 4, 8 or 16 slots) runs
 * the streaming gather with M columns per code read (fp32 throughout; with the environment
 * variable CSDR_HSDB_P16=1, 5 <= M <= 8 keeps the per-block products D.x_b in fp16 instead:
 * faster, about 2e-4 relative per value, and the transformed x's block norms must stay below
 * 65504). */
#define CSDR_HSDB_ACCUMULATE 1
#define CSDR_HSDB_TOKEN_MAJOR 2
CSDR_API int csdr_hsdb_matmul_group_ex(int n, const csdr_hsdb* const* segs, const void* const* x,
                                       int x_dtype, int M, float* const* y,
                                       const float* const* bias, int flags, void* workspace,
                                       size_t workspace_bytes, void* hip_stream);

/* As csdr_hsdb_matmul_group_ex (fp32 x, P path) with an input transform applied while x is
 * staged, so the transformed vector is never written out (decoder kernel fusion):
 *   CSDR_XOP_RMSNORM   x := x / sqrt(mean(x^2) + eps) * norm_w, per column (rms_norm,
 *                      cortex_sdk.cpp:1208-1232); M <= 16
 *   CSDR_XOP_SILU_MUL  x := silu(x) * x2 (silu_mul, :1245-1256); M <= 16
 *   CSDR_XOP_ATTN      x := the attention output combined from csdr_attn_decode's split
 *                      partials (x = its workspace, attn_splits splits, attn_head_dim); M == 1
 * Matrices need 64-column blocks. */
#define CSDR_XOP_NONE 0
#define CSDR_XOP_RMSNORM 1
#define CSDR_XOP_SILU_MUL 2
#define CSDR_XOP_ATTN 3
CSDR_API int csdr_hsdb_matmul_group_xop(int n, const csdr_hsdb* const* segs,
                                        const void* const* x, const void* const* x2, int M,
                                        float* const* y, const float* const* bias, int flags,
                                        int xop, const float* norm_w, float eps, int attn_splits,
                                        int attn_head_dim, void* workspace,
                                        size_t workspace_bytes, void* hip_stream);

/* Row `row` of W (1-row tiles) decoded into out[C] (device), bit-identical to the same row
 * of csdr_hsdb_decompress. The row is *row_dev when row_dev is not NULL (a token id produced
 * on the device, e.g. a tied embedding lookup inside a captured decode step), else row_host.
 * The CLI's lazy embedding-row decode (cortexsdr_cli.cpp:536-554) with the canonical code
 * unpacking of HierarchicalSDRStrategy.cpp:81-84. */
CSDR_API int csdr_hsdb_decode_row(const csdr_hsdb* seg, const int* row_dev, int row_host,
                                  float* out, void* hip_stream);
/* n rows at once: row i's index is rows_dev[i] (device int32), decoded into out + i * C
 * (n x C fp32, token-major). Indices outside [0, R) leave their output row untouched. The
 * batched form of the embedding lookup (build_token_embeddings, cortex_sdk.cpp:1480-1541). */
CSDR_API int csdr_hsdb_decode_rows(const csdr_hsdb* seg, const int* rows_dev, int n, float* out,
                                   void* hip_stream);

/* Dense decode to device W (R x C fp32 row-major), bit-identical to the reference decode
 * order (stage-major slot accumulation with fused multiply-adds, then the edge strips). */
CSDR_API int csdr_hsdb_decompress(const csdr_hsdb* seg, float* w, void* hip_stream);

/* Export the device codes back in stream order (tile-major, slot-major): packed[i] =
 * (sign << 15) | index, coef_abs[i] = fp16 bits of |c| (HSDB; 0x3C00 for binary HSDR).
 * Both are device buffers of n_tiles * slots uint16 (coef_abs may be NULL). */
CSDR_API int csdr_hsdb_export_codes(const csdr_hsdb* seg, uint16_t* packed, uint16_t* coef_abs,
                                    void* hip_stream);

/* ======================================================================
 * HSDR encoder (compress side)
 * ==================================================================== */

/* Hierarchical binary matching pursuit of n_tiles tiles (device, n_tiles x tile_dim fp32)
 * against D (device, n_atoms x tile_dim fp32), hierarchicalBinaryCode
 * (HierarchicalSDRStrategy.cpp:219-262): per stage l (stage_scales[l], a host array of
 * n_stages floats) k_per_stage greedy picks of the first maximum of |<D_j, r>| (atoms already
 * picked in the stage score 0), sign = +1 when that projection is >= 0, r -= scale * sign *
 * D_best. Projections are summed in the reference's AVX2 order (dot_product_simd :157-190),
 * so the picks are the reference's bit for bit. codes (device, n_tiles x n_stages *
 * k_per_stage uint16): packIndexSign (:76-80), tile-major, stage-major. Any tile_dim (the
 * last tile_dim % 8 elements are the reference's scalar tail); n_atoms <= 32768;
 * n_stages <= 32. */
CSDR_API int csdr_hsdr_encode(const float* tiles, size_t n_tiles, int tile_dim, const float* D,
                              int n_atoms, int n_stages, int k_per_stage,
                              const float* stage_scales, uint16_t* codes, void* hip_stream);
/* Size of the HSDR v2 stream csdr_hsdr_compress writes for this shape and config (0 when the
 * shape cannot be compressed: no full tile, fewer tiles than atoms). */
CSDR_API size_t csdr_hsdr_compress_bytes(uint32_t rows, uint32_t cols, uint16_t tile_rows,
                                         uint16_t tile_cols, uint16_t n_atoms,
                                         uint8_t n_stages, uint8_t k_per_stage);
/* The dictionary initialisation of fitHierarchicalKSVD (HierarchicalSDRStrategy.cpp:507-541),
 * host code: atom j = the tile std::uniform_int_distribution picks over std::mt19937(0xC0DE),
 * unit length, all scaled by the mean tile norm / max(1, sqrt(n_stages * k_per_stage)); in
 * the reference build's arithmetic (its -ffast-math 1/sqrt is the CPU's approximate
 * reciprocal square root plus one Newton step; the approximation is taken from a table of the
 * Intel Xeon the reference's golden outputs were written on, and the tile norms are summed in
 * the order its vectorised loop uses), so D (host, n_atoms x tile_dim) is that reference run's
 * bit for bit on any host CPU. tiles: host, n_tiles x tile_dim. */
CSDR_API int csdr_hsdr_init_dictionary(const float* tiles, uint32_t n_tiles, uint32_t tile_dim,
                                       uint16_t n_atoms, uint8_t n_stages, uint8_t k_per_stage,
                                       float* D);
/* HierarchicalSDRStrategy::compress (HierarchicalSDRStrategy.cpp:1064-1237) of an fp32
 * rows x cols host matrix w into out (csdr_hsdr_compress_bytes bytes): tile_rows == 1 widens
 * tiles to whole rows (configFor :1024-1046); dictionary as csdr_hsdr_init_dictionary, one
 * matching-pursuit pass on the GPU (csdr_hsdr_encode), edge strips as fp32, stage scales
 * stage_decay^l: with ksvd_iters = 0 the reference's stream byte for byte on the same CPU.
 * ksvd_iters > 0 adds that many atomUpdateStep passes (:281-490: users per atom in (tile,
 * slot) order, double corrections damped by 0.5 / sum gamma^2, the norm cap, re-seeds from the
 * fit's generator; residuals and updates on the GPU), each followed by matching pursuit again
 * (:570-573); tiles of at most 32768 values. */
CSDR_API int csdr_hsdr_compress(const float* w, uint32_t rows, uint32_t cols, uint16_t tile_rows,
                                uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                                uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay,
                                uint8_t* out, size_t out_bytes, void* hip_stream);

/* Shared-dictionary compression of a group of fp32 matrices (host, row-major):
 * compressGroupedSegments (HierarchicalSDRStrategy.cpp:2212-2502) written as
 * SharedDictArchive::writeToStream (:1967-2002). Matrices are bucketed by their config (1-row
 * tiles widen to each matrix's width; one dictionary per bucket, buckets in the order of the
 * reference's std::unordered_map over the same key and hash); a matrix whose shape is not a
 * whole number of tiles, or with more than 1e-3 non-finite values, is skipped (others are
 * zeroed: with 2-D tiles the reference re-encodes such a matrix from its raw values,
 * :2472-2476, so NaN/Inf reach its matching pursuit there; this build encodes the zeroed
 * values in both modes, a deliberate difference that no reference fixture covers); each
 * bucket's tiles are pooled, reservoir-sampled to max_tiles_for_fit when that
 * is non-zero and smaller (mt19937(0xC0DECAFE ^ cap), :2277-2395), the dictionary fitted on
 * the pool as csdr_hsdr_compress fits one matrix (ksvd_iters passes), and every matrix of
 * the bucket encoded against it as an HSDC codes stream (compressFP32WithExternalDictionary,
 * :1690-1754). The archive is returned in *out (malloc'd; release with csdr_free_buffer);
 * skipped (may be NULL) receives one flag per matrix; original_types (may be NULL: 1,
 * WEIGHTS_FP32) is stored per segment. The config's two padding bytes are written as zero. */
CSDR_API int csdr_hsda_build(int n, const char* const* names, const float* const* w,
                             const uint32_t* rows, const uint32_t* cols,
                             const uint8_t* original_types, uint16_t tile_rows,
                             uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                             uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay,
                             uint32_t max_tiles_for_fit, uint8_t** out, size_t* out_size,
                             uint8_t* skipped, void* hip_stream);
CSDR_API void csdr_free_buffer(void* p);

/* The compressor's source decode, dequantizeSegmentToFP32 (HierarchicalSDRStrategy.cpp:
 * 713-989), on the GPU: the bytes of a segment to the fp32 matrix the compressor tiles, the
 * reference's values bit for bit. Formats (CSDR_SRC_*): f32, f16, bf16, int8 as
 * (q - zero_point) * scale, and GGUF q4_0 / q8_0 (element 2j from the low nibble of byte j),
 * q4_k / q5_k (element i from byte i/2, low nibble for even i) and q6_k in the compressor's
 * element order, which for q4_k / q6_k differs from the engine's (csdr_q4k_linear,
 * csdr_gguf_linear). csdr_hsdr_source_format maps a segment's data_format name and
 * SegmentType (1 = WEIGHTS_FP32, 2 = WEIGHTS_FP16, 3 = WEIGHTS_INT8) to a format as the
 * reference dispatches them, or -1; csdr_hsdr_source_elements gives the decoded value count
 * (0 for a byte size that is not a whole number of blocks). src and out are device memory.
 * csdr_hsdr_compress_source decodes on the GPU, then compresses as csdr_hsdr_compress (the
 * decoded matrix is copied to the host for the dictionary initialisation): the reference's
 * compress of a quantized segment. */
#define CSDR_SRC_F32 0
#define CSDR_SRC_F16 1
#define CSDR_SRC_BF16 2
#define CSDR_SRC_I8 3
#define CSDR_SRC_Q4_0 4
#define CSDR_SRC_Q8_0 5
#define CSDR_SRC_Q4_K 6
#define CSDR_SRC_Q5_K 7
#define CSDR_SRC_Q6_K 8
CSDR_API int csdr_hsdr_source_format(const char* data_format, int segment_type);
CSDR_API size_t csdr_hsdr_source_elements(int format, size_t nbytes);
CSDR_API int csdr_hsdr_source_decode(const void* src, size_t nbytes, int format, float scale,
                                     float zero_point, float* out, void* hip_stream);
CSDR_API int csdr_hsdr_compress_source(const void* src, size_t nbytes, int format, float scale,
                                       float zero_point, uint32_t rows, uint32_t cols,
                                       uint16_t tile_rows, uint16_t tile_cols, uint16_t n_atoms,
                                       uint8_t n_stages, uint8_t k_per_stage, uint8_t ksvd_iters,
                                       float stage_decay, uint8_t* out, size_t out_bytes,
                                       void* hip_stream);

/* ======================================================================
 * GGUF Q4_K dequant-matmul (engine path, no fp32 W materialised)
 * ==================================================================== */

/* Element order inside a 144-byte super-block:
 *   CSDR_Q4K_GGML        32-byte group g: low nibbles = sub-block 2g, high = 2g+1 (the engine
 *                        and SDK decoders, SparseInferenceEngine.cpp:362-384,
 *                        api/cortex_sdk.cpp:352-372)
 *   CSDR_Q4K_INTERLEAVED element i = byte i/2, low nibble when i is even (HSDR compress side,
 *                        HierarchicalSDRStrategy.cpp:836-845) */
#define CSDR_Q4K_GGML 0
#define CSDR_Q4K_INTERLEAVED 1

/* y (M x R, fp32) = x (M x C) . dequant(W)^T, W = R rows of C/256 super-blocks (GGUF
 * row-major, 16-byte aligned device memory); the linear_forward convention of
 * kernels/blas_kernels.cpp:264-293 applied to the tensor decodeSupportedGGUFQuantized
 * (SparseInferenceEngine.cpp:276-469) would produce. M == 1 takes fp32 or fp16 x; M > 1 takes
 * fp16 x (MFMA path). C must be a multiple of 256. No workspace. */
CSDR_API int csdr_q4k_linear(const void* w, int R, int C, int order, const void* x, int x_dtype,
                             int M, float* y, void* hip_stream);

/* Dequantise n_blocks super-blocks to fp32 (256 values each), same arithmetic as the
 * reference: (d*sc)*q - dmin*m. */
CSDR_API int csdr_q4k_dequant(const void* w, size_t n_blocks, int order, float* out,
                              void* hip_stream);

/* ======================================================================
 * GGUF block formats of the engine (strategy-0 tensors), dequant-matmul
 * ==================================================================== */

/* Format ids (ggml's type numbers). Decoded exactly as the reference engine does
 * (SparseInferenceEngine.cpp:276-469), including its element orders: q4_0 / q4_1 / q5_0 / q5_1
 * take element i from byte i/2 (low nibble for even i); q6_k's four 32-element quarters of
 * each 128-element half use that half's scales 0, 2, 4, 6; q8_1's scale is read as fp32, q8_k's
 * as fp16 with quants at byte 4. Formats without an exact decoder in the reference (q2_k, q3_k,
 * q5_k, iq*, tq*, q4_0_x_y) take its generic rule: `bits` per element packed LSB-first at the
 * end of the block, centred on 2^(bits-1), times the fp16 scale at the block start (1 when
 * that is not finite or below 1e-12). */
#define CSDR_GGUF_Q4_0 2
#define CSDR_GGUF_Q4_1 3
#define CSDR_GGUF_Q5_0 6
#define CSDR_GGUF_Q5_1 7
#define CSDR_GGUF_Q8_0 8
#define CSDR_GGUF_Q8_1 9
#define CSDR_GGUF_Q2_K 10
#define CSDR_GGUF_Q3_K 11
#define CSDR_GGUF_Q4_K 12
#define CSDR_GGUF_Q5_K 13
#define CSDR_GGUF_Q6_K 14
#define CSDR_GGUF_Q8_K 15
#define CSDR_GGUF_IQ2_XXS 16
#define CSDR_GGUF_IQ2_XS 17
#define CSDR_GGUF_IQ3_XXS 18
#define CSDR_GGUF_IQ1_S 19
#define CSDR_GGUF_IQ4_NL 20
#define CSDR_GGUF_IQ3_S 21
#define CSDR_GGUF_IQ2_S 22
#define CSDR_GGUF_IQ4_XS 23
#define CSDR_GGUF_IQ1_M 29
#define CSDR_GGUF_Q4_0_4_4 31
#define CSDR_GGUF_Q4_0_4_8 32
#define CSDR_GGUF_Q4_0_8_8 33
#define CSDR_GGUF_TQ1_0 34
#define CSDR_GGUF_TQ2_0 35

/* The format id of a GGUF type name as segment data_format holds it (case-insensitive),
 * or -1. */
CSDR_API int csdr_gguf_format(const char* name);

/* Bytes and elements per block of a format (ggufBlockBytesForFormat /
 * ggufBlockElementsForFormat, SparseInferenceEngine.cpp:181-231). */
CSDR_API int csdr_gguf_block(int format, int* block_bytes, int* block_elems);

/* y (M x R, fp32) = x (M x C) . dequant(W)^T, W = R rows of C / block_elems blocks (row-major
 * device memory, any alignment). M == 1 takes fp32 or fp16 x; M > 1 takes fp16 x (8-byte
 * aligned) and needs C % 16 == 0 (matrix-core path, dequantised values split into fp16 hi +
 * lo, fp32 accumulation). C must be a multiple of the block's elements. No workspace. */
CSDR_API int csdr_gguf_linear(const void* w, int format, int R, int C, const void* x,
                              int x_dtype, int M, float* y, void* hip_stream);

/* Dequantise n_blocks blocks to fp32 with the reference's arithmetic. */
CSDR_API int csdr_gguf_dequant(const void* w, int format, size_t n_blocks, float* out,
                               void* hip_stream);

/* ======================================================================
 * Decoder ops (api/cortex_sdk.cpp run_transformer_decode building blocks)
 * ==================================================================== */

/* y = x / sqrt(mean(x^2) + eps) * w per row of n (rms_norm, cortex_sdk.cpp:1208-1232). */
CSDR_API int csdr_rms_norm(const float* x, const float* w, int ntok, int n, float eps, float* y,
                           void* hip_stream);
/* y (M x R) = x (M x C) . W^T for an uncoded fp32 W (R x C): Kernels::linear_forward's
 * layout (blas_kernels.cpp:264-293), the dense fallback of matmulForLayer for strategy-0
 * segments (SparseInferenceEngine.cpp:1290-1311). */
CSDR_API int csdr_dense_linear(const float* w, int R, int C, const float* x, int M, float* y,
                               void* hip_stream);
/* As csdr_dense_linear, plus bias (R floats, may be NULL) and flags (CSDR_HSDB_ACCUMULATE:
 * y += x . W^T + bias). M >= 8 (C % 4 == 0, w and x 16-byte aligned) runs on the fp32 matrix
 * cores (v_mfma_f32_16x16x4_f32, fp32 accumulation); smaller M one wave per row of W. The
 * decoder's batched prefill multiplies the prompt rows by each coded weight decoded once with
 * csdr_hsdb_decompress through this call. */
CSDR_API int csdr_dense_linear_ex(const float* w, int R, int C, const float* x, int M, float* y,
                                  const float* bias, int flags, void* hip_stream);
/* y = silu(g) * u (silu_mul, cortex_sdk.cpp:1245-1256). */
CSDR_API int csdr_silu_mul(const float* g, const float* u, size_t n, float* y, void* hip_stream);
/* RoPE on adjacent pairs (get_rope_cache/apply_rope_inplace, cortex_sdk.cpp:1363-1423) of
 * q (ntok x Hq x hd) and k (ntok x Hkv x hd) in place at positions *pos_dev + t, then k and v
 * appended to the fp16 caches [position][kv head][hd] (capacity max_ctx positions). */
CSDR_API int csdr_rope_kv(float* q, float* k, const float* v, int ntok, int Hq, int Hkv, int hd,
                          const int* pos_dev, float theta, uint16_t* kcache, uint16_t* vcache,
                          int max_ctx, void* hip_stream);
/* Decode attention: out (B x Hq x hd) = softmax(q.K^T * scale) V over cached positions
 * [0, len_b) (len_b = lens_dev[b], or len_host when lens_dev is NULL; a length outside
 * [0, T] is clamped into it, so no row past the cache is read or written); caches (B x T x Hkv x
 * hd) fp16; GQA as repeat_kv_heads (cortex_sdk.cpp:1453-1478); scale 0 = 1/sqrt(hd).
 * Split over chunks of 64..256 positions (about T / 8; workspace csdr_attn_decode_workspace_bytes)
 * then combined. 2..16 query heads per KV head run on the matrix cores (fp16 hi + lo operands,
 * fp32 accumulate); CSDR_ATTN_MFMA=0 selects the vector-ALU kernel instead.
 * head_dim 64 or 128. Replaces Kernels::multi_head_attention's full-context recompute
 * (attention_kernels.cpp:26-113) with the cached form flash_attention.cpp:165-247 intends. */
CSDR_API size_t csdr_attn_decode_workspace_bytes(int B, int Hq, int hd, int T);
CSDR_API int csdr_attn_decode(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                              const int* lens_dev, int len_host, int B, int T, int Hq, int Hkv,
                              int hd, float scale, float* out, void* workspace,
                              size_t workspace_bytes, void* hip_stream);
/* Number of position splits csdr_attn_decode uses for this shape (the partial count the
 * CSDR_XOP_ATTN x op combines). */
CSDR_API int csdr_attn_decode_splits(int B, int Hq, int Hkv, int hd, int T);
/* Decode attention fused with RoPE and the KV append, for one new token per batch entry at
 * position lens_dev[b] - 1: q (B x Hq x hd) and k_new (B x Hkv x hd) are rotated in
 * registers (apply_rope_inplace, cortex_sdk.cpp:1395-1423), k_new and v_new are rounded to
 * fp16 and appended to the caches at that position, and the attention reads them from there.
 * out = NULL leaves the split partials in the workspace for a consumer that combines them
 * (csdr_hsdb_matmul_group_xop with CSDR_XOP_ATTN); otherwise as csdr_attn_decode. */
CSDR_API int csdr_attn_decode_rope(const float* q, const float* k_new, const float* v_new,
                                   uint16_t* kcache, uint16_t* vcache, const int* lens_dev, int B,
                                   int T, int Hq, int Hkv, int hd, float theta, float scale,
                                   float* out, void* workspace, size_t workspace_bytes,
                                   void* hip_stream);
/* As csdr_attn_decode_rope with the cache element type given: CSDR_F16 (the form above) or
 * CSDR_F32 (caches of fp32 values, B x T x Hkv x hd; the K/V precision of the reference's
 * recompute, run_transformer_decode cortex_sdk.cpp:1543-1696, on the vector ALU kernel).
 * csdr_attn_decode_splits_kv: the split count such a call produces. */
CSDR_API int csdr_attn_decode_rope_kv(const float* q, const float* k_new, const float* v_new,
                                      void* kcache, void* vcache, int kv_dtype,
                                      const int* lens_dev, int B, int T, int Hq, int Hkv, int hd,
                                      float theta, float scale, float* out, void* workspace,
                                      size_t workspace_bytes, void* hip_stream);
CSDR_API int csdr_attn_decode_splits_kv(int B, int Hq, int Hkv, int hd, int T, int kv_dtype);
/* Multi-token (prefill) forms: B sequences of T new tokens each, row b * T + t of q
 * (B T x Hq x hd), k and v (B T x Hkv x hd) at position p0 + t of sequence b; caches
 * B x max_ctx x Hkv x hd of kv_dtype (CSDR_F32 or CSDR_F16) elements, p0 + T <= max_ctx.
 * csdr_rope_kv_rows rotates q and k in place (apply_rope_inplace, cortex_sdk.cpp:1395-1423,
 * the decode step's arithmetic) and appends k and v to the caches at their positions.
 * csdr_attn_prefill then computes out (same layout as q) = causal softmax(q.K^T * scale) V
 * over positions [0, p0 + t] of the caches (Kernels::multi_head_attention with the causal
 * mask, attention_kernels.cpp:26-113, the tiled form flash_attention.cpp:17-163; GQA as
 * repeat_kv_heads; scale 0 = 1/sqrt(hd)); head_dim 64 or 128, fp32 matrix-core products,
 * 16-byte aligned buffers. */
CSDR_API int csdr_rope_kv_rows(float* q, float* k, const float* v, int B, int T, int p0, int Hq,
                               int Hkv, int hd, float theta, void* kcache, void* vcache,
                               int kv_dtype, int max_ctx, void* hip_stream);
CSDR_API int csdr_attn_prefill(const float* q, const void* kcache, const void* vcache,
                               int kv_dtype, int B, int T, int p0, int max_ctx, int Hq, int Hkv,
                               int hd, float scale, float* out, void* hip_stream);
/* Next token as select_best_from_logits (cortex_sdk.cpp:1005-1030): score = logit /
 * temperature (temperature <= 0: 1) minus penalty where repeated[i] != 0 (repeated may be
 * NULL); best finite score, lowest index on ties; -1 when none is finite. Writes the token to
 * *out_token (device); when pos_dev is not NULL increments *pos_dev, and when repeated_update
 * is not NULL sets repeated_update[token] = 1 (both for captured decode loops). */
CSDR_API size_t csdr_select_workspace_bytes(void);
CSDR_API int csdr_select_best(const float* logits, int n, const uint8_t* repeated,
                              float temperature, float penalty, int* out_token, int* pos_dev,
                              uint8_t* repeated_update, void* workspace, size_t workspace_bytes,
                              void* hip_stream);

/* Lazy HSDR embedding of the text CLI (src/cortexsdr_cli.cpp): rows decoded and the
 * vocabulary scored straight from the codes of an HSDR stream with 1-row tiles (vocabulary =
 * n_tiles rows of tile_cols), no dense table. csdr_lazy_hsdr_load reads the stream as
 * parse_hsdr_codes_for_embedding (:488-534; magic HSDR, version not checked), with code words
 * read as packIndexSign wrote them (CSDR_LAZY_UNPACK_PACKED: bit 15 sign, bits 0-14 index,
 * HierarchicalSDRStrategy.cpp:76-84) or as the CLI reads them (CSDR_LAZY_UNPACK_CLI: index =
 * v >> 1, sign = v & 1, :545-546, :716-717, a compatibility reading); indices >= K are
 * skipped. csdr_lazy_hsdr_decode_rows: hsdr_decode_row (:536-554) for n tokens (device ids
 * rows_dev[i], or row_host when rows_dev is NULL; a device id outside the vocabulary gives a
 * zero row), out n x cols. csdr_lazy_hsdr_select: select_next_token_from_lazy_hsdr
 * (:687-732) for `rows` hidden states (rows x cols, device): atom . hidden summed in fp64 and
 * rounded to float, per token the float sum over its slots in order of (gamma * sign) *
 * (atom . hidden), times 1 / temperature when temperature > 0, minus `penalty` (the CLI:
 * 1.0) where repeated[row][token] != 0 (repeated may be NULL); the first strictly largest
 * score wins (-1 when none beats -infinity). tokens (device, rows) receive the choice;
 * pos_dev (may be NULL) is incremented once, repeated_update (may be NULL) marks the chosen
 * tokens, scores (may be NULL, rows x vocabulary) receives the sums before temperature and
 * penalty. No counterpart for the CLI's host-side tokenizer. */
typedef struct csdr_lazy_hsdr csdr_lazy_hsdr;
#define CSDR_LAZY_UNPACK_PACKED 0
#define CSDR_LAZY_UNPACK_CLI 1
CSDR_API int csdr_lazy_hsdr_load(const void* stream, size_t nbytes, int unpack, void* hip_stream,
                                 csdr_lazy_hsdr** out);
CSDR_API int csdr_lazy_hsdr_free(csdr_lazy_hsdr* h);
CSDR_API int csdr_lazy_hsdr_info(const csdr_lazy_hsdr* h, uint32_t* rows, uint32_t* cols);
CSDR_API int csdr_lazy_hsdr_decode_rows(const csdr_lazy_hsdr* h, const int* rows_dev,
                                        int row_host, int n, float* out, void* hip_stream);
CSDR_API size_t csdr_lazy_hsdr_workspace_bytes(const csdr_lazy_hsdr* h, int rows);
CSDR_API int csdr_lazy_hsdr_select(const csdr_lazy_hsdr* h, const float* hidden, int rows,
                                   const uint8_t* repeated, float temperature, float penalty,
                                   int* tokens, int* pos_dev, uint8_t* repeated_update,
                                   float* scores, void* workspace, size_t workspace_bytes,
                                   void* hip_stream);

/* ======================================================================
 * Containers: the .sdr archive, HSDC codes-only streams, the HSDA shared-dictionary archive
 * (host parsing; loads go to the current device)
 * ==================================================================== */

/* Open .sdr archive: the index is read once (AIDecompressor::readArchiveIndex,
 * core/AIDecompressor.cpp:78-262, magic "CORTEXSR", versions 1-2) and one file handle is kept
 * for payload reads (the reference re-opens the file per read, :418-435). */
typedef struct csdr_archive csdr_archive;
/* One index entry (CompressedSegmentHeader, core/AICompressor.hpp:51-65). The strings stay
 * valid until csdr_archive_close. At most 8 dims / shape entries are reported. */
typedef struct csdr_segment_info {
    const char* name;
    const char* data_format;
    const char* layer_type;
    const char* layer_name;
    uint32_t original_type; /* SegmentType (core/ModelSegment.hpp:35-55) */
    uint32_t strategy_id;   /* 0 raw, 5 HSDR (SparseInferenceEngine.cpp:725-751) */
    uint64_t original_size, compressed_size, data_offset;
    uint32_t layer_index;
    uint32_t has_metadata, n_dims, dims[8];
    float sparsity_ratio;
    uint32_t n_input_dims, input_shape[8], n_output_dims, output_shape[8];
} csdr_segment_info;

CSDR_API int csdr_archive_open(const char* path, csdr_archive** out);
CSDR_API int csdr_archive_close(csdr_archive* archive);
CSDR_API size_t csdr_archive_count(const csdr_archive* archive);
CSDR_API int csdr_archive_info(const csdr_archive* archive, size_t index, csdr_segment_info* info);
/* Index of the first entry named `name` (SDRModelLoader::findSegmentHeader,
 * SparseInferenceEngine.cpp:1066-1072). */
CSDR_API int csdr_archive_find(const csdr_archive* archive, const char* name, size_t* index);
/* The stored (compressed) payload bytes of entry `index` (readCompressedBytes). With
 * buf == NULL only *nbytes is set; otherwise cap must be >= the payload size. */
CSDR_API int csdr_archive_read(const csdr_archive* archive, size_t index, void* buf, size_t cap,
                               size_t* nbytes);

/* External dictionary of a codes-only stream (HierarchicalSDRStrategy::SharedDictionary:
 * config + stage scales + atoms, n_atoms * tile_rows * tile_cols floats). */
typedef struct csdr_dictionary {
    uint32_t tile_rows, tile_cols, n_atoms, n_stages, k_per_stage;
    float stage_decay;
    const float* stage_scales;
    uint32_t n_stage_scales;
    const float* atoms;
    size_t n_atom_floats;
} csdr_dictionary;
/* Load an HSDC codes-only stream (HSDRCodesHeader, HierarchicalSDRStrategy.cpp:675-691) with
 * its external dictionary as a device segment; the geometry checks of parseCodesStream
 * (:1766-1801). The segment then serves csdr_hsdb_matmul (matmulWithExternalDictionary,
 * :1830-1883) and csdr_hsdb_decompress (decompressWithExternalDictionary, :1804-1828). */
CSDR_API int csdr_hsdb_load_codes(const void* codes, size_t nbytes, const csdr_dictionary* dict,
                                  void* hip_stream, csdr_hsdb** out);

/* HSDA shared-dictionary archive (SharedDictArchive::readFromStream,
 * HierarchicalSDRStrategy.cpp:1937-2081) with HSDAReader's by-name access (:2506-2550):
 * csdr_hsda_load builds the named segment's device form, which then serves matmul and
 * decompress. */
typedef struct csdr_hsda csdr_hsda;
CSDR_API int csdr_hsda_open(const char* path, csdr_hsda** out);
CSDR_API int csdr_hsda_open_memory(const void* data, size_t nbytes, csdr_hsda** out);
CSDR_API int csdr_hsda_close(csdr_hsda* hsda);
CSDR_API size_t csdr_hsda_count(const csdr_hsda* hsda);
CSDR_API size_t csdr_hsda_dictionary_count(const csdr_hsda* hsda);
CSDR_API int csdr_hsda_segment(const csdr_hsda* hsda, size_t index, const char** name,
                               uint32_t* dict_index, uint64_t* original_size);
CSDR_API int csdr_hsda_load(const csdr_hsda* hsda, const char* name, void* hip_stream,
                            csdr_hsdb** out);

/* ======================================================================
 * Decoder engine (api/cortex_sdk.cpp run_transformer_decode :1543-1696 and
 * cortex_inference_engine_generate_text :1951-2054)
 *
 * A Llama/Qwen-style decoder whose linears are loaded csdr_hsdb segments (the decoder keeps
 * the pointers; the caller keeps the segments alive). K/V are kept in a per-layer cache
 * (max_ctx positions, fp32 or fp16) instead of the reference's whole-context recompute; each step is one
 * replay of a captured HIP graph. Token choice as select_next_token_from_embedding_transpose
 * (cortex_sdk.cpp:1032-1206): output RMSNorm, sanitize_hidden_for_sampling (:959-976), lm_head
 * scores, select_best_from_logits with `temperature` and `penalty` for tokens generated so far
 * (the reference's generate_text uses 0.8 and 1.5). Not reentrant: one thread per decoder.
 *
 * Batch: csdr_decoder_create_batched decodes `batch` (1..16) sequences in lockstep, one
 * position for all (the batch of an SDK engine, cortex_inference_engine_set_batch_size,
 * cortex_sdk.cpp:1793-1802). Per-sequence data is sequence-major: prompts and tokens
 * batch x count, logits batch x vocab, imported K/V batch x n positions; every projection
 * is one product over the batch's columns.
 * ==================================================================== */
typedef struct csdr_decoder csdr_decoder;
typedef struct csdr_decoder_config {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    float rope_theta; /* RoPE base (get_rope_cache, cortex_sdk.cpp:1363; 1e6 there) */
    float rms_eps;    /* RMSNorm epsilon (rms_norm, cortex_sdk.cpp:1212; 1e-5 there) */
    int kv_dtype;     /* K/V cache element: CSDR_F32 (0, the precision of the reference's
                       * recompute) or CSDR_F16 (half the bytes; its rounding is amplified by
                       * sharp attention, e.g. 8e-3 of the scores on a random-init 24-layer
                       * model) */
} csdr_decoder_config;

CSDR_API int csdr_decoder_create(const csdr_decoder_config* cfg, csdr_decoder** out);
CSDR_API int csdr_decoder_create_batched(const csdr_decoder_config* cfg, int batch,
                                         csdr_decoder** out);
/* Sequences per step (-1 for NULL). */
CSDR_API int csdr_decoder_batch(const csdr_decoder* dec);
CSDR_API int csdr_decoder_free(csdr_decoder* dec);
/* Block `layer`'s weights (transformer_blocks names attn_q/k/v/output, ffn_gate/up/down,
 * attn_norm, ffn_norm; cortex_sdk.cpp:1570-1660). Shapes: q,o H x H; k,v (Hkv*hd) x H;
 * gate,up F x H; down H x F; all 1-row-tile HSDB. Norm weights (H floats, host) required;
 * q/k/v biases optional (NULL = none; the reference applies none). */
CSDR_API int csdr_decoder_set_layer(csdr_decoder* dec, int layer, const csdr_hsdb* wq,
                                    const csdr_hsdb* wk, const csdr_hsdb* wv, const csdr_hsdb* wo,
                                    const csdr_hsdb* wgate, const csdr_hsdb* wup,
                                    const csdr_hsdb* wdown, const float* attn_norm,
                                    const float* ffn_norm, const float* bq, const float* bk,
                                    const float* bv);
/* On-demand layer streaming. A block whose seven segments are host-resident
 * (csdr_hsdb_load_host) is streamed: when it runs, its code words are copied to one of two
 * device staging buffers on a second stream and its products read them there (the other
 * blocks stay resident; a block mixing both kinds is refused). With prefetch on (the
 * default, as the SDK engine enables it, cortex_sdk.cpp:1770) the copy of the block after
 * next is issued as soon as a block finishes, so the next block's copy runs under the
 * current block's kernels (double buffering, prefetchNextLayer SparseInferenceEngine.cpp:
 * 3461-3467); off, each copy waits for the previous block (no overlap). The copies are part
 * of the captured step graph. The kernels and code words are the resident decoder's, so
 * results equal its results to the products' float-atomic summation order. */
CSDR_API int csdr_decoder_set_layer_prefetch(csdr_decoder* dec, int enable);
/* Code bytes the streamed blocks copy per step (0 when every block is resident). */
CSDR_API int64_t csdr_decoder_streamed_bytes(const csdr_decoder* dec);
/* Output projection (vocab x H) and output norm (NULL = none, as when output_norm_layer_name
 * is empty, cortex_sdk.cpp:1682-1688); embedding NULL = tied (rows of lm_head). */
CSDR_API int csdr_decoder_set_output(csdr_decoder* dec, const csdr_hsdb* lm_head,
                                     const float* final_norm, const csdr_hsdb* embedding);
/* Runs the prompt from position 0 (resetting the cache and the generated-token set) and
 * selects the first new token (it lands at position n_prompt). prompt: batch x n_prompt ids.
 * Positions 0 .. n_prompt - 2 run as multi-token passes of up to the prefill chunk tokens per
 * sequence (csdr_decoder_set_prefill_chunk): every weight decoded once per pass to dense fp32
 * and multiplied on the matrix cores for all the pass's tokens, causal prompt attention
 * (csdr_attn_prefill); the last prompt position runs the decode step, which selects. */
CSDR_API int csdr_decoder_prefill(csdr_decoder* dec, const int32_t* prompt, int n_prompt,
                                  float temperature, float penalty);
/* Token choice by the text CLI's lazy HSDR scoring (select_next_token_from_lazy_hsdr,
 * cortexsdr_cli.cpp:687-732) instead of the lm_head scores: each head step scores the
 * output-normed hidden state (not sanitized, as the CLI passes its decoder output) against
 * emb (vocab x hidden, kept alive by the caller) with the step's temperature and `penalty`
 * for generated tokens (the CLI uses 0.8 and 1.0); csdr_decoder_logits then returns the raw
 * lazy scores. emb NULL restores the lm_head choice. */
CSDR_API int csdr_decoder_set_lazy_selection(csdr_decoder* dec, const csdr_lazy_hsdr* emb,
                                             float penalty);
/* Tokens per sequence in one prefill pass (default 512); 0 runs every prompt position as a
 * decode step instead (the token-at-a-time form). Buffers for B x chunk rows and one dense
 * weight (the largest, F x H fp32) are allocated at the first prefill that needs them. */
CSDR_API int csdr_decoder_set_prefill_chunk(csdr_decoder* dec, int tokens);
/* n_steps further tokens, one graph replay each; synchronises at the end. */
CSDR_API int csdr_decoder_decode(csdr_decoder* dec, int n_steps, float temperature,
                                 float penalty);
/* Host copy of the tokens at positions [first, first + count) (prompt, then generated):
 * batch x count. */
CSDR_API int csdr_decoder_tokens(const csdr_decoder* dec, int first, int count, int32_t* out);
/* generate_text's loop: prefill, then max_new_tokens - 1 decode steps; out_tokens receives
 * batch x max_new_tokens ids, n_generated[b] (batch ints) stops after eos_id (eos_id < 0:
 * none). */
CSDR_API int csdr_decoder_generate(csdr_decoder* dec, const int32_t* prompt, int n_prompt,
                                   int max_new_tokens, float temperature, float penalty,
                                   int eos_id, int32_t* out_tokens, int* n_generated);
/* Host copy of the last head step's lm_head scores (batch x vocab floats, before
 * temperature). */
CSDR_API int csdr_decoder_logits(const csdr_decoder* dec, float* out);
/* Number of positions processed so far (-1 for NULL). */
CSDR_API int csdr_decoder_position(const csdr_decoder* dec);
/* Import a precomputed context (a cached prompt prefix): fp16 K and V of positions [0, n) for
 * one layer, [sequence][position][kv head][head_dim], from host or device memory (widened
 * into an fp32 cache). */
CSDR_API int csdr_decoder_load_kv(csdr_decoder* dec, int layer, const uint16_t* k,
                                  const uint16_t* v, int n);
/* Continue from an imported context: positions [0, position) count as processed and `token`
 * is the token at `position` of every sequence, consumed by the next csdr_decoder_decode step
 * (the _batch form: tokens[b] for sequence b). */
CSDR_API int csdr_decoder_set_position(csdr_decoder* dec, int position, int32_t token);
CSDR_API int csdr_decoder_set_position_batch(csdr_decoder* dec, int position,
                                             const int32_t* tokens);

#ifdef __cplusplus
}
#endif
#endif /* CORTEXSDR_HIP_H */
