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
CSDR_API int csdr_hsdb_free(csdr_hsdb* seg);
CSDR_API int csdr_hsdb_get_info(const csdr_hsdb* seg, csdr_hsdb_info* info);

/* Device workspace bytes csdr_hsdb_matmul needs for batch M (it holds P = D . X). Calls
 * that share a workspace must be ordered (same stream); concurrent calls need their own. */
CSDR_API size_t csdr_hsdb_workspace_bytes(const csdr_hsdb* seg, int M);

/* Y = W . X with W never materialised. X: device, (C x M) row-major (feature-major, the
 * matmulRowMajor convention), element type x_dtype; Y: device fp32 (R x M) row-major.
 * tile_rows must be 1. fp32 accumulation throughout. */
CSDR_API int csdr_hsdb_matmul(const csdr_hsdb* seg, const void* x, int x_dtype, int M,
                              float* y, void* workspace, size_t workspace_bytes,
                              void* hip_stream);

/* Grouped form: n (1..8) independent products Y_i = W_i . X_i (all with the same M and
 * x_dtype), e.g. the q/k/v or gate/up projections of a decoder layer, in two launches:
 * a dx launch (P = D . X per block column into the workspace, Y = 0) and a gather launch
 * (Y += the coded rows gathered from P). The workspace is
 * csdr_hsdb_group_workspace_bytes(n, segs, M) bytes. csdr_hsdb_matmul is the n = 1 case.
 * Y rows are accumulated over block-column chunks with device-scope float atomics, so
 * repeated calls agree to fp32 rounding, not bit for bit. */
CSDR_API size_t csdr_hsdb_group_workspace_bytes(int n, const csdr_hsdb* const* segs, int M);
CSDR_API int csdr_hsdb_matmul_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream);
/* The two launches of csdr_hsdb_matmul_group, separately (same arguments; dx must precede
 * gather on the stream, with the same workspace and X). */
CSDR_API int csdr_hsdb_dx_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                int x_dtype, int M, float* const* y, void* workspace,
                                size_t workspace_bytes, void* hip_stream);
CSDR_API int csdr_hsdb_gather_group(int n, const csdr_hsdb* const* segs, const void* const* x,
                                    int x_dtype, int M, float* const* y, void* workspace,
                                    size_t workspace_bytes, void* hip_stream);

/* Dense decode to device W (R x C fp32 row-major), bit-identical to the reference decode
 * order (stage-major slot accumulation with fused multiply-adds, then the edge strips). */
CSDR_API int csdr_hsdb_decompress(const csdr_hsdb* seg, float* w, void* hip_stream);

/* Export the device codes back in stream order (tile-major, slot-major): packed[i] =
 * (sign << 15) | index, coef_abs[i] = fp16 bits of |c| (HSDB; 0x3C00 for binary HSDR).
 * Both are device buffers of n_tiles * slots uint16 (coef_abs may be NULL). */
CSDR_API int csdr_hsdb_export_codes(const csdr_hsdb* seg, uint16_t* packed, uint16_t* coef_abs,
                                    void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif /* CORTEXSDR_HIP_H */
