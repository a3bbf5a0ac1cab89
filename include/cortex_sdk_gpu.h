/*
 * cortex_sdk_gpu.h — the reference SDK's inference-engine C API (cortexSDR
 * src/ai_compression/api/cortex_sdk.h:37-281, error type c_api.hpp:18-29), served by the
 * MI355X path in libcortexsdr_amd.so.
 *
 * Same symbol names, argument meaning and return convention (CortexError by value, code 0 =
 * success, the SDK's negative codes otherwise), so code written against the reference SDK
 * links unchanged for the functions declared here. What differs, deliberately:
 *   - strategy-5 (HSDR/HSDB) segments are parsed once into device-resident segments and
 *     cached; uncoded fp32 2-D segments run a dense device GEMV; strategy-0 "q4_k" segments
 *     run the Q4_K dequant-matmul; other strategies are rejected (CORTEX_ERROR_UNSUPPORTED_FORMAT).
 *   - error messages are owned by the library (thread-local, valid until the next call on
 *     the thread); cortex_error_free accepts them and frees nothing. Strings returned through
 *     char** are malloc'd and released with cortex_free_string (free), fixing the reference's
 *     new[]/free mismatch (cortex_sdk.cpp:124-128, 2092-2094).
 *   - the handle table is guarded by a mutex (the reference's is an unsynchronised map,
 *     cortex_sdk.cpp:114); one handle must still not be used by two threads at once.
 *   - generate_text takes the prompt as whitespace-separated token ids and returns the
 *     generated ids the same way: the tokenizer (LLMTokenizer) is outside this path.
 *   - cortex_inference_engine_run (whole-graph execution of non-decoder models) returns
 *     CORTEX_ERROR_UNSUPPORTED_FORMAT: the graph executor is outside the coded-weight path.
 */
#ifndef CORTEX_SDK_GPU_H
#define CORTEX_SDK_GPU_H

#include <stddef.h>
#include <stdint.h>

#include "cortexsdr_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* SDK status codes (cortex_sdk.cpp:56-64). */
#define CORTEX_SUCCESS 0
#define CORTEX_ERROR_INVALID_ARGUMENT (-1)
#define CORTEX_ERROR_FILE_IO (-2)
#define CORTEX_ERROR_MEMORY (-3)
#define CORTEX_ERROR_UNSUPPORTED_FORMAT (-4)
#define CORTEX_ERROR_COMPRESSION (-5)
#define CORTEX_ERROR_DECOMPRESSION (-6)
#define CORTEX_ERROR_INFERENCE (-7)
#define CORTEX_ERROR_UNKNOWN (-99)

typedef struct {
    const char* message;
    int code;
} CortexError;

typedef struct CortexInferenceEngine* CortexInferenceEngineHandle;

/* Opens a .sdr archive (index only; segments load on first use). */
CSDR_API CortexError cortex_inference_engine_create(const char* compressed_model_path,
                                                    CortexInferenceEngineHandle* handle);
CSDR_API CortexError cortex_inference_engine_set_batch_size(CortexInferenceEngineHandle handle,
                                                            size_t batch_size);
/* Stored; inference has no dropout. */
CSDR_API CortexError cortex_inference_engine_enable_dropout(CortexInferenceEngineHandle handle,
                                                            int enable);
CSDR_API CortexError cortex_inference_engine_set_mode(CortexInferenceEngineHandle handle,
                                                      int training_mode);
/* Device budget (MiB) for cached segments: least recently used segments are released when a
 * load would exceed it (0 = unbounded). */
CSDR_API CortexError cortex_inference_engine_init_memory_pool(CortexInferenceEngineHandle handle,
                                                              size_t max_memory_mb);
/* Release each segment right after the call that used it (the reference's eviction between
 * layers). */
CSDR_API CortexError cortex_inference_engine_enable_aggressive_memory(
    CortexInferenceEngineHandle handle, int enable);
/* Device bytes held by cached segments. */
CSDR_API CortexError cortex_inference_engine_get_memory_usage(CortexInferenceEngineHandle handle,
                                                              size_t* bytes);
/* Stored; segments stay resident once loaded, so there is nothing to prefetch per call. */
CSDR_API CortexError cortex_inference_engine_enable_layer_prefetch(
    CortexInferenceEngineHandle handle, int enable);
/* JSON of the last run_layer / generate_text call (free with cortex_free_string). */
CSDR_API CortexError cortex_inference_engine_get_last_run_stats_json(
    CortexInferenceEngineHandle handle, char** out_json);
CSDR_API void cortex_free_string(char* s);
CSDR_API void cortex_error_free(CortexError* error);

CSDR_API CortexError cortex_inference_engine_run(CortexInferenceEngineHandle handle,
                                                 const float* input_data, size_t input_size,
                                                 float* output_data, size_t output_size,
                                                 size_t* actual_output_size);
/* Y = W . x for the named 2-D weight segment (name, else name + ".weight", as
 * applyLinearLayer, SparseInferenceEngine.cpp:1490-1494): input is M x C (M = input_size / C
 * rows of C features), output M x R. Output too small: CORTEX_ERROR_MEMORY with the needed
 * count in *actual_output_size. */
CSDR_API CortexError cortex_inference_engine_run_layer(CortexInferenceEngineHandle handle,
                                                       const char* layer_name,
                                                       const float* input_data,
                                                       size_t input_size, float* output_data,
                                                       size_t output_size,
                                                       size_t* actual_output_size);
/* The native decoder over the archive's blk.N.* tensors (discover_native_llm_paths,
 * cortex_sdk.cpp:477-545): prompt and result are whitespace-separated token ids. */
CSDR_API CortexError cortex_inference_engine_generate_text(CortexInferenceEngineHandle handle,
                                                           const char* prompt,
                                                           int max_new_tokens, char** out_text);
CSDR_API CortexError cortex_inference_engine_free(CortexInferenceEngineHandle handle);
CSDR_API const char* cortex_sdk_version(void);

/* Device-side form of run_layer for callers whose activations already live in HBM: x is
 * C x M feature-major (matmulRowMajor's convention), y R x M fp32, both device pointers, on
 * hip_stream. Strategy-5 segments only. */
CSDR_API CortexError cortex_inference_engine_matmul_device(CortexInferenceEngineHandle handle,
                                                           const char* layer_name,
                                                           const void* x, int x_dtype, int M,
                                                           float* y, void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif /* CORTEX_SDK_GPU_H */
