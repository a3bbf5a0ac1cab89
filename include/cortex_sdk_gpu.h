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
 *   - cortex_inference_engine_run runs the archive's layers in the reference's execution
 *     order as a chain of linear layers (see below); layers that are not 2-D weights of the
 *     device path (conv, pooling, graph ops) return CORTEX_ERROR_UNSUPPORTED_FORMAT.
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

/* SDRInferenceEngine::run (SparseInferenceEngine.cpp:2220-2262) without an ONNX graph: the
 * archive's weight-like segments in getExecutionOrder's order (:2852-2893: layer_index and
 * layer_name first, then names; token embeddings skipped), run on demand as
 * runLayersOnDemand does (:2911-3027), each layer's output the next one's input: strategy-5
 * layers through the coded product (no bias, as the reference's HSDR stub), fp32 / q4_k / GGUF
 * layers through their device products plus a `name.bias` segment when present. The input
 * is M x C of the first layer (M = input_size / C). get_last_run_stats_json then lists the
 * layers with their load and device times. */
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

/* ======================================================================
 * The rest of the reference SDK surface (api/c_api.hpp:46-117, api/cortex_sdk.h:42-103,
 * 252-281), so that the reference CLI (src/cortexsdr_cli.cpp:918, :1639) and its Python
 * wrapper (python/cortexsdr_sdk/_bindings.cpp:28, :55) link unchanged. Host-only functions
 * behave as the reference's; the compression / extraction family returns
 * CORTEX_ERROR_UNSUPPORTED_FORMAT (model parsers, strategy chain and archive writer are not
 * part of this inference library) and never yields a handle.
 * ==================================================================== */

/* c_api.hpp:18-24 status codes of the compressor API */
#define CORTEX_OK 0
#define CORTEX_ERR_INVALID_ARG 1
#define CORTEX_ERR_FILE_NOT_FOUND 2
#define CORTEX_ERR_UNSUPPORTED_FORMAT 3
#define CORTEX_ERR_INTERNAL 100

typedef struct CortexCompressor* CortexCompressorHandle;
typedef void* CortexDecompressorHandle;

/* c_api.hpp:32-43 */
typedef struct {
    size_t num_threads;
    int verbose;
    int show_stats;
    int use_delta_encoding;
    int use_rle;
    int compression_level;
    int use_quantization;
    int quantization_bits;
    int use_hsdr;
    float sparsity;
} CortexCompressionOptions;

/* Reference defaults (c_api.cpp:298-317). */
CSDR_API CortexError cortex_compression_options_init(CortexCompressionOptions* options);
/* c_api.cpp:680-689. */
CSDR_API const char* cortex_error_string(int code);
/* findModelParts (c_api.cpp:55-110, 490-514): the existing parts of a
 * "<base>-NNNNN-of-MMMMM<ext>" set, else the path itself; returns the count. *parts_out is a
 * malloc'd array of malloc'd strings (free each with cortex_free_string, then the array). */
CSDR_API int cortex_model_get_parts(const char* model_path, char*** parts_out, int* num_parts);
/* cortex_sdk.cpp:2096-2150: tokenizer assets by segment name (sentencepiece / gpt2-bpe);
 * *out_tokenizer_type is freed with cortex_free_string. */
CSDR_API CortexError cortex_archive_get_tokenizer_info(const char* archive_path,
                                                       int* out_has_tokenizer,
                                                       char** out_tokenizer_type);
/* Unsupported here (see above). */
CSDR_API CortexError cortex_compressor_create(const char* model_path, const char* format,
                                              const CortexCompressionOptions* options,
                                              CortexCompressorHandle* handle);
CSDR_API CortexError cortex_compressor_add_file(CortexCompressorHandle handle,
                                                const char* model_path);
CSDR_API CortexError cortex_compressor_compress(CortexCompressorHandle handle,
                                                const char* output_path);
CSDR_API CortexError cortex_compressor_get_stats(CortexCompressorHandle handle,
                                                 size_t* original_size, size_t* compressed_size,
                                                 double* compression_ratio,
                                                 double* compression_time_ms);
CSDR_API CortexError cortex_compressor_free(CortexCompressorHandle handle);
CSDR_API CortexError cortex_decompressor_create(const char* compressed_path,
                                                CortexDecompressorHandle* handle, float sparsity);
CSDR_API CortexError cortex_decompressor_decompress(CortexDecompressorHandle handle,
                                                    const char* compressed_path,
                                                    const char* output_path);
CSDR_API CortexError cortex_decompressor_free(CortexDecompressorHandle handle);
CSDR_API CortexError cortex_archive_extract(const char* compressed_path, const char* output_dir,
                                            float sparsity);
CSDR_API CortexError cortex_compress_from_url(const char* url_or_path, const char* format,
                                              const char* output_path, float sparsity);

/* Device-side form of run_layer for callers whose activations already live in HBM: x is
 * C x M feature-major (matmulRowMajor's convention), y R x M fp32, both device pointers, on
 * hip_stream. Strategy-5 segments only. */
CSDR_API CortexError cortex_inference_engine_matmul_device(CortexInferenceEngineHandle handle,
                                                           const char* layer_name,
                                                           const void* x, int x_dtype, int M,
                                                           float* y, void* hip_stream);

/* Extension (no SDK counterpart): generate_text chooses tokens as the text CLI's native path
 * does with an HSDR token embedding, select_next_token_from_lazy_hsdr
 * (src/cortexsdr_cli.cpp:687-732: the decoder's output-normed hidden state scored against
 * the embedding's codes, temperature 0.8, repeat penalty 1.0), instead of the SDK's lm_head
 * choice. mode 0: off (default); 1: codes read as packIndexSign wrote them; 2: codes read
 * as the CLI reads them (index = v >> 1, sign = v & 1, :545-546). The token embedding must
 * be a strategy-5 HSDR segment with 1-row tiles. */
CSDR_API CortexError cortex_inference_engine_set_lazy_hsdr_selection(CortexInferenceEngineHandle handle,
                                                                     int mode);

#ifdef __cplusplus
}
#endif
#endif /* CORTEX_SDK_GPU_H */
