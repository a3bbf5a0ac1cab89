"""The reference SDK's C surface links against libcortexsdr_amd.so unchanged (CPU only).

A C translation unit declares the prototypes the reference's callers use (api/c_api.hpp:46-117,
api/cortex_sdk.h:110-281: the text CLI src/cortexsdr_cli.cpp:918, :1639 and the Python
wrapper python/cortexsdr_sdk/_bindings.cpp:28, :55) with their own types, is linked against
the library with gcc, and runs the host-only functions (option defaults c_api.cpp:298-317,
error strings :680-689, multi-part detection :55-110, the tokenizer probe
cortex_sdk.cpp:2096-2150); the compression family reports CORTEX_ERROR_UNSUPPORTED_FORMAT.
No GPU is touched.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import ROOT

PKG = os.path.join(ROOT, "cortexsdr_amd")
LIB = os.path.join(PKG, "libcortexsdr_amd.so")

PROG = r"""
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { const char* message; int code; } CortexError;
typedef struct CortexCompressor* CortexCompressorHandle;
typedef void* CortexDecompressorHandle;
typedef struct CortexInferenceEngine* CortexInferenceEngineHandle;
typedef struct {
    size_t num_threads; int verbose; int show_stats; int use_delta_encoding; int use_rle;
    int compression_level; int use_quantization; int quantization_bits; int use_hsdr;
    float sparsity;
} CortexCompressionOptions;

CortexError cortex_compression_options_init(CortexCompressionOptions* options);
CortexError cortex_compressor_create(const char* model_path, const char* format,
                                     const CortexCompressionOptions* options,
                                     CortexCompressorHandle* handle);
int cortex_model_get_parts(const char* model_path, char*** parts_out, int* num_parts);
CortexError cortex_compressor_add_file(CortexCompressorHandle handle, const char* model_path);
CortexError cortex_compressor_compress(CortexCompressorHandle handle, const char* output_path);
CortexError cortex_compressor_get_stats(CortexCompressorHandle handle, size_t* original_size,
                                        size_t* compressed_size, double* compression_ratio,
                                        double* compression_time_ms);
CortexError cortex_compressor_free(CortexCompressorHandle handle);
CortexError cortex_decompressor_create(const char* compressed_path,
                                       CortexDecompressorHandle* handle, float sparsity);
CortexError cortex_decompressor_decompress(CortexDecompressorHandle handle,
                                           const char* compressed_path, const char* output_path);
CortexError cortex_archive_extract(const char* compressed_path, const char* output_dir,
                                   float sparsity);
CortexError cortex_decompressor_free(CortexDecompressorHandle handle);
void cortex_error_free(CortexError* error);
const char* cortex_error_string(int code);
CortexError cortex_inference_engine_create(const char* compressed_model_path,
                                           CortexInferenceEngineHandle* handle);
CortexError cortex_inference_engine_set_batch_size(CortexInferenceEngineHandle h, size_t b);
CortexError cortex_inference_engine_enable_dropout(CortexInferenceEngineHandle h, int e);
CortexError cortex_inference_engine_set_mode(CortexInferenceEngineHandle h, int m);
CortexError cortex_inference_engine_init_memory_pool(CortexInferenceEngineHandle h, size_t mb);
CortexError cortex_inference_engine_enable_aggressive_memory(CortexInferenceEngineHandle h, int e);
CortexError cortex_inference_engine_get_memory_usage(CortexInferenceEngineHandle h, size_t* b);
CortexError cortex_inference_engine_enable_layer_prefetch(CortexInferenceEngineHandle h, int e);
CortexError cortex_inference_engine_get_last_run_stats_json(CortexInferenceEngineHandle h,
                                                            char** out_json);
void cortex_free_string(char* s);
CortexError cortex_inference_engine_run(CortexInferenceEngineHandle h, const float* in,
                                        size_t in_size, float* out, size_t out_size,
                                        size_t* actual);
CortexError cortex_inference_engine_run_layer(CortexInferenceEngineHandle h, const char* name,
                                              const float* in, size_t in_size, float* out,
                                              size_t out_size, size_t* actual);
CortexError cortex_inference_engine_generate_text(CortexInferenceEngineHandle h,
                                                  const char* prompt, int max_new_tokens,
                                                  char** out_text);
CortexError cortex_inference_engine_free(CortexInferenceEngineHandle h);
const char* cortex_sdk_version(void);
CortexError cortex_compress_from_url(const char* url_or_path, const char* format,
                                     const char* output_path, float sparsity);
CortexError cortex_archive_get_tokenizer_info(const char* archive_path, int* out_has_tokenizer,
                                              char** out_tokenizer_type);

/* every symbol the reference's callers bind, referenced so that the link resolves each */
static void* const every[] = {
    (void*)cortex_compression_options_init, (void*)cortex_compressor_create,
    (void*)cortex_model_get_parts, (void*)cortex_compressor_add_file,
    (void*)cortex_compressor_compress, (void*)cortex_compressor_get_stats,
    (void*)cortex_compressor_free, (void*)cortex_decompressor_create,
    (void*)cortex_decompressor_decompress, (void*)cortex_archive_extract,
    (void*)cortex_decompressor_free, (void*)cortex_error_free, (void*)cortex_error_string,
    (void*)cortex_inference_engine_create, (void*)cortex_inference_engine_set_batch_size,
    (void*)cortex_inference_engine_enable_dropout, (void*)cortex_inference_engine_set_mode,
    (void*)cortex_inference_engine_init_memory_pool,
    (void*)cortex_inference_engine_enable_aggressive_memory,
    (void*)cortex_inference_engine_get_memory_usage,
    (void*)cortex_inference_engine_enable_layer_prefetch,
    (void*)cortex_inference_engine_get_last_run_stats_json, (void*)cortex_free_string,
    (void*)cortex_inference_engine_run, (void*)cortex_inference_engine_run_layer,
    (void*)cortex_inference_engine_generate_text, (void*)cortex_inference_engine_free,
    (void*)cortex_sdk_version, (void*)cortex_compress_from_url,
    (void*)cortex_archive_get_tokenizer_info,
};

int main(int argc, char** argv) {
    for (size_t i = 0; i < sizeof every / sizeof every[0]; ++i)
        if (!every[i]) return 10;
    CortexCompressionOptions o;
    memset(&o, 0xAB, sizeof o);
    CortexError e = cortex_compression_options_init(&o);
    printf("options %d %zu %d %d %d %d %d %d %d %d %g\n", e.code, o.num_threads, o.verbose,
           o.show_stats, o.use_delta_encoding, o.use_rle, o.compression_level,
           o.use_quantization, o.quantization_bits, o.use_hsdr, (double)o.sparsity);
    printf("errstr %s|%s|%s|%s|%s|%s\n", cortex_error_string(0), cortex_error_string(1),
           cortex_error_string(2), cortex_error_string(3), cortex_error_string(100),
           cortex_error_string(7));
    char** parts = NULL;
    int n = 0;
    int r = cortex_model_get_parts(argv[1], &parts, &n);
    printf("parts %d %d", r, n);
    for (int i = 0; i < n; ++i) {
        const char* s = strrchr(parts[i], '/');
        printf(" %s", s ? s + 1 : parts[i]);
        cortex_free_string(parts[i]);
    }
    free(parts);
    printf("\n");
    for (int a = 2; a < argc; ++a) {
        int has = -1;
        char* type = NULL;
        e = cortex_archive_get_tokenizer_info(argv[a], &has, &type);
        printf("tok %d %d %s\n", e.code, has, type ? type : "-");
        if (type) cortex_free_string(type);
    }
    CortexCompressorHandle ch = (CortexCompressorHandle)1;
    e = cortex_compressor_create("m.gguf", "gguf", &o, &ch);
    printf("compress %d %d %d\n", e.code, ch == NULL, e.message != NULL);
    cortex_error_free(&e);
    e = cortex_compress_from_url("m.gguf", "gguf", "o.sdr", 0.02f);
    printf("url %d\n", e.code);
    e = cortex_archive_extract("a.sdr", "out", 0.02f);
    printf("extract %d\n", e.code);
    e = cortex_compressor_free(NULL);
    printf("free %d\n", e.code);
    return 0;
}
"""


def _build(tmp_path):
    if not os.path.exists(LIB):
        pytest.fail("libcortexsdr_amd.so not built (run __graft_entry__.build())")
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("no gcc")
    src = tmp_path / "ref_caller.c"
    src.write_text(PROG)
    exe = str(tmp_path / "ref_caller")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", str(src), "-o", exe, "-L" + PKG,
                    "-lcortexsdr_amd", "-Wl,-rpath," + PKG, "-Wl,-rpath-link,/opt/rocm/lib"],
                   check=True, capture_output=True, text=True)
    return exe


def test_reference_callers_link_and_host_functions(tmp_path):
    from cortexsdr_amd import formats

    exe = _build(tmp_path)
    # a three-part model set with part 2 missing, and archives with / without tokenizer assets
    for i in (1, 3):
        (tmp_path / f"model-{i:05d}-of-00003.gguf").write_bytes(b"x")
    spm = str(tmp_path / "spm.sdr")
    bpe = str(tmp_path / "bpe.sdr")
    none = str(tmp_path / "none.sdr")
    gguf = str(tmp_path / "gguf.sdr")
    w = np.zeros(4, np.float32)
    formats.write_sdr(spm, [formats.SdrEntry(name="tokenizer.model", payload=b"spm"),
                            formats.SdrEntry(name="w", payload=w.tobytes(), dims=(2, 2))])
    formats.write_sdr(bpe, [formats.SdrEntry(name="tokenizer/vocab.json", payload=b"{}"),
                            formats.SdrEntry(name="tokenizer/merges.txt", payload=b"a b")])
    formats.write_sdr(none, [formats.SdrEntry(name="vocab.json", payload=b"{}"),
                             formats.SdrEntry(name="w", payload=w.tobytes(), dims=(2, 2))])
    formats.write_sdr(gguf, [formats.SdrEntry(name="gguf_tokenizer_model", payload=b"gpt2")])
    out = subprocess.run([exe, str(tmp_path / "model-00003-of-00003.gguf"), spm, bpe, none,
                          gguf, str(tmp_path / "missing.sdr")],
                         check=True, capture_output=True, text=True).stdout.splitlines()
    assert out[0] == "options 0 1 0 0 1 1 6 1 8 0 0.02"
    assert out[1] == ("errstr Success|Invalid argument|File not found|Unsupported format|"
                      "Internal error|Unknown error")
    assert out[2] == "parts 2 2 model-00001-of-00003.gguf model-00003-of-00003.gguf"
    assert out[3] == "tok 0 1 sentencepiece"
    assert out[4] == "tok 0 1 gpt2-bpe"
    assert out[5] == "tok 0 0 -"          # vocab without merges: no tokenizer
    assert out[6] == "tok 0 1 gpt2-bpe"   # gguf_tokenizer_model text names gpt2
    assert out[7].startswith("tok -2 ")   # missing file: CORTEX_ERROR_FILE_IO
    assert out[8] == "compress -4 1 1"
    assert out[9] == "url -4"
    assert out[10] == "extract -4"
    assert out[11] == "free 0"


def test_model_parts_single_file(tmp_path):
    exe = _build(tmp_path)
    (tmp_path / "one.gguf").write_bytes(b"x")
    out = subprocess.run([exe, str(tmp_path / "one.gguf")], check=True, capture_output=True,
                         text=True).stdout.splitlines()
    assert out[2] == "parts 1 1 one.gguf"
