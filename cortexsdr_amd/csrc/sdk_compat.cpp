// sdk_compat.cpp — the rest of the reference SDK's C surface, so that its own callers link
// against libcortexsdr_amd.so unchanged.
//
// Reference (cortexSDR tree): api/c_api.hpp:46-117 (options, compressor, decompressor,
// archive extraction, multi-part detection, error strings; implementations api/c_api.cpp) and
// api/cortex_sdk.h:252-281 (cortex_compress_from_url, cortex_archive_get_tokenizer_info,
// cortex_archive_extract; implementations api/cortex_sdk.cpp:2096-2170). Callers:
// src/cortexsdr_cli.cpp:918 (tokenizer probe), :1639 (compress from URL) and the Python
// wrapper python/cortexsdr_sdk/_bindings.cpp:28,55 (compressor / decompressor classes).
//
// What is served here:
//   - host-only functions with their reference behaviour: cortex_compression_options_init
//     (c_api.cpp:298-317 defaults), cortex_error_string (:680-689), cortex_model_get_parts
//     (findModelParts, :55-110: "<base>-NNNNN-of-MMMMM<ext>" siblings that exist, else the
//     path itself), cortex_archive_get_tokenizer_info (the archive-index name scan of
//     cortex_sdk.cpp:2109-2145, read through this library's .sdr reader);
//   - the compression / extraction family (model parsers, strategy chain, archive writer):
//     outside the coded-weight inference path, so each returns
//     CORTEX_ERROR_UNSUPPORTED_FORMAT with a library-owned message and no handle; the free
//     functions accept NULL.
// Strings handed to the caller are malloc'd (released with cortex_free_string, i.e. free);
// error messages are thread-local and owned by the library.
#include <algorithm>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <filesystem>
#include <regex>
#include <string>
#include <vector>

#include "../../include/cortex_sdk_gpu.h"

namespace {

thread_local std::string t_msg;

CortexError ok() { return {nullptr, CORTEX_SUCCESS}; }
CortexError fail(int code, const std::string& m) {
    t_msg = m;
    return {t_msg.c_str(), code};
}

// No C++ exception crosses the C ABI: every CortexError entry point runs its body inside
// CORTEX_GUARD_BEGIN ... CORTEX_GUARD_END(name), which turns std::bad_alloc into
// CORTEX_ERROR_MEMORY and any other exception into CORTEX_ERROR_UNKNOWN with its message.
#define CORTEX_GUARD_BEGIN try {
#define CORTEX_GUARD_END(fn_)                                                            \
    }                                                                                    \
    catch (const std::bad_alloc&) {                                                      \
        return fail(CORTEX_ERROR_MEMORY, std::string(fn_) + ": out of host memory");    \
    }                                                                                    \
    catch (const std::exception& ex_) {                                                  \
        return fail(CORTEX_ERROR_UNKNOWN, std::string(fn_) + ": " + ex_.what());        \
    }                                                                                    \
    catch (...) {                                                                        \
        return fail(CORTEX_ERROR_UNKNOWN, std::string(fn_) + ": unknown exception");    \
    }
CortexError unsupported(const char* what) {
    return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                std::string(what) +
                    ": model compression and archive extraction are not part of the MI355X "
                    "inference library (it reads .sdr archives and runs coded weights)");
}

char* dup_c(const std::string& s) {
    char* p = static_cast<char*>(std::malloc(s.size() + 1));
    if (p) std::memcpy(p, s.c_str(), s.size() + 1);
    return p;
}

std::string lower(std::string s) {
    for (auto& c : s) c = (char)std::tolower((unsigned char)c);
    return s;
}

// Parts of a Hugging Face style multi-part model ("<base>-00001-of-00005<ext>"): every part
// of the set that exists, in order; the path itself when it is not part of a set, when no
// sibling exists, or when the path does not exist.
std::vector<std::string> model_parts(const std::string& model_path) {
    namespace fs = std::filesystem;
    std::error_code ec;
    const fs::path path(model_path);
    if (!fs::exists(path, ec)) return {model_path};
    fs::path parent = path.parent_path();
    if (parent.empty()) parent = fs::current_path(ec);
    const std::string name = path.filename().string();
    static const std::regex pat(R"(^(.+)-(\d+)-of-(\d+)(\..+)$)");
    std::smatch m;
    if (std::regex_match(name, m, pat)) {
        const std::string base = m[1].str(), ext = m[4].str();
        const int total = std::atoi(m[3].str().c_str());
        std::vector<std::string> parts;
        for (int i = 1; i <= total && i <= 100000; ++i) {
            char mid[64];
            std::snprintf(mid, sizeof mid, "-%05d-of-%05d", i, total);
            const fs::path p = parent / (base + mid + ext);
            if (fs::exists(p, ec)) parts.push_back(p.string());
        }
        if (!parts.empty()) return parts;
    }
    return {model_path};
}

}  // namespace

extern "C" {

CSDR_API CortexError cortex_compression_options_init(CortexCompressionOptions* options) {
    CORTEX_GUARD_BEGIN
    if (!options) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid options pointer");
    options->num_threads = 1;
    options->verbose = 0;
    options->show_stats = 0;
    options->use_delta_encoding = 1;
    options->use_rle = 1;
    options->compression_level = 6;
    options->use_quantization = 1;
    options->quantization_bits = 8;
    options->use_hsdr = 0;
    options->sparsity = 0.02f;
    return ok();
    CORTEX_GUARD_END("cortex_compression_options_init")
}

CSDR_API const char* cortex_error_string(int code) {
    switch (code) {
        case CORTEX_OK: return "Success";
        case CORTEX_ERR_INVALID_ARG: return "Invalid argument";
        case CORTEX_ERR_FILE_NOT_FOUND: return "File not found";
        case CORTEX_ERR_UNSUPPORTED_FORMAT: return "Unsupported format";
        case CORTEX_ERR_INTERNAL: return "Internal error";
        default: return "Unknown error";
    }
}

CSDR_API int cortex_model_get_parts(const char* model_path, char*** parts_out, int* num_parts) {
    if (!model_path) return 0;
    try {
        const std::vector<std::string> parts = model_parts(model_path);
        if (num_parts) *num_parts = (int)parts.size();
        if (parts_out) {
            *parts_out = static_cast<char**>(std::malloc(parts.size() * sizeof(char*)));
            if (!*parts_out) return 0;
            for (size_t i = 0; i < parts.size(); ++i) (*parts_out)[i] = dup_c(parts[i]);
        }
        return (int)parts.size();
    } catch (const std::exception&) {
        return 0;
    }
}

CSDR_API CortexError cortex_archive_get_tokenizer_info(const char* archive_path,
                                                       int* out_has_tokenizer,
                                                       char** out_tokenizer_type) {
    CORTEX_GUARD_BEGIN
    if (!archive_path || !out_has_tokenizer)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid argument(s)");
    *out_has_tokenizer = 0;
    if (out_tokenizer_type) *out_tokenizer_type = nullptr;
    csdr_archive* ar = nullptr;
    const int rc = csdr_archive_open(archive_path, &ar);
    if (rc)
        return fail(rc == CSDR_E_INVALID ? CORTEX_ERROR_FILE_IO : CORTEX_ERROR_DECOMPRESSION,
                    csdr_last_error());
    bool spm = false, vocab = false, merges = false, gpt2 = false;
    try {
        const size_t n = csdr_archive_count(ar);
        for (size_t i = 0; i < n; ++i) {
            csdr_segment_info info;
            if (csdr_archive_info(ar, i, &info) != CSDR_OK) continue;
            const std::string nm = lower(info.name ? info.name : "");
            if (nm.find("tokenizer.model") != std::string::npos ||
                nm.find("sentencepiece") != std::string::npos ||
                nm.find(".spm") != std::string::npos)
                spm = true;
            if (nm.find("vocab") != std::string::npos) vocab = true;
            if (nm.find("merges") != std::string::npos) merges = true;
            // the GGUF tokenizer-model string names the family; a raw (strategy 0) payload is
            // the text itself
            if (nm == "gguf_tokenizer_model" && info.strategy_id == 0 &&
                info.compressed_size < ((uint64_t)1 << 26)) {
                std::string text((size_t)info.compressed_size, '\0');
                size_t got = 0;
                if (csdr_archive_read(ar, i, text.data(), text.size(), &got) == CSDR_OK) {
                    const std::string lt = lower(text.substr(0, got));
                    spm = spm || lt.find("sentencepiece") != std::string::npos;
                    gpt2 = gpt2 || lt.find("gpt2") != std::string::npos;
                }
            }
        }
    } catch (const std::exception& ex) {
        csdr_archive_close(ar);
        return fail(CORTEX_ERROR_UNKNOWN, ex.what());
    }
    csdr_archive_close(ar);
    if (spm || gpt2 || (vocab && merges)) {
        *out_has_tokenizer = 1;
        if (out_tokenizer_type) *out_tokenizer_type = dup_c(spm ? "sentencepiece" : "gpt2-bpe");
    }
    return ok();
    CORTEX_GUARD_END("cortex_archive_get_tokenizer_info")
}

CSDR_API CortexError cortex_compressor_create(const char* model_path, const char* format,
                                              const CortexCompressionOptions* options,
                                              CortexCompressorHandle* handle) {
    CORTEX_GUARD_BEGIN
    (void)model_path;
    (void)format;
    (void)options;
    if (handle) *handle = nullptr;
    return unsupported("cortex_compressor_create");
    CORTEX_GUARD_END("cortex_compressor_create")
}

CSDR_API CortexError cortex_compressor_add_file(CortexCompressorHandle handle,
                                                const char* model_path) {
    CORTEX_GUARD_BEGIN
    (void)handle;
    (void)model_path;
    return unsupported("cortex_compressor_add_file");
    CORTEX_GUARD_END("cortex_compressor_add_file")
}

CSDR_API CortexError cortex_compressor_compress(CortexCompressorHandle handle,
                                                const char* output_path) {
    CORTEX_GUARD_BEGIN
    (void)handle;
    (void)output_path;
    return unsupported("cortex_compressor_compress");
    CORTEX_GUARD_END("cortex_compressor_compress")
}

CSDR_API CortexError cortex_compressor_get_stats(CortexCompressorHandle handle,
                                                 size_t* original_size, size_t* compressed_size,
                                                 double* compression_ratio,
                                                 double* compression_time_ms) {
    CORTEX_GUARD_BEGIN
    (void)handle;
    (void)original_size;
    (void)compressed_size;
    (void)compression_ratio;
    (void)compression_time_ms;
    return unsupported("cortex_compressor_get_stats");
    CORTEX_GUARD_END("cortex_compressor_get_stats")
}

CSDR_API CortexError cortex_compressor_free(CortexCompressorHandle handle) {
    CORTEX_GUARD_BEGIN
    if (handle) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid compressor handle");
    return ok();
    CORTEX_GUARD_END("cortex_compressor_free")
}

CSDR_API CortexError cortex_decompressor_create(const char* compressed_path,
                                                CortexDecompressorHandle* handle, float sparsity) {
    CORTEX_GUARD_BEGIN
    (void)compressed_path;
    (void)sparsity;
    if (handle) *handle = nullptr;
    return unsupported("cortex_decompressor_create");
    CORTEX_GUARD_END("cortex_decompressor_create")
}

CSDR_API CortexError cortex_decompressor_decompress(CortexDecompressorHandle handle,
                                                    const char* compressed_path,
                                                    const char* output_path) {
    CORTEX_GUARD_BEGIN
    (void)handle;
    (void)compressed_path;
    (void)output_path;
    return unsupported("cortex_decompressor_decompress");
    CORTEX_GUARD_END("cortex_decompressor_decompress")
}

CSDR_API CortexError cortex_decompressor_free(CortexDecompressorHandle handle) {
    CORTEX_GUARD_BEGIN
    if (handle) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid decompressor handle");
    return ok();
    CORTEX_GUARD_END("cortex_decompressor_free")
}

CSDR_API CortexError cortex_archive_extract(const char* compressed_path, const char* output_dir,
                                            float sparsity) {
    CORTEX_GUARD_BEGIN
    (void)compressed_path;
    (void)output_dir;
    (void)sparsity;
    return unsupported("cortex_archive_extract");
    CORTEX_GUARD_END("cortex_archive_extract")
}

CSDR_API CortexError cortex_compress_from_url(const char* url_or_path, const char* format,
                                              const char* output_path, float sparsity) {
    CORTEX_GUARD_BEGIN
    (void)url_or_path;
    (void)format;
    (void)output_path;
    (void)sparsity;
    return unsupported("cortex_compress_from_url");
    CORTEX_GUARD_END("cortex_compress_from_url")
}

}  // extern "C"
