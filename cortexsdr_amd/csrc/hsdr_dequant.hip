// hsdr_dequant.hip — the HSDR compressor's source decode on the GPU (gfx950).
//
// Reference: dequantizeSegmentToFP32 (strategies/HierarchicalSDRStrategy.cpp:713-989), which
// turns a segment's bytes into the fp32 matrix the compressor tiles: bf16, f32, f16, int8
// with (scale, zero point), and the GGUF blocks q4_0 / q8_0 (element 2j from the low nibble
// of byte j, 2j + 1 from the high: :749-764), q4_k / q5_k (element i of a super-block from
// byte i / 2 of the quants, low nibble for even i, 6-bit sub-block scales and mins unpacked
// as :802-814; q5_k's fifth bit from qh[i / 8] bit i % 8), q6_k (two 128-element halves,
// element e of a half from ql[e / 2] and the 2-bit pair (e % 4) of qh[e / 4], sub-block
// scale e / 16). Dispatch follows the reference's: the data_format name first (bf16, q4_0,
// q8_0, q4_k, q5_k, q6_k), then f32 / f16 / int8 by name or segment type.
//
// One thread per output element (grid-stride), the element's block header read through the
// caches. Every value is exact in fp32 (an fp16 scale times a 6-bit scale or an 8-bit
// integer, times a quant of at most 6 bits, minus an equally exact min), so the output is the
// reference's bit for bit whatever the operation order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace {

using csdr::set_error;

constexpr int kThreads = 256;

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return csdr::h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// 6-bit scale and min of sub-block is (0..7) from the 12 packed bytes (:802-814)
__device__ __forceinline__ void k_scale_min(const uint8_t* s12, int is, int& sc, int& mn) {
    if (is < 4) {
        sc = s12[is] & 0x3F;
        mn = s12[is + 4] & 0x3F;
    } else {
        sc = (s12[is + 4] & 0x0F) | ((s12[is - 4] >> 6) << 4);
        mn = (s12[is + 4] >> 4) | ((s12[is] >> 6) << 4);
    }
}

template <int FMT>
__device__ __forceinline__ float decode_one(const uint8_t* __restrict__ src, size_t i, float scale,
                                            float zp) {
    if constexpr (FMT == CSDR_SRC_F32) {
        return reinterpret_cast<const float*>(src)[i];
    } else if constexpr (FMT == CSDR_SRC_F16) {
        return csdr::h2f(reinterpret_cast<const uint16_t*>(src)[i]);
    } else if constexpr (FMT == CSDR_SRC_BF16) {
        return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(src)[i] << 16);
    } else if constexpr (FMT == CSDR_SRC_I8) {
        return ((float)reinterpret_cast<const int8_t*>(src)[i] - zp) * scale;
    } else if constexpr (FMT == CSDR_SRC_Q4_0) {
        const uint8_t* b = src + (i / 32) * 18;
        const int j = (int)(i % 32);
        const uint8_t byte = b[2 + j / 2];
        const int q = ((j & 1) ? (byte >> 4) : (byte & 0x0F)) - 8;
        return (float)q * f16_at(b);
    } else if constexpr (FMT == CSDR_SRC_Q8_0) {
        const uint8_t* b = src + (i / 32) * 34;
        return (float)(int8_t)b[2 + i % 32] * f16_at(b);
    } else if constexpr (FMT == CSDR_SRC_Q4_K || FMT == CSDR_SRC_Q5_K) {
        constexpr int kBytes = FMT == CSDR_SRC_Q4_K ? 144 : 176;
        const uint8_t* b = src + (i / 256) * kBytes;
        const int idx = (int)(i % 256);
        int sc, mn;
        k_scale_min(b + 4, idx / 32, sc, mn);
        const float ds = f16_at(b) * (float)sc;
        const float dm = f16_at(b + 2) * (float)mn;
        const uint8_t* qs = b + (FMT == CSDR_SRC_Q4_K ? 16 : 48);
        const uint8_t byte = qs[idx / 2];
        int q = (idx & 1) ? (byte >> 4) : (byte & 0x0F);
        if constexpr (FMT == CSDR_SRC_Q5_K) q |= ((b[16 + idx / 8] >> (idx % 8)) & 1) << 4;
        return (float)q * ds - dm;
    } else {  // CSDR_SRC_Q6_K
        const uint8_t* b = src + (i / 256) * 210;
        const int idx = (int)(i % 256), half = idx / 128, e = idx % 128;
        const float ds = f16_at(b + 208) * (float)(int8_t)b[192 + half * 8 + e / 16];
        const uint8_t qlb = b[half * 64 + e / 2];
        const int lo = (e & 1) ? (qlb >> 4) : (qlb & 0x0F);
        const int hi = (b[128 + half * 32 + e / 4] >> ((e % 4) * 2)) & 3;
        return (float)(((hi << 4) | lo) - 32) * ds;
    }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void source_decode_kernel(const uint8_t* __restrict__ src,
                                                                 size_t n, float scale, float zp,
                                                                 float* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads)
        out[i] = decode_one<FMT>(src, i, scale, zp);
}

// Bytes and elements per block of a source format (elements are single values for the plain
// formats).
bool block_geometry(int fmt, size_t& bytes, size_t& elems) {
    switch (fmt) {
        case CSDR_SRC_F32: bytes = 4, elems = 1; return true;
        case CSDR_SRC_F16:
        case CSDR_SRC_BF16: bytes = 2, elems = 1; return true;
        case CSDR_SRC_I8: bytes = 1, elems = 1; return true;
        case CSDR_SRC_Q4_0: bytes = 18, elems = 32; return true;
        case CSDR_SRC_Q8_0: bytes = 34, elems = 32; return true;
        case CSDR_SRC_Q4_K: bytes = 144, elems = 256; return true;
        case CSDR_SRC_Q5_K: bytes = 176, elems = 256; return true;
        case CSDR_SRC_Q6_K: bytes = 210, elems = 256; return true;
        default: return false;
    }
}

}  // namespace

extern "C" {

CSDR_API int csdr_hsdr_source_format(const char* data_format, int segment_type) {
    std::string f;
    for (const char* p = data_format ? data_format : ""; *p; ++p)
        f.push_back((char)std::tolower((unsigned char)*p));
    if (f == "bf16" || f == "bfloat16") return CSDR_SRC_BF16;
    if (f == "q4_0") return CSDR_SRC_Q4_0;
    if (f == "q8_0") return CSDR_SRC_Q8_0;
    if (f == "q4_k") return CSDR_SRC_Q4_K;
    if (f == "q5_k") return CSDR_SRC_Q5_K;
    if (f == "q6_k") return CSDR_SRC_Q6_K;
    if (segment_type == 1 || f == "f32" || f == "fp32" || f == "float32") return CSDR_SRC_F32;
    if (segment_type == 2 || f == "f16" || f == "fp16" || f == "float16" || f == "half")
        return CSDR_SRC_F16;
    if (segment_type == 3 || f == "i8" || f == "int8") return CSDR_SRC_I8;
    return -1;
}

CSDR_API size_t csdr_hsdr_source_elements(int format, size_t nbytes) {
    size_t bb = 0, be = 0;
    if (!block_geometry(format, bb, be) || nbytes % bb) return 0;
    return nbytes / bb * be;
}

CSDR_API int csdr_hsdr_source_decode(const void* src, size_t nbytes, int format, float scale,
                                     float zero_point, float* out, void* hip_stream) {
    size_t bb = 0, be = 0;
    if (!block_geometry(format, bb, be))
        return set_error(CSDR_E_UNSUPPORTED, "hsdr_source_decode: unsupported source format " +
                                                 std::to_string(format));
    if (nbytes % bb)
        return set_error(CSDR_E_FORMAT, "hsdr_source_decode: byte size not a multiple of " +
                                            std::to_string(bb));
    if (!src || !out) return set_error(CSDR_E_INVALID, "hsdr_source_decode: null buffer");
    if ((format == CSDR_SRC_F32 && reinterpret_cast<uintptr_t>(src) % 4) ||
        ((format == CSDR_SRC_F16 || format == CSDR_SRC_BF16) && reinterpret_cast<uintptr_t>(src) % 2))
        return set_error(CSDR_E_INVALID, "hsdr_source_decode: source misaligned for its format");
    const size_t n = nbytes / bb * be;
    if (!n) return CSDR_OK;
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const unsigned grid = (unsigned)std::min<size_t>((n + kThreads - 1) / kThreads, 65536);
    const auto* s = static_cast<const uint8_t*>(src);
    switch (format) {
        case CSDR_SRC_F32: source_decode_kernel<CSDR_SRC_F32><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_F16: source_decode_kernel<CSDR_SRC_F16><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_BF16: source_decode_kernel<CSDR_SRC_BF16><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_I8: source_decode_kernel<CSDR_SRC_I8><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_Q4_0: source_decode_kernel<CSDR_SRC_Q4_0><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_Q8_0: source_decode_kernel<CSDR_SRC_Q8_0><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_Q4_K: source_decode_kernel<CSDR_SRC_Q4_K><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        case CSDR_SRC_Q5_K: source_decode_kernel<CSDR_SRC_Q5_K><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
        default: source_decode_kernel<CSDR_SRC_Q6_K><<<grid, kThreads, 0, st>>>(s, n, scale, zero_point, out); break;
    }
    CSDR_LAUNCH_CHECK("hsdr_source_decode");
    return CSDR_OK;
}

CSDR_API int csdr_hsdr_compress_source(const void* src, size_t nbytes, int format, float scale,
                                       float zero_point, uint32_t rows, uint32_t cols,
                                       uint16_t tile_rows, uint16_t tile_cols, uint16_t n_atoms,
                                       uint8_t n_stages, uint8_t k_per_stage, uint8_t ksvd_iters,
                                       float stage_decay, uint8_t* out, size_t out_bytes,
                                       void* hip_stream) {
    size_t bb = 0, be = 0;
    if (!block_geometry(format, bb, be))
        return set_error(CSDR_E_UNSUPPORTED, "hsdr_compress_source: unsupported source format " +
                                                 std::to_string(format));
    if (nbytes % bb)
        return set_error(CSDR_E_FORMAT, "hsdr_compress_source: byte size not a multiple of " +
                                            std::to_string(bb));
    const size_t n = nbytes / bb * be;
    if ((size_t)rows * cols != n || n == 0)
        return set_error(CSDR_E_INVALID, "hsdr_compress_source: " + std::to_string(n) +
                                             " decoded values for a " + std::to_string(rows) +
                                             " x " + std::to_string(cols) + " matrix");
    float* w = nullptr;
    CSDR_HIP_CHECK(hipMalloc(&w, std::max<size_t>(n, 1) * 4));
    int rc = csdr_hsdr_source_decode(src, nbytes, format, scale, zero_point, w, hip_stream);
    std::vector<float> host;
    if (rc == CSDR_OK) {
        // the dictionary initialisation runs on the host over the decoded matrix
        try {
            host.resize(n);
        } catch (const std::exception&) {
            rc = set_error(CSDR_E_INVALID, "hsdr_compress_source: out of host memory");
        }
    }
    if (rc == CSDR_OK &&
        (hipMemcpyAsync(host.data(), w, n * 4, hipMemcpyDeviceToHost,
                        static_cast<hipStream_t>(hip_stream)) != hipSuccess ||
         hipStreamSynchronize(static_cast<hipStream_t>(hip_stream)) != hipSuccess))
        rc = set_error(CSDR_E_HIP, "hsdr_compress_source: copy of the decoded matrix failed");
    (void)hipFree(w);
    if (rc != CSDR_OK) return rc;
    return csdr_hsdr_compress(host.data(), rows, cols, tile_rows, tile_cols, n_atoms, n_stages,
                              k_per_stage, ksvd_iters, stage_decay, out, out_bytes, hip_stream);
}

}  // extern "C"
