// common.hpp — shared host/device helpers of the cortexsdr_amd HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/cortexsdr_hip.h"

namespace csdr {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string& msg);
void clear_error();
const char* last_error();

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Decode attention split partials in a workspace, n of them: the n (max, sum) pairs, then the
// n unnormalised head_dim vectors from this float offset (16-byte aligned).
__host__ __device__ inline size_t attn_vec_offset(size_t n) { return (2 * n + 3) & ~(size_t)3; }

// Penalised argmax of `rows` rows of n scores (csdr_select_best per row; the position
// advances once). Workspace select_workspace_rows(rows) bytes.
size_t select_workspace_rows(int rows);
int select_best_rows(const float* logits, int n, int rows, const uint8_t* repeated,
                     float temperature, float penalty, int* out_tokens, int* pos_dev,
                     uint8_t* repeated_update, void* workspace, size_t workspace_bytes,
                     hipStream_t st);

#define CSDR_HIP_CHECK(expr)                                                          \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::csdr::set_error(CSDR_E_HIP, std::string(#expr " failed: ") +      \
                                                     hipGetErrorString(e_));           \
    } while (0)

// Launch-status check after a kernel launch.
#define CSDR_LAUNCH_CHECK(what)                                                       \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess)                                                          \
            return ::csdr::set_error(CSDR_E_HIP, std::string(what) + " launch failed: " + \
                                                     hipGetErrorString(e_));           \
    } while (0)

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) {
    return v;
}
template <>
__device__ __forceinline__ float to_f32<_Float16>(_Float16 v) {
    return static_cast<float>(v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace csdr
