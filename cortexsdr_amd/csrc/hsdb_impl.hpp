// hsdb_impl.hpp — the device-resident segment shared by the HSDB kernels (hsdb.hip: parse,
// M == 1 and generic products, decode; hsdb_mfma.hip: the batched MFMA product).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"

struct csdr_hsdb {
    uint32_t R = 0, C = 0, tile_rows = 1, tile_cols = 0, K = 0, S = 0, k = 0, slots = 0;
    uint32_t n_row_tiles = 0, NB = 0, n_tiles = 0, R_full = 0, C_full = 0, Ce = 0;
    uint32_t NBc = 1, nchunks = 1;
    int is_hsdb = 0;
    int device = 0;
    float* d_dict = nullptr;        // K x tile_dim fp32
    _Float16* d_dict16p = nullptr;  // 64-wide blocks: K x 64 fp16, rows in kperm64 order
    uint32_t* d_codes = nullptr;    // n_tiles * slots words
    float* d_slot_gamma = nullptr;  // slots floats: gamma[j / k]
    float* d_edge = nullptr;        // top-right strip (R_full x Ce) then bottom strip
    float h_slot_gamma[32] = {};    // host copy of the first 32 slot gammas (kernel args)
    size_t edge_floats = 0;
    size_t device_bytes = 0;
};

namespace csdr {

// Position of k (0..63) inside a 64-long block stored in the matrix-core k order: with
// k = 16s + 4q + i (s, q, i in 0..3) it sits at 16q + 4s + i, so the 16 values a lane
// feeds to four 16-deep MFMA steps are contiguous. An involution.
__host__ __device__ __forceinline__ int kperm64(int k) {
    return (k & 3) | ((k >> 2) & 3) << 4 | ((k >> 4) & 3) << 2;
}

// Batched (M >= 2) product on matrix cores: decoded 64-column tiles times X (fp16 MFMA,
// fp32 accumulation). eligible(): every matrix has 1-row tiles of 64, at most 1024 atoms
// and 4, 8 or 16 slots, and CSDR_HSDB_MFMA is not 0.
bool mfma_eligible(int n, const csdr_hsdb* const* segs, int M);
size_t mfma_workspace_bytes(int n, const csdr_hsdb* const* segs, int M);
int mfma_matmul(int n, const csdr_hsdb* const* segs, const void* const* xs, int x_dtype, int M,
                float* const* ys, const float* const* bias, int accumulate, void* workspace,
                size_t workspace_bytes, hipStream_t st);

}  // namespace csdr
