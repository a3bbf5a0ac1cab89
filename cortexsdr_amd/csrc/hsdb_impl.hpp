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
    float* d_dict = nullptr;        // K x tile_dim fp32 (shared, see dict_ref)
    _Float16* d_dict16p = nullptr;  // 64-wide blocks: K x 64 fp16, rows in kperm64 order
    uint32_t* d_codes = nullptr;    // n_tiles * slots words (null for host-resident codes)
    uint32_t* h_codes = nullptr;    // host-resident segments: the same words in pinned host
                                    // memory (a decoder streams them to the device per layer)
    float* d_slot_gamma = nullptr;  // slots floats: gamma[j / k]
    float* d_edge = nullptr;        // top-right strip (R_full x Ce) then bottom strip
    float h_slot_gamma[32] = {};    // host copy of the first 32 slot gammas (kernel args)
    size_t edge_floats = 0;
    // the device dictionary (d_dict, d_dict16p) is held through a reference-counted entry
    // shared by every segment on the device with the same dictionary bytes and tile shape
    void* dict_ref = nullptr;
    size_t device_bytes = 0;
};

namespace csdr {

// Bytes of the segment's device code words (4 per slot).
inline size_t code_bytes(const csdr_hsdb* s) { return (size_t)s->n_tiles * s->slots * 4; }

// The kernels read code words from device memory: false for a host-resident segment (whose
// words are in pinned host memory until a caller stages them).
inline bool codes_on_device(const csdr_hsdb* s) { return s->d_codes || code_bytes(s) == 0; }

// ---- chunk-major code layout of 1-row tiles
// Block columns are grouped in chunks: full chunks of NBc (a power of two) columns, then the
// remainder NB % NBc split into power-of-two chunks, largest first (e.g. NB = 14, NBc = 8:
// widths 8, 4, 2). Chunk c covering columns [b0, b0 + nbc) is stored at word b0 * R * slots,
// each row's nbc tiles back to back, so every chunk's rows form one contiguous run and every
// row of a chunk spans a power-of-two number of 16-byte pieces.
__host__ __device__ __forceinline__ uint32_t n_chunks(uint32_t NB, uint32_t NBc) {
    return NB / NBc + (uint32_t)__builtin_popcount(NB % NBc);
}

// First column b0 and width nbc of chunk c (nbc = 0 past the last chunk).
__host__ __device__ __forceinline__ void chunk_span(uint32_t c, uint32_t NB, uint32_t NBc,
                                                   uint32_t& b0, uint32_t& nbc) {
    const uint32_t nfull = NB / NBc;
    if (c < nfull) {
        b0 = c * NBc;
        nbc = NBc;
        return;
    }
    const uint32_t rem = NB - nfull * NBc;
    b0 = nfull * NBc;
    c -= nfull;
    nbc = 0;
    for (uint32_t bit = NBc >> 1; bit; bit >>= 1) {
        if (!(rem & bit)) continue;
        if (c == 0) {
            nbc = bit;
            return;
        }
        --c;
        b0 += bit;
    }
}

// Chunk c, first column b0 and width nbc of the chunk holding block column b (b < NB).
__host__ __device__ __forceinline__ void chunk_of(uint32_t b, uint32_t NB, uint32_t NBc,
                                                 uint32_t& c, uint32_t& b0, uint32_t& nbc) {
    const uint32_t nfull = NB / NBc;
    if (b < nfull * NBc) {
        c = b / NBc;
        b0 = c * NBc;
        nbc = NBc;
        return;
    }
    const uint32_t rem = NB - nfull * NBc;
    c = nfull;
    b0 = nfull * NBc;
    nbc = 0;
    for (uint32_t bit = NBc >> 1; bit; bit >>= 1) {
        if (!(rem & bit)) continue;
        if (b < b0 + bit) {
            nbc = bit;
            return;
        }
        ++c;
        b0 += bit;
    }
}

// Word offset of tile (r, b) (its first slot) in the chunk-major layout.
__host__ __device__ __forceinline__ size_t tile_word_offset(uint32_t r, uint32_t b, uint32_t R,
                                                           uint32_t NB, uint32_t NBc,
                                                           uint32_t slots) {
    uint32_t c, b0, nbc;
    chunk_of(b, NB, NBc, c, b0, nbc);
    return ((size_t)b0 * R + (size_t)r * nbc + (b - b0)) * slots;
}

// Every product workspace starts with kWsHead bytes (the RMSNorm x op's per-column 1 / rms at
// M > 1: 16 floats per matrix of a group of up to 8); the data (P, transposed X) follows.
constexpr size_t kWsHead = 1024;

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
// token_major: X is M x C and Y is M x R (else C x M and R x M).
int mfma_matmul(int n, const csdr_hsdb* const* segs, const void* const* xs, int x_dtype, int M,
                float* const* ys, const float* const* bias, int accumulate, int token_major,
                void* workspace, size_t workspace_bytes, hipStream_t st);

}  // namespace csdr
