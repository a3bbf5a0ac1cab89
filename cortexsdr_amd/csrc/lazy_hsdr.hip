// lazy_hsdr.hip — the text CLI's lazy HSDR embedding on the GPU (gfx950): row decode and
// vocabulary scoring straight from the codes, without the dense vocab x hidden table.
//
// Reference (src/cortexsdr_cli.cpp): parse_hsdr_codes_for_embedding :488-534 (the 36-byte HSDR
// header, 1-row tiles: vocabulary = n_tiles rows of tile_cols; then stage scales, atoms
// K x C, packed codes), hsdr_decode_row :536-554 and select_next_token_from_lazy_hsdr
// :687-732. Code words are read either as packIndexSign wrote them (bit 15 sign, bits 0-14
// index; HierarchicalSDRStrategy.cpp:76-84) or as the CLI reads them (index = v >> 1, sign =
// v & 1, :545-546, :716-717), chosen at load; indices >= K are skipped.
//
// Selection, per sequence row:
//   lazy_ah_kernel     ah[a] = float(sum_c double(atom[a][c]) * hidden[c]): one thread per atom
//                      adding the (exact) fp64 products in feature order, as the CLI does, so
//                      ah is the CLI's value bit for bit;
//   lazy_score_kernel  one thread per token: the float sum over its slots in order of
//                      (gamma_l * sign) * ah[idx] (separately rounded multiply and add, as the
//                      CLI's source evaluates it), optionally stored, times 1 / temperature
//                      (temperature > 0), minus the penalty when the token was generated;
//                      a workgroup's best (strictly larger wins, the lower index on ties);
//   lazy_pick_kernel   the best over the workgroups; optionally advances a device position and
//                      marks the token generated (a captured decode step reads and writes
//                      both on the device).
// A score that is NaN or -infinity never wins (the CLI's strict comparison against an initial
// -infinity); the token is -1 when no score wins.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>

#include "common.hpp"

struct csdr_lazy_hsdr {
    uint32_t R = 0, C = 0, K = 0, S = 0, k = 0;
    int unpack = CSDR_LAZY_UNPACK_PACKED;
    float* gamma = nullptr;     // S
    float* atoms = nullptr;     // K x C
    uint16_t* packed = nullptr; // R x S*k
};

namespace {

using csdr::set_error;

constexpr int kThreads = 256;
constexpr int kPickBlocks = 256;  // workgroups of the score pass, at most

__device__ __forceinline__ void lazy_code(uint16_t v, int unpack, uint32_t& idx, float& sgn) {
    if (unpack == CSDR_LAZY_UNPACK_CLI) {
        idx = v >> 1;
        sgn = (v & 1u) ? -1.0f : 1.0f;
    } else {
        idx = v & 0x7FFFu;
        sgn = (v & 0x8000u) ? -1.0f : 1.0f;
    }
}

// Row blockIdx.y of out (C floats) = token rows_dev[blockIdx.y] (or row_host) decoded: threads
// over the features, the slots in order for each (zeros for a token outside the vocabulary).
__global__ __launch_bounds__(kThreads) void lazy_row_kernel(csdr_lazy_hsdr h, const int* rows_dev,
                                                            int row_host, float* __restrict__ out) {
    const int r = rows_dev ? rows_dev[blockIdx.y] : row_host;
    float* o = out + (size_t)blockIdx.y * h.C;
    const bool live = r >= 0 && (uint32_t)r < h.R;
    const size_t slots = (size_t)h.S * h.k;
    for (uint32_t c = blockIdx.x * kThreads + threadIdx.x; c < h.C; c += gridDim.x * kThreads) {
        float acc = 0.0f;
        if (live) {
            const uint16_t* code = h.packed + (size_t)r * slots;
            for (uint32_t l = 0; l < h.S; ++l) {
                const float g = h.gamma[l];
                for (uint32_t b = 0; b < h.k; ++b) {
                    uint32_t idx;
                    float sgn;
                    lazy_code(code[l * h.k + b], h.unpack, idx, sgn);
                    if (idx >= h.K) continue;
                    acc = __fadd_rn(acc, __fmul_rn(g * sgn, h.atoms[(size_t)idx * h.C + c]));
                }
            }
        }
        o[c] = acc;
    }
}

// ah[row][a] = (float) sum_c atom_a[c] * hidden[c] in fp64, one thread per atom adding the
// products in feature order, as the CLI's loop does (cortexsdr_cli.cpp:700-704): each product
// of two floats is exact in fp64, so the sum's rounding sequence, and the float it rounds to,
// is the reference's. The workgroup's atoms are staged kAhTile features at a time through LDS
// (coalesced row reads; rows padded by one float so a column read meets distinct banks).
constexpr int kAhTile = 32;

__global__ __launch_bounds__(kThreads) void lazy_ah_kernel(csdr_lazy_hsdr h,
                                                           const float* __restrict__ hidden,
                                                           float* __restrict__ ah) {
    __shared__ float tile[kThreads * (kAhTile + 1)];
    __shared__ float xs[kAhTile];
    const int tid = threadIdx.x;
    const uint32_t a0 = blockIdx.x * kThreads;
    const int row = blockIdx.y;
    const float* x = hidden + (size_t)row * h.C;
    double s = 0.0;
    for (uint32_t c0 = 0; c0 < h.C; c0 += kAhTile) {
        const uint32_t nc = min((uint32_t)kAhTile, h.C - c0);
        __syncthreads();
        // atoms a0 .. a0 + kThreads - 1, features c0 .. c0 + nc - 1: consecutive threads read
        // consecutive features of one atom
        for (uint32_t i = tid; i < (uint32_t)kThreads * kAhTile; i += kThreads) {
            const uint32_t r = i / kAhTile, c = i - r * kAhTile;
            const uint32_t a = a0 + r;
            tile[r * (kAhTile + 1) + c] =
                (a < h.K && c < nc) ? h.atoms[(size_t)a * h.C + c0 + c] : 0.0f;
        }
        if (tid < kAhTile) xs[tid] = tid < (int)nc ? x[c0 + tid] : 0.0f;
        __syncthreads();
        const float* t = tile + tid * (kAhTile + 1);
        for (uint32_t c = 0; c < nc; ++c) s += (double)t[c] * (double)xs[c];
    }
    if (a0 + tid < h.K) ah[(size_t)row * h.K + a0 + tid] = (float)s;
}

__device__ __forceinline__ bool better(float s, int i, float bs, int bi) {
    return i >= 0 && (bi < 0 || s > bs || (s == bs && i < bi));
}

__global__ __launch_bounds__(kThreads) void lazy_score_kernel(
    csdr_lazy_hsdr h, const float* __restrict__ ah_all, const uint8_t* __restrict__ repeated,
    float ts, float penalty, float* __restrict__ scores, float* __restrict__ ws_s,
    int* __restrict__ ws_i) {
    const int row = blockIdx.y;
    const float* ah = ah_all + (size_t)row * h.K;
    const uint8_t* rep = repeated ? repeated + (size_t)row * h.R : nullptr;
    __shared__ float ss[kThreads];
    __shared__ int si[kThreads];
    const size_t slots = (size_t)h.S * h.k;
    float bs = -INFINITY;
    int bi = -1;
    for (uint32_t t = blockIdx.x * kThreads + threadIdx.x; t < h.R; t += gridDim.x * kThreads) {
        const uint16_t* code = h.packed + (size_t)t * slots;
        float score = 0.0f;
        for (uint32_t l = 0; l < h.S; ++l) {
            const float g = h.gamma[l];
            for (uint32_t b = 0; b < h.k; ++b) {
                uint32_t idx;
                float sgn;
                lazy_code(code[l * h.k + b], h.unpack, idx, sgn);
                if (idx >= h.K) continue;
                score = __fadd_rn(score, __fmul_rn(g * sgn, ah[idx]));
            }
        }
        if (scores) scores[(size_t)row * h.R + t] = score;
        score = __fmul_rn(score, ts);
        if (rep && rep[t]) score = __fsub_rn(score, penalty);
        if (score > bs) {  // strictly larger (NaN and -inf never win); t ascends per thread
            bs = score;
            bi = (int)t;
        }
    }
    ss[threadIdx.x] = bs;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off && better(ss[threadIdx.x + off], si[threadIdx.x + off],
                                        ss[threadIdx.x], si[threadIdx.x])) {
            ss[threadIdx.x] = ss[threadIdx.x + off];
            si[threadIdx.x] = si[threadIdx.x + off];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ws_s[(size_t)row * gridDim.x + blockIdx.x] = ss[0];
        ws_i[(size_t)row * gridDim.x + blockIdx.x] = si[0];
    }
}

__global__ __launch_bounds__(kThreads) void lazy_pick_kernel(const float* __restrict__ ws_s,
                                                             const int* __restrict__ ws_i, int nb,
                                                             int R, int* __restrict__ tokens,
                                                             int* __restrict__ pos_dev,
                                                             uint8_t* __restrict__ rep_update) {
    const int row = blockIdx.x;
    __shared__ float ss[kThreads];
    __shared__ int si[kThreads];
    float bs = -INFINITY;
    int bi = -1;
    for (int i = threadIdx.x; i < nb; i += kThreads) {
        const float s = ws_s[(size_t)row * nb + i];
        const int ix = ws_i[(size_t)row * nb + i];
        if (better(s, ix, bs, bi)) {
            bs = s;
            bi = ix;
        }
    }
    ss[threadIdx.x] = bs;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off && better(ss[threadIdx.x + off], si[threadIdx.x + off],
                                        ss[threadIdx.x], si[threadIdx.x])) {
            ss[threadIdx.x] = ss[threadIdx.x + off];
            si[threadIdx.x] = si[threadIdx.x + off];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        tokens[row] = si[0];
        if (pos_dev && row == 0) *pos_dev += 1;
        if (rep_update && si[0] >= 0) rep_update[(size_t)row * R + si[0]] = 1;
    }
}

int pick_blocks(uint32_t R) {
    return (int)std::max<uint32_t>(1, std::min<uint32_t>(kPickBlocks, (R + kThreads - 1) / kThreads));
}

uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

}  // namespace

namespace csdr {
size_t lazy_select_workspace(const csdr_lazy_hsdr* h, int rows) {
    return align_up((size_t)rows * h->K * 4, 256) + (size_t)rows * pick_blocks(h->R) * 8;
}
}  // namespace csdr

extern "C" {

CSDR_API int csdr_lazy_hsdr_load(const void* stream, size_t nbytes, int unpack, void* hip_stream,
                                 csdr_lazy_hsdr** out) {
    if (!stream || !out) return set_error(CSDR_E_INVALID, "lazy_hsdr_load: null argument");
    *out = nullptr;
    if (unpack != CSDR_LAZY_UNPACK_PACKED && unpack != CSDR_LAZY_UNPACK_CLI)
        return set_error(CSDR_E_INVALID, "lazy_hsdr_load: unknown code reading");
    const auto* b = static_cast<const uint8_t*>(stream);
    if (nbytes < 36) return set_error(CSDR_E_FORMAT, "lazy_hsdr_load: stream shorter than a header");
    if (std::memcmp(b, "HSDR", 4) != 0)
        return set_error(CSDR_E_FORMAT, "lazy_hsdr_load: not an HSDR stream");
    if (rd16(b + 20) != 1)
        return set_error(CSDR_E_FORMAT, "lazy_hsdr_load: only 1-row tiles are lazily decodable");
    csdr_lazy_hsdr h;
    h.R = rd32(b + 16);
    h.C = rd16(b + 22);
    h.K = rd16(b + 24);
    h.S = b[26];
    h.k = b[27];
    h.unpack = unpack;
    if (!h.R || !h.C || !h.S || !h.k)
        return set_error(CSDR_E_FORMAT, "lazy_hsdr_load: empty geometry");
    const size_t n_gamma = h.S, n_atoms = (size_t)h.K * h.C, n_codes = (size_t)h.R * h.S * h.k;
    const size_t off_atoms = 36 + 4 * n_gamma, off_codes = off_atoms + 4 * n_atoms;
    if (off_codes + 2 * n_codes > nbytes)
        return set_error(CSDR_E_FORMAT, "lazy_hsdr_load: stream truncated");
    auto* p = new (std::nothrow) csdr_lazy_hsdr(h);
    if (!p) return set_error(CSDR_E_INVALID, "lazy_hsdr_load: out of host memory");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    int rc = CSDR_OK;
    if (hipMalloc(&p->gamma, n_gamma * 4) != hipSuccess ||
        hipMalloc(&p->atoms, std::max<size_t>(n_atoms, 1) * 4) != hipSuccess ||
        hipMalloc(&p->packed, n_codes * 2) != hipSuccess ||
        hipMemcpyAsync(p->gamma, b + 36, n_gamma * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        (n_atoms && hipMemcpyAsync(p->atoms, b + off_atoms, n_atoms * 4, hipMemcpyHostToDevice,
                                   st) != hipSuccess) ||
        hipMemcpyAsync(p->packed, b + off_codes, n_codes * 2, hipMemcpyHostToDevice, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        rc = set_error(CSDR_E_HIP, "lazy_hsdr_load: device upload failed");
    if (rc) {
        csdr_lazy_hsdr_free(p);
        return rc;
    }
    *out = p;
    return CSDR_OK;
}

CSDR_API int csdr_lazy_hsdr_free(csdr_lazy_hsdr* h) {
    if (!h) return CSDR_OK;
    if (h->gamma) (void)hipFree(h->gamma);
    if (h->atoms) (void)hipFree(h->atoms);
    if (h->packed) (void)hipFree(h->packed);
    delete h;
    return CSDR_OK;
}

CSDR_API int csdr_lazy_hsdr_info(const csdr_lazy_hsdr* h, uint32_t* rows, uint32_t* cols) {
    if (!h) return set_error(CSDR_E_INVALID, "lazy_hsdr_info: null handle");
    if (rows) *rows = h->R;
    if (cols) *cols = h->C;
    return CSDR_OK;
}

CSDR_API int csdr_lazy_hsdr_decode_rows(const csdr_lazy_hsdr* h, const int* rows_dev, int row_host,
                                        int n, float* out, void* hip_stream) {
    if (!h || !out || n <= 0 || n > 65535)
        return set_error(CSDR_E_INVALID, "lazy_hsdr_decode_rows: bad argument");
    if (!rows_dev && (row_host < 0 || (uint32_t)row_host >= h->R))
        return set_error(CSDR_E_INVALID, "lazy_hsdr_decode_rows: row out of range");
    dim3 grid((h->C + kThreads - 1) / kThreads, n);
    lazy_row_kernel<<<grid, kThreads, 0, static_cast<hipStream_t>(hip_stream)>>>(*h, rows_dev,
                                                                              row_host, out);
    CSDR_LAUNCH_CHECK("lazy_hsdr_decode_rows");
    return CSDR_OK;
}

CSDR_API size_t csdr_lazy_hsdr_workspace_bytes(const csdr_lazy_hsdr* h, int rows) {
    return h && rows > 0 ? csdr::lazy_select_workspace(h, rows) : 0;
}

CSDR_API int csdr_lazy_hsdr_select(const csdr_lazy_hsdr* h, const float* hidden, int rows,
                                   const uint8_t* repeated, float temperature, float penalty,
                                   int* tokens, int* pos_dev, uint8_t* repeated_update,
                                   float* scores, void* workspace, size_t workspace_bytes,
                                   void* hip_stream) {
    if (!h || !hidden || !tokens || rows <= 0 || rows > 65535)
        return set_error(CSDR_E_INVALID, "lazy_hsdr_select: bad argument");
    const size_t need = csdr::lazy_select_workspace(h, rows);
    if (!workspace || workspace_bytes < need)
        return set_error(CSDR_E_WORKSPACE,
                         "lazy_hsdr_select: workspace needs " + std::to_string(need) + " bytes");
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    char* ws = static_cast<char*>(workspace);
    float* ah = reinterpret_cast<float*>(ws);
    const int nb = pick_blocks(h->R);
    float* ws_s = reinterpret_cast<float*>(ws + csdr::align_up((size_t)rows * h->K * 4, 256));
    int* ws_i = reinterpret_cast<int*>(ws_s + (size_t)rows * nb);
    const float ts = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    if (h->K) {
        lazy_ah_kernel<<<dim3((h->K + kThreads - 1) / kThreads, rows), kThreads, 0, st>>>(
            *h, hidden, ah);
        CSDR_LAUNCH_CHECK("lazy_hsdr ah");
    }
    lazy_score_kernel<<<dim3(nb, rows), kThreads, 0, st>>>(*h, ah, repeated, ts, penalty, scores,
                                                           ws_s, ws_i);
    CSDR_LAUNCH_CHECK("lazy_hsdr score");
    lazy_pick_kernel<<<rows, kThreads, 0, st>>>(ws_s, ws_i, nb, (int)h->R, tokens, pos_dev,
                                                repeated_update);
    CSDR_LAUNCH_CHECK("lazy_hsdr pick");
    return CSDR_OK;
}

}  // extern "C"
