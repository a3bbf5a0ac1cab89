// decoder.hip — a Llama/Qwen-style decoder over device-resident HSDB-coded weights.
//
// Reference: the SDK's native decoder run_transformer_decode (api/cortex_sdk.cpp:1543-1696),
// its token choice select_next_token_from_embedding_transpose (:1032-1206, with
// sanitize_hidden_for_sampling :959-976 and select_best_from_logits :1005-1030) and the
// generate_text loop (:1951-2054). Per block: RMSNorm -> q/k/v projections -> RoPE -> GQA
// attention -> o projection + residual -> RMSNorm -> gate/up -> SiLU*up -> down + residual;
// then the output RMSNorm, the lm_head scores of the sanitized hidden state and the
// penalised argmax. The reference recomputes the whole context for every token over dense
// fp32 weights; here the weights stay coded in HBM, K/V live in an fp16 cache, and one step
// is a fixed kernel sequence captured once in a HIP graph and replayed per token: the token,
// position and context length are device integers that each step reads and advances.
//
// Device token ring: ring[p] holds the token at position p (prompt tokens, then the tokens
// the steps select). A step at position p reads ring[p], appends K/V at p and, when it has the
// output head, selects the token for p + 1 and writes it to ring[p + 1]. Prompt positions
// before the last run the body-only step (no head; the reference's generate_text samples only
// after the whole prompt).
//
// Biases fold into the projections' output initialisation and the residual adds into the
// o/down projections (CSDR_HSDB_ACCUMULATE); the embedding is the lm_head row of the token
// (tied embeddings, decoded on the device) unless a separate coded embedding is set.
//
// Batch: B sequences advance in lockstep (one position for all; sequence b has its own token
// ring, K/V cache and generated-token set). Activations are token-major [b][feature], so
// every projection is one product of M = B columns (CSDR_HSDB_TOKEN_MAJOR; B <= 8 streams
// each code word once for all B columns) and the attention reads q/k/v rows as they are
// written. At B = 1 the attention's split combine is fused into the o projection's input.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"
#include "hsdb_impl.hpp"

namespace {

using csdr::set_error;

constexpr int kSanThreads = 256;
constexpr int kMaxBatch = 16;  // sequences per decoder (the fused x ops take up to 16 columns)

// Sequence b (thread b < B): its length and the token at the current position.
__global__ void step_begin_kernel(const int* __restrict__ pos, const int* __restrict__ ring,
                                  int cap, int B, int* __restrict__ tok, int* __restrict__ len) {
    const int b = threadIdx.x;
    if (b < B) {
        const int p = *pos;
        len[b] = p + 1;
        tok[b] = (p >= 0 && p < cap) ? ring[(size_t)b * cap + p] : -1;
    }
}

// fp16 K/V rows (each sequence's `per` values contiguous) into an fp32 cache whose sequences
// start `pitch` values apart.
__global__ void widen_kv_kernel(const uint16_t* __restrict__ src, size_t per, size_t pitch,
                                size_t count, float* __restrict__ dst) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t b = i / per, j = i - b * per;
        dst[b * pitch + j] = (float)__builtin_bit_cast(_Float16, src[i]);
    }
}

// Body-only step end: advance the position.
__global__ void advance_kernel(int* __restrict__ pos) {
    if (threadIdx.x == 0) *pos += 1;
}

// Head step end (after select_best advanced the position): sequence b's ring[pos] = its
// selected token.
__global__ void record_kernel(const int* __restrict__ tok, const int* __restrict__ pos,
                              int* __restrict__ ring, int cap, int B) {
    const int b = threadIdx.x;
    if (b < B) {
        const int p = *pos;
        if (p >= 0 && p < cap) ring[(size_t)b * cap + p] = tok[b];
    }
}

// sanitize_hidden_for_sampling (cortex_sdk.cpp:959-976) in place on row blockIdx.x of n
// floats: non-finite -> 0, then a uniform scale to max |h| = 1000 when the largest finite
// magnitude exceeds 1000.
__global__ __launch_bounds__(kSanThreads) void sanitize_kernel(float* __restrict__ h, int n) {
    h += (size_t)blockIdx.x * n;
    __shared__ float red[kSanThreads];
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += kSanThreads) {
        float v = h[i];
        if (!isfinite(v)) {
            v = 0.0f;
            h[i] = 0.0f;
        }
        m = fmaxf(m, fabsf(v));
    }
    red[threadIdx.x] = m;
    __syncthreads();
    for (int off = kSanThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + off]);
        __syncthreads();
    }
    const float mx = red[0];
    if (mx > 1000.0f) {
        const float scale = 1000.0f / mx;
        for (int i = threadIdx.x; i < n; i += kSanThreads) h[i] *= scale;
    }
}

constexpr int kBlockMats = 7;  // q, k, v, o, gate, up, down

struct Layer {
    const csdr_hsdb *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    const csdr_hsdb *gate = nullptr, *up = nullptr, *down = nullptr;
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    float *bq = nullptr, *bk = nullptr, *bv = nullptr;
    void *kc = nullptr, *vc = nullptr;  // cfg.kv_dtype elements
    // streamed block: the caller's host-resident segments, and device views of them whose
    // code words are the block's copy in staging buffer `slot` (at off[i])
    bool streamed = false;
    const csdr_hsdb* src[kBlockMats] = {};
    csdr_hsdb view[kBlockMats];
    size_t off[kBlockMats] = {};
    size_t bytes = 0;
    int slot = 0, rank = 0;  // staging buffer; position among the streamed blocks
};

}  // namespace

struct csdr_decoder {
    csdr_decoder_config cfg{};
    int B = 1;  // sequences decoded in lockstep
    std::vector<Layer> layers;
    const csdr_hsdb* lm = nullptr;
    const csdr_hsdb* emb = nullptr;
    float* final_norm = nullptr;
    float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *a = nullptr;
    float *g = nullptr, *u = nullptr, *logits = nullptr;
    int *tok = nullptr, *pos = nullptr, *len = nullptr, *ring = nullptr;
    uint8_t* repeated = nullptr;
    void* ws_hsdb = nullptr;
    size_t ws_hsdb_bytes = 0, ws_hsdb_alloc = 0;
    void* ws_attn = nullptr;
    size_t ws_attn_bytes = 0;
    void* ws_sel = nullptr;
    size_t ws_sel_bytes = 0;
    hipStream_t stream = nullptr;
    hipGraph_t graph[2] = {nullptr, nullptr};  // [0] body-only step, [1] step with head
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    float g_temp = 0.0f, g_pen = 0.0f;  // sampling parameters graph[1] was captured with
    int host_pos = 0;                   // positions processed (host mirror of *pos)
    bool use_graph = true;              // CSDR_DECODER_GRAPH=0: issue each step's kernels directly
    bool fused = true;                  // CSDR_DECODER_FUSED=0: one launch per op (reference order)
    int attn_splits = 1;
    int n_prompt = 0;
    std::vector<void*> allocs;
    // lazy HSDR token choice (the text CLI's), when set
    const csdr_lazy_hsdr* lazy = nullptr;
    float lazy_penalty = 1.0f;
    void* ws_lazy = nullptr;
    size_t ws_lazy_bytes = 0;
    // batched prefill: tokens per sequence per pass, and its buffers (rows = B x tokens)
    int prefill_chunk = 512;
    int pf_rows = 0;
    float *pf_x = nullptr, *pf_h = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
    float *pf_a = nullptr, *pf_g = nullptr, *pf_u = nullptr, *pf_w = nullptr;
    int* pf_tok = nullptr;
    // on-demand layer streaming (blocks of host-resident segments)
    bool prefetch = true;           // copy block j + 2 while block j + 1 runs (else j + 1 after j)
    bool stage_ready = false;       // staging buffers, views, copy stream and events built
    std::vector<int> streamed;      // the streamed blocks in order
    void* stage[2] = {nullptr, nullptr};
    size_t stage_bytes = 0;
    hipStream_t cstream = nullptr;  // the staging copies' stream (default priority)
    std::vector<hipEvent_t> ev_copied, ev_done;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace {

template <typename T>
int dalloc(csdr_decoder* d, T** p, size_t count) {
    void* ptr = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 4);
    CSDR_HIP_CHECK(hipMalloc(&ptr, bytes));
    d->allocs.push_back(ptr);
    CSDR_HIP_CHECK(hipMemset(ptr, 0, bytes));
    // the null stream's fill does not order the decoder's non-blocking stream
    CSDR_HIP_CHECK(hipDeviceSynchronize());
    *p = static_cast<T*>(ptr);
    return CSDR_OK;
}

int upload_vec(csdr_decoder* d, float** dst, const float* host, size_t n) {
    if (!host) {
        *dst = nullptr;
        return CSDR_OK;
    }
    if (!*dst) {
        int rc = dalloc(d, dst, n);
        if (rc) return rc;
    }
    CSDR_HIP_CHECK(hipMemcpy(*dst, host, n * 4, hipMemcpyHostToDevice));
    return CSDR_OK;
}

int check_shape(const csdr_hsdb* s, uint32_t R, uint32_t C, const char* what) {
    csdr_hsdb_info info;
    if (!s || csdr_hsdb_get_info(s, &info) != CSDR_OK)
        return set_error(CSDR_E_INVALID, std::string("decoder: missing ") + what);
    if (info.rows != R || info.cols != C || info.tile_rows != 1)
        return set_error(CSDR_E_INVALID, std::string("decoder: ") + what + " is " +
                                             std::to_string(info.rows) + "x" +
                                             std::to_string(info.cols) + ", expected " +
                                             std::to_string(R) + "x" + std::to_string(C));
    return CSDR_OK;
}

#define RC(expr)                        \
    do {                                \
        int rc_ = (expr);               \
        if (rc_ != CSDR_OK) return rc_; \
    } while (0)

int mm(csdr_decoder* d, int n, const csdr_hsdb* const* segs, const float* x, float* const* ys,
       const float* const* bias, int flags, hipStream_t st) {
    const void* xs[4];
    for (int i = 0; i < n; ++i) xs[i] = x;
    return csdr_hsdb_matmul_group_ex(n, segs, xs, CSDR_F32, d->B, ys, bias,
                                     flags | CSDR_HSDB_TOKEN_MAJOR, d->ws_hsdb, d->ws_hsdb_bytes,
                                     st);
}

int mm_xop(csdr_decoder* d, int n, const csdr_hsdb* const* segs, const float* x, const float* x2,
           float* const* ys, const float* const* bias, int flags, int xop, const float* nw,
           hipStream_t st) {
    const void* xs[4];
    const void* x2s[4];
    for (int i = 0; i < n; ++i) {
        xs[i] = x;
        x2s[i] = x2;
    }
    const csdr_decoder_config& c = d->cfg;
    return csdr_hsdb_matmul_group_xop(n, segs, xs, x2s, d->B, ys, bias,
                                      flags | CSDR_HSDB_TOKEN_MAJOR, xop, nw, c.rms_eps,
                                      d->attn_splits, c.head_dim, d->ws_hsdb, d->ws_hsdb_bytes,
                                      st);
}

// ---- on-demand layer streaming
// A streamed block's code words are copied (on d->cstream) into staging buffer slot
// rank % 2 before the block runs; the copy of the block `depth` places later (2 with
// prefetch, else 1) waits for this block's kernels to finish, the last reader of that
// buffer. Events order the two streams, so the same sequence works issued directly or
// captured into the step graph (the copies become graph nodes).

void free_streaming(csdr_decoder* d) {
    if (d->cstream) {
        (void)hipStreamSynchronize(d->cstream);
        (void)hipStreamDestroy(d->cstream);
    }
    for (hipEvent_t e : d->ev_copied) if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : d->ev_done) if (e) (void)hipEventDestroy(e);
    if (d->ev_fork) (void)hipEventDestroy(d->ev_fork);
    if (d->ev_join) (void)hipEventDestroy(d->ev_join);
    for (void*& p : d->stage) {
        if (p) (void)hipFree(p);
        p = nullptr;
    }
    d->cstream = nullptr;
    d->ev_copied.clear();
    d->ev_done.clear();
    d->ev_fork = d->ev_join = nullptr;
    d->stage_bytes = 0;
    d->stage_ready = false;
}

// Staging buffers sized for the largest streamed block, the blocks' device views, the copy
// stream and the events.
int setup_streaming(csdr_decoder* d) {
    free_streaming(d);
    d->streamed.clear();
    size_t most = 0;
    for (int l = 0; l < (int)d->layers.size(); ++l) {
        Layer& L = d->layers[l];
        if (!L.streamed) continue;
        L.rank = (int)d->streamed.size();
        L.slot = L.rank % 2;
        d->streamed.push_back(l);
        size_t off = 0;
        for (int i = 0; i < kBlockMats; ++i) {
            L.off[i] = off;
            off += csdr::align_up(csdr::code_bytes(L.src[i]), 256);
        }
        L.bytes = off;
        most = std::max(most, off);
    }
    if (d->streamed.empty()) {
        d->stage_ready = true;
        return CSDR_OK;
    }
    for (void*& p : d->stage)
        if (hipMalloc(&p, std::max<size_t>(most, 256)) != hipSuccess) {
            free_streaming(d);
            return set_error(CSDR_E_HIP, "decoder: out of device memory for the layer staging "
                                         "buffers (2 x " + std::to_string(most) + " bytes)");
        }
    d->stage_bytes = most;
    for (int l : d->streamed) {
        Layer& L = d->layers[l];
        for (int i = 0; i < kBlockMats; ++i) {
            L.view[i] = *L.src[i];
            L.view[i].h_codes = nullptr;
            L.view[i].dict_ref = nullptr;  // a view: never released
            L.view[i].d_codes =
                reinterpret_cast<uint32_t*>(static_cast<char*>(d->stage[L.slot]) + L.off[i]);
        }
    }
    if (hipStreamCreateWithFlags(&d->cstream, hipStreamNonBlocking) != hipSuccess) {
        free_streaming(d);
        return set_error(CSDR_E_HIP, "decoder: copy stream creation failed");
    }
    const size_t nl = d->layers.size();
    d->ev_copied.assign(nl, nullptr);
    d->ev_done.assign(nl, nullptr);
    bool okv = hipEventCreateWithFlags(&d->ev_fork, hipEventDisableTiming) == hipSuccess &&
               hipEventCreateWithFlags(&d->ev_join, hipEventDisableTiming) == hipSuccess;
    for (int l : d->streamed)
        okv = okv &&
              hipEventCreateWithFlags(&d->ev_copied[l], hipEventDisableTiming) == hipSuccess &&
              hipEventCreateWithFlags(&d->ev_done[l], hipEventDisableTiming) == hipSuccess;
    if (!okv) {
        free_streaming(d);
        return set_error(CSDR_E_HIP, "decoder: event creation failed");
    }
    d->stage_ready = true;
    return CSDR_OK;
}

// Block l's code words into its staging buffer, on the copy stream.
int stage_copy(csdr_decoder* d, int l) {
    const Layer& L = d->layers[l];
    char* dst = static_cast<char*>(d->stage[L.slot]);
    for (int i = 0; i < kBlockMats; ++i) {
        const size_t n = csdr::code_bytes(L.src[i]);
        if (n)
            CSDR_HIP_CHECK(hipMemcpyAsync(dst + L.off[i], L.src[i]->h_codes, n,
                                          hipMemcpyHostToDevice, d->cstream));
    }
    CSDR_HIP_CHECK(hipEventRecord(d->ev_copied[l], d->cstream));
    return CSDR_OK;
}

int stream_depth(const csdr_decoder* d) { return d->prefetch ? 2 : 1; }

// Before the first block of a step or pass: the copy stream joins st's work, and the first
// blocks' copies start.
int stream_begin(csdr_decoder* d, hipStream_t st) {
    if (d->streamed.empty()) return CSDR_OK;
    CSDR_HIP_CHECK(hipEventRecord(d->ev_fork, st));
    CSDR_HIP_CHECK(hipStreamWaitEvent(d->cstream, d->ev_fork, 0));
    const int n = std::min<int>(stream_depth(d), (int)d->streamed.size());
    for (int j = 0; j < n; ++j) RC(stage_copy(d, d->streamed[j]));
    return CSDR_OK;
}

// Block l runs after its copy.
int layer_begin(csdr_decoder* d, int l, hipStream_t st) {
    if (!d->layers[l].streamed) return CSDR_OK;
    CSDR_HIP_CHECK(hipStreamWaitEvent(st, d->ev_copied[l], 0));
    return CSDR_OK;
}

// After block l: the copy into its buffer of the block `depth` streamed places later.
int layer_end(csdr_decoder* d, int l, hipStream_t st) {
    const Layer& L = d->layers[l];
    if (!L.streamed) return CSDR_OK;
    CSDR_HIP_CHECK(hipEventRecord(d->ev_done[l], st));
    const int j = L.rank + stream_depth(d);
    if (j < (int)d->streamed.size()) {
        CSDR_HIP_CHECK(hipStreamWaitEvent(d->cstream, d->ev_done[l], 0));
        RC(stage_copy(d, d->streamed[j]));
    }
    return CSDR_OK;
}

// After the last block: st waits for the copy stream's work (joins a captured fork).
int stream_end(csdr_decoder* d, hipStream_t st) {
    if (d->streamed.empty()) return CSDR_OK;
    CSDR_HIP_CHECK(hipEventRecord(d->ev_join, d->cstream));
    CSDR_HIP_CHECK(hipStreamWaitEvent(st, d->ev_join, 0));
    return CSDR_OK;
}

// Prefill pass rows: row b * T + t takes sequence b's token at position p0 + t.
__global__ void pass_tokens_kernel(const int* __restrict__ ring, int cap, int B, int T, int p0,
                                   int* __restrict__ tok) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B * T) tok[i] = ring[(size_t)(i / T) * cap + p0 + i % T];
}

void free_prefill(csdr_decoder* d) {
    for (float* p : {d->pf_x, d->pf_h, d->pf_q, d->pf_k, d->pf_v, d->pf_a, d->pf_g, d->pf_u,
                     d->pf_w})
        if (p) (void)hipFree(p);
    if (d->pf_tok) (void)hipFree(d->pf_tok);
    d->pf_x = d->pf_h = d->pf_q = d->pf_k = d->pf_v = d->pf_a = d->pf_g = d->pf_u = d->pf_w =
        nullptr;
    d->pf_tok = nullptr;
    d->pf_rows = 0;
}

// Buffers of a prefill pass over `rows` token rows (kept for later passes of up to as many).
int ensure_prefill(csdr_decoder* d, int rows) {
    if (rows <= d->pf_rows) return CSDR_OK;
    free_prefill(d);
    const csdr_decoder_config& c = d->cfg;
    const size_t n = (size_t)rows, H = c.hidden, F = c.ffn;
    const size_t kvw = (size_t)c.n_kv_heads * c.head_dim;
    const size_t wmax = std::max({H * H, kvw * H, F * H});
    const std::pair<float**, size_t> bufs[] = {
        {&d->pf_x, n * H},   {&d->pf_h, n * H},   {&d->pf_q, n * H},
        {&d->pf_k, n * kvw}, {&d->pf_v, n * kvw}, {&d->pf_a, n * std::max(H, F)},
        {&d->pf_g, n * F},   {&d->pf_u, n * F},   {&d->pf_w, wmax}};
    for (const auto& b : bufs) {
        void* p = nullptr;
        if (hipMalloc(&p, b.second * 4) != hipSuccess) {
            free_prefill(d);
            return set_error(CSDR_E_HIP, "decoder_prefill: out of device memory for " +
                                             std::to_string(rows) + " prefill rows");
        }
        *b.first = static_cast<float*>(p);
    }
    void* p = nullptr;
    if (hipMalloc(&p, n * 4) != hipSuccess) {
        free_prefill(d);
        return set_error(CSDR_E_HIP, "decoder_prefill: out of device memory");
    }
    d->pf_tok = static_cast<int*>(p);
    d->pf_rows = rows;
    return CSDR_OK;
}

// y (M x R) (+)= x (M x C) . W^T + bias for a coded W: decoded to dense fp32 once, then the
// matrix-core product over all M rows.
int pass_linear(csdr_decoder* d, const csdr_hsdb* w, const float* x, int M, float* y,
                const float* bias, int flags, hipStream_t st) {
    csdr_hsdb_info info;
    RC(csdr_hsdb_get_info(w, &info));
    RC(csdr_hsdb_decompress(w, d->pf_w, st));
    return csdr_dense_linear_ex(d->pf_w, (int)info.rows, (int)info.cols, x, M, y, bias, flags, st);
}

// The decoder body (no head) over positions [p0, p0 + T) of every sequence as one pass of
// M = B x T token rows: K/V of those positions land in the caches as the decode step would
// write them.
int prefill_pass(csdr_decoder* d, int p0, int T, hipStream_t st) {
    const csdr_decoder_config& c = d->cfg;
    const int B = d->B, M = B * T, H = c.hidden, F = c.ffn;
    const int cap = c.max_ctx + 1;
    pass_tokens_kernel<<<(M + 255) / 256, 256, 0, st>>>(d->ring, cap, B, T, p0, d->pf_tok);
    CSDR_LAUNCH_CHECK("decoder pass tokens");
    RC(csdr_hsdb_decode_rows(d->emb, d->pf_tok, M, d->pf_x, st));
    RC(stream_begin(d, st));
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer& L = d->layers[l];
        RC(layer_begin(d, l, st));
        RC(csdr_rms_norm(d->pf_x, L.attn_norm, M, H, c.rms_eps, d->pf_h, st));
        RC(pass_linear(d, L.q, d->pf_h, M, d->pf_q, L.bq, 0, st));
        RC(pass_linear(d, L.k, d->pf_h, M, d->pf_k, L.bk, 0, st));
        RC(pass_linear(d, L.v, d->pf_h, M, d->pf_v, L.bv, 0, st));
        RC(csdr_rope_kv_rows(d->pf_q, d->pf_k, d->pf_v, B, T, p0, c.n_heads, c.n_kv_heads,
                             c.head_dim, c.rope_theta, L.kc, L.vc, c.kv_dtype, c.max_ctx, st));
        RC(csdr_attn_prefill(d->pf_q, L.kc, L.vc, c.kv_dtype, B, T, p0, c.max_ctx, c.n_heads,
                             c.n_kv_heads, c.head_dim, 0.0f, d->pf_a, st));
        RC(pass_linear(d, L.o, d->pf_a, M, d->pf_x, nullptr, CSDR_HSDB_ACCUMULATE, st));
        RC(csdr_rms_norm(d->pf_x, L.ffn_norm, M, H, c.rms_eps, d->pf_h, st));
        RC(pass_linear(d, L.gate, d->pf_h, M, d->pf_g, nullptr, 0, st));
        RC(pass_linear(d, L.up, d->pf_h, M, d->pf_u, nullptr, 0, st));
        RC(csdr_silu_mul(d->pf_g, d->pf_u, (size_t)M * F, d->pf_a, st));
        RC(pass_linear(d, L.down, d->pf_a, M, d->pf_x, nullptr, CSDR_HSDB_ACCUMULATE, st));
        RC(layer_end(d, l, st));
    }
    return stream_end(d, st);
}

// One step at device position *pos for the token ring[*pos]; with_head adds the output norm,
// the lm_head scores and the token selection.
int step(csdr_decoder* d, hipStream_t st, bool with_head, float temperature, float penalty) {
    const csdr_decoder_config& c = d->cfg;
    const int H = c.hidden, Hq = c.n_heads, Hkv = c.n_kv_heads, hd = c.head_dim;
    const int cap = c.max_ctx + 1, B = d->B;
    step_begin_kernel<<<1, 64, 0, st>>>(d->pos, d->ring, cap, B, d->tok, d->len);
    CSDR_LAUNCH_CHECK("decoder step_begin");
    RC(csdr_hsdb_decode_rows(d->emb, d->tok, B, d->x, st));
    if (!d->fused && (B > 1 || c.kv_dtype != CSDR_F16))
        return set_error(CSDR_E_UNSUPPORTED,
                         "decoder: the unfused step runs batch 1 over an fp16 K/V cache only");
    RC(stream_begin(d, st));
    for (int l = 0; l < c.n_layers && d->fused; ++l) {
        // fused form: 5 calls (9 launches) per block; the normed inputs, the rotated q/k, the
        // attention output and silu(gate)*up are never written out
        const Layer& L = d->layers[l];
        RC(layer_begin(d, l, st));
        {
            const csdr_hsdb* segs[3] = {L.q, L.k, L.v};
            float* ys[3] = {d->q, d->k, d->v};
            const float* bias[3] = {L.bq, L.bk, L.bv};
            RC(mm_xop(d, 3, segs, d->x, nullptr, ys, bias, 0, CSDR_XOP_RMSNORM, L.attn_norm, st));
        }
        // B == 1: the split partials stay in the workspace and the o projection combines
        // them while staging its input; B > 1: combined into a (B x H) first
        RC(csdr_attn_decode_rope_kv(d->q, d->k, d->v, L.kc, L.vc, c.kv_dtype, d->len, B,
                                    c.max_ctx, Hq, Hkv, hd, c.rope_theta, 0.0f,
                                    B > 1 ? d->a : nullptr, d->ws_attn, d->ws_attn_bytes, st));
        {
            const csdr_hsdb* segs[1] = {L.o};
            float* ys[1] = {d->x};  // x += o(attention)
            if (B == 1)
                RC(mm_xop(d, 1, segs, static_cast<const float*>(d->ws_attn), nullptr, ys, nullptr,
                          CSDR_HSDB_ACCUMULATE, CSDR_XOP_ATTN, nullptr, st));
            else
                RC(mm(d, 1, segs, d->a, ys, nullptr, CSDR_HSDB_ACCUMULATE, st));
        }
        {
            const csdr_hsdb* segs[2] = {L.gate, L.up};
            float* ys[2] = {d->g, d->u};
            RC(mm_xop(d, 2, segs, d->x, nullptr, ys, nullptr, 0, CSDR_XOP_RMSNORM, L.ffn_norm, st));
        }
        {
            const csdr_hsdb* segs[1] = {L.down};
            float* ys[1] = {d->x};  // x += down(silu(gate) * up)
            RC(mm_xop(d, 1, segs, d->g, d->u, ys, nullptr, CSDR_HSDB_ACCUMULATE,
                      CSDR_XOP_SILU_MUL, nullptr, st));
        }
        RC(layer_end(d, l, st));
    }
    for (int l = 0; l < c.n_layers && !d->fused; ++l) {
        const Layer& L = d->layers[l];
        RC(layer_begin(d, l, st));
        RC(csdr_rms_norm(d->x, L.attn_norm, 1, H, c.rms_eps, d->h, st));
        {
            const csdr_hsdb* segs[3] = {L.q, L.k, L.v};
            float* ys[3] = {d->q, d->k, d->v};
            const float* bias[3] = {L.bq, L.bk, L.bv};
            RC(mm(d, 3, segs, d->h, ys, bias, 0, st));
        }
        RC(csdr_rope_kv(d->q, d->k, d->v, 1, Hq, Hkv, hd, d->pos, c.rope_theta,
                        static_cast<uint16_t*>(L.kc), static_cast<uint16_t*>(L.vc),
                        c.max_ctx, st));
        RC(csdr_attn_decode(d->q, static_cast<const uint16_t*>(L.kc),
                            static_cast<const uint16_t*>(L.vc), d->len, 0, 1, c.max_ctx, Hq, Hkv,
                            hd, 0.0f, d->a,
                            d->ws_attn, d->ws_attn_bytes, st));
        {
            const csdr_hsdb* segs[1] = {L.o};
            float* ys[1] = {d->x};
            RC(mm(d, 1, segs, d->a, ys, nullptr, CSDR_HSDB_ACCUMULATE, st));  // x += o(a)
        }
        RC(csdr_rms_norm(d->x, L.ffn_norm, 1, H, c.rms_eps, d->h, st));
        {
            const csdr_hsdb* segs[2] = {L.gate, L.up};
            float* ys[2] = {d->g, d->u};
            RC(mm(d, 2, segs, d->h, ys, nullptr, 0, st));
        }
        RC(csdr_silu_mul(d->g, d->u, (size_t)c.ffn, d->a, st));
        {
            const csdr_hsdb* segs[1] = {L.down};
            float* ys[1] = {d->x};
            RC(mm(d, 1, segs, d->a, ys, nullptr, CSDR_HSDB_ACCUMULATE, st));  // x += down(a)
        }
        RC(layer_end(d, l, st));
    }
    RC(stream_end(d, st));
    if (!with_head) {
        advance_kernel<<<1, 64, 0, st>>>(d->pos);
        CSDR_LAUNCH_CHECK("decoder advance");
        return CSDR_OK;
    }
    if (d->final_norm) RC(csdr_rms_norm(d->x, d->final_norm, B, H, c.rms_eps, d->h, st));
    else CSDR_HIP_CHECK(hipMemcpyAsync(d->h, d->x, (size_t)B * H * 4, hipMemcpyDeviceToDevice, st));
    if (d->lazy) {
        // the CLI's lazy HSDR scoring of the normed hidden state
        RC(csdr_lazy_hsdr_select(d->lazy, d->h, B, d->repeated, temperature, d->lazy_penalty,
                                 d->tok, d->pos, d->repeated, d->logits, d->ws_lazy,
                                 d->ws_lazy_bytes, st));
        record_kernel<<<1, 64, 0, st>>>(d->tok, d->pos, d->ring, cap, B);
        CSDR_LAUNCH_CHECK("decoder record");
        return CSDR_OK;
    }
    sanitize_kernel<<<B, kSanThreads, 0, st>>>(d->h, H);
    CSDR_LAUNCH_CHECK("decoder sanitize");
    {
        const csdr_hsdb* segs[1] = {d->lm};
        float* ys[1] = {d->logits};
        RC(mm(d, 1, segs, d->h, ys, nullptr, 0, st));
    }
    RC(csdr::select_best_rows(d->logits, c.vocab, B, d->repeated, temperature, penalty, d->tok,
                              d->pos, d->repeated, d->ws_sel, d->ws_sel_bytes, st));
    record_kernel<<<1, 64, 0, st>>>(d->tok, d->pos, d->ring, cap, B);
    CSDR_LAUNCH_CHECK("decoder record");
    return CSDR_OK;
}

void destroy_graphs(csdr_decoder* d) {
    for (int i = 0; i < 2; ++i) {
        if (d->exec[i]) (void)hipGraphExecDestroy(d->exec[i]);
        if (d->graph[i]) (void)hipGraphDestroy(d->graph[i]);
        d->exec[i] = nullptr;
        d->graph[i] = nullptr;
    }
}

int ready(csdr_decoder* d) {
    if (!d) return set_error(CSDR_E_INVALID, "decoder: null handle");
    for (size_t l = 0; l < d->layers.size(); ++l)
        if (!d->layers[l].q)
            return set_error(CSDR_E_INVALID, "decoder: layer " + std::to_string(l) + " not set");
    if (!d->lm || !d->emb) return set_error(CSDR_E_INVALID, "decoder: output head not set");
    if (!d->stage_ready) {
        destroy_graphs(d);
        RC(setup_streaming(d));
    }
    if (d->ws_hsdb_alloc < d->ws_hsdb_bytes) {
        unsigned char* p = nullptr;
        RC(dalloc(d, &p, d->ws_hsdb_bytes));
        d->ws_hsdb = p;
        d->ws_hsdb_alloc = d->ws_hsdb_bytes;
        destroy_graphs(d);
    }
    return CSDR_OK;
}

// Captures graph[i] (i = with_head) if it is missing or was captured with other parameters.
int ensure_graph(csdr_decoder* d, int i, float temperature, float penalty) {
    if (d->exec[i] && (i == 0 || (d->g_temp == temperature && d->g_pen == penalty)))
        return CSDR_OK;
    if (d->exec[i]) (void)hipGraphExecDestroy(d->exec[i]);
    if (d->graph[i]) (void)hipGraphDestroy(d->graph[i]);
    d->exec[i] = nullptr;
    d->graph[i] = nullptr;
    CSDR_HIP_CHECK(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    const int rc = step(d, d->stream, i == 1, temperature, penalty);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(d->stream, &g);
    if (rc != CSDR_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess || !g)
        return set_error(CSDR_E_HIP, std::string("decoder: graph capture failed: ") +
                                         hipGetErrorString(e));
    d->graph[i] = g;
    CSDR_HIP_CHECK(hipGraphInstantiate(&d->exec[i], g, nullptr, nullptr, 0));
    if (i == 1) {
        d->g_temp = temperature;
        d->g_pen = penalty;
    }
    return CSDR_OK;
}

// One step: a replay of the captured graph, or the kernels issued directly on the stream.
int run_step(csdr_decoder* d, int i, float temperature, float penalty) {
    if (!d->use_graph) return step(d, d->stream, i == 1, temperature, penalty);
    CSDR_HIP_CHECK(hipGraphLaunch(d->exec[i], d->stream));
    return CSDR_OK;
}

}  // namespace

extern "C" {

CSDR_API int csdr_decoder_create(const csdr_decoder_config* cfg, csdr_decoder** out) {
    return csdr_decoder_create_batched(cfg, 1, out);
}

CSDR_API int csdr_decoder_create_batched(const csdr_decoder_config* cfg, int batch,
                                         csdr_decoder** out) {
    if (!cfg || !out) return set_error(CSDR_E_INVALID, "decoder_create: null argument");
    *out = nullptr;
    if (batch < 1 || batch > kMaxBatch)
        return set_error(CSDR_E_INVALID, "decoder_create: batch must be 1.." +
                                             std::to_string(kMaxBatch));
    const csdr_decoder_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
        c.n_heads % c.n_kv_heads || c.head_dim * c.n_heads != c.hidden || c.ffn <= 0 ||
        c.vocab <= 0 || c.max_ctx <= 0 || (c.head_dim != 64 && c.head_dim != 128) ||
        (c.kv_dtype != CSDR_F32 && c.kv_dtype != CSDR_F16) ||
        !(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0f))
        return set_error(CSDR_E_INVALID, "decoder_create: inconsistent config");
    csdr_decoder* d = new (std::nothrow) csdr_decoder();
    if (!d) return set_error(CSDR_E_INVALID, "decoder_create: out of host memory");
    d->cfg = c;
    d->B = batch;
    const int B = batch;
    d->layers.resize(c.n_layers);
    if (const char* e = getenv("CSDR_DECODER_GRAPH")) d->use_graph = atoi(e) != 0;
    if (const char* e = getenv("CSDR_DECODER_FUSED")) d->fused = atoi(e) != 0;
    d->attn_splits = csdr_attn_decode_splits_kv(B, c.n_heads, c.n_kv_heads, c.head_dim, c.max_ctx,
                                                c.kv_dtype);
    int rc = CSDR_OK;
    // per layer: sequence b's cache at b * max_ctx positions, fp32 or fp16 elements
    const size_t kvn = (size_t)B * c.max_ctx * c.n_kv_heads * c.head_dim *
                       (c.kv_dtype == CSDR_F32 ? 2 : 1);
    for (auto& L : d->layers) {
        uint16_t *kc = nullptr, *vc = nullptr;
        if ((rc = dalloc(d, &kc, kvn)) || (rc = dalloc(d, &vc, kvn))) break;
        L.kc = kc;
        L.vc = vc;
    }
    const size_t kvw = (size_t)c.n_kv_heads * c.head_dim;
    const size_t wide = std::max(c.hidden, c.ffn);
    if (!rc) rc = dalloc(d, &d->x, (size_t)B * c.hidden);
    if (!rc) rc = dalloc(d, &d->h, (size_t)B * c.hidden);
    if (!rc) rc = dalloc(d, &d->q, (size_t)B * c.hidden);
    if (!rc) rc = dalloc(d, &d->k, B * kvw);
    if (!rc) rc = dalloc(d, &d->v, B * kvw);
    if (!rc) rc = dalloc(d, &d->a, B * wide);
    if (!rc) rc = dalloc(d, &d->g, (size_t)B * c.ffn);
    if (!rc) rc = dalloc(d, &d->u, (size_t)B * c.ffn);
    if (!rc) rc = dalloc(d, &d->logits, (size_t)B * c.vocab);
    if (!rc) rc = dalloc(d, &d->tok, (size_t)B);
    if (!rc) rc = dalloc(d, &d->pos, 1);
    if (!rc) rc = dalloc(d, &d->len, (size_t)B);
    if (!rc) rc = dalloc(d, &d->ring, (size_t)B * (c.max_ctx + 1));
    if (!rc) rc = dalloc(d, &d->repeated, (size_t)B * c.vocab);
    if (!rc) {
        d->ws_attn_bytes = csdr_attn_decode_workspace_bytes(B, c.n_heads, c.head_dim, c.max_ctx);
        unsigned char* p = nullptr;
        rc = dalloc(d, &p, d->ws_attn_bytes);
        d->ws_attn = p;
    }
    if (!rc) {
        d->ws_sel_bytes = csdr::select_workspace_rows(B);
        unsigned char* p = nullptr;
        rc = dalloc(d, &p, d->ws_sel_bytes);
        d->ws_sel = p;
    }
    if (!rc && hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess)
        rc = set_error(CSDR_E_HIP, "decoder_create: stream creation failed");
    if (rc) {
        csdr_decoder_free(d);
        return rc;
    }
    *out = d;
    return CSDR_OK;
}

CSDR_API int csdr_decoder_free(csdr_decoder* d) {
    if (!d) return CSDR_OK;
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    destroy_graphs(d);
    free_streaming(d);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    free_prefill(d);
    for (void* p : d->allocs) (void)hipFree(p);
    delete d;
    return CSDR_OK;
}

CSDR_API int csdr_decoder_set_layer(csdr_decoder* d, int layer, const csdr_hsdb* wq,
                                    const csdr_hsdb* wk, const csdr_hsdb* wv, const csdr_hsdb* wo,
                                    const csdr_hsdb* wgate, const csdr_hsdb* wup,
                                    const csdr_hsdb* wdown, const float* attn_norm,
                                    const float* ffn_norm, const float* bq, const float* bk,
                                    const float* bv) {
    if (!d || layer < 0 || layer >= d->cfg.n_layers || !attn_norm || !ffn_norm)
        return set_error(CSDR_E_INVALID, "decoder_set_layer: bad argument");
    const csdr_decoder_config& c = d->cfg;
    const uint32_t H = c.hidden, kvw = c.n_kv_heads * c.head_dim, F = c.ffn;
    RC(check_shape(wq, H, H, "q"));
    RC(check_shape(wk, kvw, H, "k"));
    RC(check_shape(wv, kvw, H, "v"));
    RC(check_shape(wo, H, H, "o"));
    RC(check_shape(wgate, F, H, "gate"));
    RC(check_shape(wup, F, H, "up"));
    RC(check_shape(wdown, H, F, "down"));
    const csdr_hsdb* w7[kBlockMats] = {wq, wk, wv, wo, wgate, wup, wdown};
    int on_host = 0;
    for (const csdr_hsdb* w : w7) on_host += csdr::codes_on_device(w) ? 0 : 1;
    if (on_host != 0 && on_host != kBlockMats)
        return set_error(CSDR_E_INVALID, "decoder_set_layer: a block's segments must be all "
                                         "device-resident or all host-resident");
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    destroy_graphs(d);
    if (d->cstream) CSDR_HIP_CHECK(hipStreamSynchronize(d->cstream));
    d->stage_ready = false;  // the staging layout is rebuilt before the next run
    Layer& L = d->layers[layer];
    L.streamed = on_host == kBlockMats;
    if (L.streamed) {
        for (int i = 0; i < kBlockMats; ++i) L.src[i] = w7[i];
        L.q = &L.view[0], L.k = &L.view[1], L.v = &L.view[2], L.o = &L.view[3];
        L.gate = &L.view[4], L.up = &L.view[5], L.down = &L.view[6];
    } else {
        L.q = wq, L.k = wk, L.v = wv, L.o = wo, L.gate = wgate, L.up = wup, L.down = wdown;
    }
    RC(upload_vec(d, &L.attn_norm, attn_norm, H));
    RC(upload_vec(d, &L.ffn_norm, ffn_norm, H));
    RC(upload_vec(d, &L.bq, bq, H));
    RC(upload_vec(d, &L.bk, bk, kvw));
    RC(upload_vec(d, &L.bv, bv, kvw));
    const csdr_hsdb* qkv[3] = {wq, wk, wv};
    const csdr_hsdb* gu[2] = {wgate, wup};
    const int B = d->B;
    d->ws_hsdb_bytes = std::max({d->ws_hsdb_bytes, csdr_hsdb_group_workspace_bytes(3, qkv, B),
                                 csdr_hsdb_group_workspace_bytes(1, &wo, B),
                                 csdr_hsdb_group_workspace_bytes(2, gu, B),
                                 csdr_hsdb_group_workspace_bytes(1, &wdown, B)});
    return CSDR_OK;
}

CSDR_API int csdr_decoder_set_layer_prefetch(csdr_decoder* d, int enable) {
    if (!d) return set_error(CSDR_E_INVALID, "decoder_set_layer_prefetch: null handle");
    if (d->prefetch == (enable != 0)) return CSDR_OK;
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    destroy_graphs(d);  // the captured copy dependencies change
    d->prefetch = enable != 0;
    return CSDR_OK;
}

CSDR_API int64_t csdr_decoder_streamed_bytes(const csdr_decoder* d) {
    if (!d) return -1;
    int64_t n = 0;
    for (const Layer& L : d->layers)
        if (L.streamed)
            for (const csdr_hsdb* w : L.src) n += (int64_t)csdr::code_bytes(w);
    return n;
}

CSDR_API int csdr_decoder_set_output(csdr_decoder* d, const csdr_hsdb* lm_head,
                                     const float* final_norm, const csdr_hsdb* embedding) {
    if (!d) return set_error(CSDR_E_INVALID, "decoder_set_output: null handle");
    const csdr_decoder_config& c = d->cfg;
    RC(check_shape(lm_head, c.vocab, c.hidden, "lm_head"));
    if (embedding) RC(check_shape(embedding, c.vocab, c.hidden, "embedding"));
    if (!csdr::codes_on_device(lm_head) || (embedding && !csdr::codes_on_device(embedding)))
        return set_error(CSDR_E_INVALID, "decoder_set_output: the output head and embedding "
                                         "must be device-resident segments");
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    destroy_graphs(d);
    d->lm = lm_head;
    d->emb = embedding ? embedding : lm_head;
    RC(upload_vec(d, &d->final_norm, final_norm, c.hidden));
    d->ws_hsdb_bytes =
        std::max(d->ws_hsdb_bytes, csdr_hsdb_group_workspace_bytes(1, &lm_head, d->B));
    return CSDR_OK;
}

CSDR_API int csdr_decoder_prefill(csdr_decoder* d, const int32_t* prompt, int n_prompt,
                                  float temperature, float penalty) {
    RC(ready(d));
    const csdr_decoder_config& c = d->cfg;
    if (!prompt || n_prompt <= 0)
        return set_error(CSDR_E_INVALID, "decoder_prefill: empty prompt");
    if (n_prompt > c.max_ctx)
        return set_error(CSDR_E_INVALID, "decoder_prefill: prompt longer than the context");
    const int B = d->B;
    for (long long i = 0; i < (long long)B * n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= c.vocab)
            return set_error(CSDR_E_INVALID, "decoder_prefill: token id out of range");
    if (d->use_graph) {
        RC(ensure_graph(d, 0, temperature, penalty));
        RC(ensure_graph(d, 1, temperature, penalty));
    }
    hipStream_t st = d->stream;
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    const size_t cap = (size_t)c.max_ctx + 1;
    // resets on the decoder's stream (ordered before its steps)
    CSDR_HIP_CHECK(hipMemsetAsync(d->pos, 0, 4, st));
    CSDR_HIP_CHECK(hipMemsetAsync(d->repeated, 0, (size_t)B * c.vocab, st));
    CSDR_HIP_CHECK(hipMemsetAsync(d->ring, 0xFF, (size_t)B * cap * 4, st));
    CSDR_HIP_CHECK(hipMemcpy2DAsync(d->ring, cap * 4, prompt, (size_t)n_prompt * 4,
                                    (size_t)n_prompt * 4, B, hipMemcpyHostToDevice, st));
    const int body = n_prompt - 1;
    if (d->prefill_chunk > 0 && body > 0) {
        // positions [0, body) in multi-token passes, then the last one as a decode step
        const int chunk = std::min(d->prefill_chunk, body);
        RC(ensure_prefill(d, B * chunk));
        for (int p0 = 0; p0 < body; p0 += chunk) RC(prefill_pass(d, p0, std::min(chunk, body - p0), st));
        CSDR_HIP_CHECK(hipMemcpyAsync(d->pos, &body, 4, hipMemcpyHostToDevice, st));
    } else {
        for (int i = 0; i < body; ++i) RC(run_step(d, 0, temperature, penalty));
    }
    RC(run_step(d, 1, temperature, penalty));
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    d->host_pos = n_prompt;
    d->n_prompt = n_prompt;
    return CSDR_OK;
}

CSDR_API int csdr_decoder_set_lazy_selection(csdr_decoder* d, const csdr_lazy_hsdr* emb,
                                             float penalty) {
    if (!d) return set_error(CSDR_E_INVALID, "decoder_set_lazy_selection: null handle");
    if (emb) {
        uint32_t rows = 0, cols = 0;
        RC(csdr_lazy_hsdr_info(emb, &rows, &cols));
        if (rows != (uint32_t)d->cfg.vocab || cols != (uint32_t)d->cfg.hidden)
            return set_error(CSDR_E_INVALID,
                             "decoder_set_lazy_selection: embedding is " + std::to_string(rows) +
                                 " x " + std::to_string(cols) + ", expected vocab x hidden " +
                                 std::to_string(d->cfg.vocab) + " x " + std::to_string(d->cfg.hidden));
        const size_t need = csdr_lazy_hsdr_workspace_bytes(emb, d->B);
        if (need > d->ws_lazy_bytes) {
            unsigned char* p = nullptr;
            RC(dalloc(d, &p, need));
            d->ws_lazy = p;
            d->ws_lazy_bytes = need;
        }
    }
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    destroy_graphs(d);
    d->lazy = emb;
    d->lazy_penalty = penalty;
    return CSDR_OK;
}

CSDR_API int csdr_decoder_set_prefill_chunk(csdr_decoder* d, int tokens) {
    if (!d || tokens < 0) return set_error(CSDR_E_INVALID, "decoder_set_prefill_chunk: bad argument");
    d->prefill_chunk = std::min(tokens, d->cfg.max_ctx);
    return CSDR_OK;
}

CSDR_API int csdr_decoder_decode(csdr_decoder* d, int n_steps, float temperature, float penalty) {
    RC(ready(d));
    if (n_steps < 0) return set_error(CSDR_E_INVALID, "decoder_decode: negative step count");
    if (d->n_prompt == 0) return set_error(CSDR_E_INVALID, "decoder_decode: prefill first");
    if (d->host_pos + n_steps > d->cfg.max_ctx)
        return set_error(CSDR_E_INVALID, "decoder_decode: context capacity exceeded");
    if (d->use_graph) RC(ensure_graph(d, 1, temperature, penalty));
    for (int i = 0; i < n_steps; ++i) RC(run_step(d, 1, temperature, penalty));
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    d->host_pos += n_steps;
    return CSDR_OK;
}

CSDR_API int csdr_decoder_tokens(const csdr_decoder* d, int first, int count, int32_t* out) {
    if (!d || !out || first < 0 || count < 0 || first + count > d->cfg.max_ctx + 1)
        return set_error(CSDR_E_INVALID, "decoder_tokens: bad argument");
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    const size_t cap = (size_t)d->cfg.max_ctx + 1;
    if (count)
        CSDR_HIP_CHECK(hipMemcpy2D(out, (size_t)count * 4, d->ring + first, cap * 4,
                                   (size_t)count * 4, d->B, hipMemcpyDeviceToHost));
    return CSDR_OK;
}

CSDR_API int csdr_decoder_generate(csdr_decoder* d, const int32_t* prompt, int n_prompt,
                                   int max_new_tokens, float temperature, float penalty,
                                   int eos_id, int32_t* out_tokens, int* n_generated) {
    if (!d || !out_tokens || !n_generated)
        return set_error(CSDR_E_INVALID, "decoder_generate: null argument");
    *n_generated = 0;
    const int steps = std::max(1, max_new_tokens);
    if ((long long)n_prompt + steps > d->cfg.max_ctx + 1LL)
        return set_error(CSDR_E_INVALID, "decoder_generate: context capacity exceeded");
    RC(csdr_decoder_prefill(d, prompt, n_prompt, temperature, penalty));
    RC(csdr_decoder_decode(d, steps - 1, temperature, penalty));
    RC(csdr_decoder_tokens(d, n_prompt, steps, out_tokens));
    bool any = false;
    for (int b = 0; b < d->B; ++b) {
        const int32_t* t = out_tokens + (size_t)b * steps;
        int n = 0;
        while (n < steps) {
            if (t[n] < 0) break;  // no finite score: the reference fails the step
            ++n;
            if (eos_id >= 0 && t[n - 1] == eos_id) break;
        }
        n_generated[b] = n;
        any = any || n > 0;
    }
    if (!any) return set_error(CSDR_E_UNSUPPORTED, "decoder_generate: no finite logit");
    return CSDR_OK;
}

CSDR_API int csdr_decoder_logits(const csdr_decoder* d, float* out) {
    if (!d || !out) return set_error(CSDR_E_INVALID, "decoder_logits: bad argument");
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    CSDR_HIP_CHECK(
        hipMemcpy(out, d->logits, (size_t)d->B * d->cfg.vocab * 4, hipMemcpyDeviceToHost));
    return CSDR_OK;
}

CSDR_API int csdr_decoder_position(const csdr_decoder* d) { return d ? d->host_pos : -1; }

// Imports a precomputed context: K and V of positions [0, n) for `layer` (fp16
// [position][kv head][head_dim], host or device memory).
CSDR_API int csdr_decoder_load_kv(csdr_decoder* d, int layer, const uint16_t* k, const uint16_t* v,
                                  int n) {
    if (!d || layer < 0 || layer >= d->cfg.n_layers || !k || !v || n < 0 || n > d->cfg.max_ctx)
        return set_error(CSDR_E_INVALID, "decoder_load_kv: bad argument");
    // sequence b's n rows follow sequence b - 1's in the source, and start at b * max_ctx in
    // the cache
    const size_t kvw = (size_t)d->cfg.n_kv_heads * d->cfg.head_dim;
    const size_t row = kvw * 2;
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    if (!n) return CSDR_OK;
    if (d->cfg.kv_dtype == CSDR_F16) {
        CSDR_HIP_CHECK(hipMemcpy2D(d->layers[layer].kc, row * d->cfg.max_ctx, k, row * n, row * n,
                                   d->B, hipMemcpyDefault));
        CSDR_HIP_CHECK(hipMemcpy2D(d->layers[layer].vc, row * d->cfg.max_ctx, v, row * n, row * n,
                                   d->B, hipMemcpyDefault));
        return CSDR_OK;
    }
    // fp32 cache: the fp16 rows staged on the device, then widened into place
    const size_t count = (size_t)d->B * n * kvw;
    uint16_t* stage = nullptr;
    CSDR_HIP_CHECK(hipMalloc(&stage, count * 2));
    int rc = CSDR_OK;
    for (int which = 0; which < 2 && rc == CSDR_OK; ++which) {
        if (hipMemcpy(stage, which ? v : k, count * 2, hipMemcpyDefault) != hipSuccess) {
            rc = set_error(CSDR_E_HIP, "decoder_load_kv: staging copy failed");
            break;
        }
        float* dst = static_cast<float*>(which ? d->layers[layer].vc : d->layers[layer].kc);
        widen_kv_kernel<<<(unsigned)std::min<size_t>((count + 255) / 256, 65536), 256, 0,
                          d->stream>>>(stage, (size_t)n * kvw, (size_t)d->cfg.max_ctx * kvw,
                                       count, dst);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(d->stream) != hipSuccess)
            rc = set_error(CSDR_E_HIP, "decoder_load_kv: widening failed");
    }
    (void)hipFree(stage);
    return rc;
}

// Continues from an imported context: positions [0, position) count as processed and
// `token` is the token at `position` (the next decode step consumes it). The
// generated-token set starts empty.
CSDR_API int csdr_decoder_set_position(csdr_decoder* d, int position, int32_t token) {
    if (!d) return set_error(CSDR_E_INVALID, "decoder_set_position: bad argument");
    std::vector<int32_t> t((size_t)d->B, token);
    return csdr_decoder_set_position_batch(d, position, t.data());
}

CSDR_API int csdr_decoder_set_position_batch(csdr_decoder* d, int position,
                                             const int32_t* tokens) {
    if (!d || !tokens || position < 0 || position >= d->cfg.max_ctx)
        return set_error(CSDR_E_INVALID, "decoder_set_position: bad argument");
    for (int b = 0; b < d->B; ++b)
        if (tokens[b] < 0 || tokens[b] >= d->cfg.vocab)
            return set_error(CSDR_E_INVALID, "decoder_set_position: token id out of range");
    const size_t cap = (size_t)d->cfg.max_ctx + 1;
    CSDR_HIP_CHECK(hipStreamSynchronize(d->stream));
    hipStream_t st = d->stream;
    CSDR_HIP_CHECK(hipMemcpyAsync(d->pos, &position, 4, hipMemcpyHostToDevice, st));
    CSDR_HIP_CHECK(hipMemsetAsync(d->repeated, 0, (size_t)d->B * d->cfg.vocab, st));
    CSDR_HIP_CHECK(hipMemsetAsync(d->ring, 0xFF, (size_t)d->B * cap * 4, st));
    CSDR_HIP_CHECK(hipMemcpy2DAsync(d->ring + position, cap * 4, tokens, 4, 4, d->B,
                                    hipMemcpyHostToDevice, st));
    CSDR_HIP_CHECK(hipStreamSynchronize(st));
    d->host_pos = position;
    d->n_prompt = std::max(1, position);
    return CSDR_OK;
}

CSDR_API int csdr_decoder_batch(const csdr_decoder* d) { return d ? d->B : -1; }

}  // extern "C"
