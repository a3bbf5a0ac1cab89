// engine.cpp — the SDK inference-engine C API (cortex_inference_engine_*) over the device path.
//
// Reference (cortexSDR tree): api/cortex_sdk.cpp — CortexInferenceEngine (:72-111), create
// (:1752-1791), the option setters (:1793-1870), run_layer (:1888-1931), generate_text
// (:1951-2054), discover_native_llm_paths (:477-545), infer_attention_layout (:1311-1352);
// the routing underneath it, SDRModelLoader::matmulHSDR and SDRInferenceEngine::matmulForLayer
// (SparseInferenceEngine.cpp:1074-1091, 1271-1311).
//
// One engine = one open .sdr archive (archive.cpp) + a device cache of loaded segments keyed
// by index entry: strategy 5 payloads become csdr_hsdb segments, uncoded fp32 2-D tensors and
// strategy-0 GGUF block tensors (every format decodeSupportedGGUFQuantized decodes,
// SparseInferenceEngine.cpp:276-469) are uploaded as they are. Every product runs on the engine's HIP
// stream; host buffers are staged through pinned-free device staging buffers owned by the
// engine. generate_text builds a csdr_decoder from the archive's blk.N.* tensors.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <regex>
#include <exception>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/cortex_sdk_gpu.h"
#include "common.hpp"

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
// A csdr_* status as an SDK error.
CortexError from_csdr(int rc, const std::string& what) {
    int code = CORTEX_ERROR_UNKNOWN;
    switch (rc) {
        case CSDR_E_INVALID: code = CORTEX_ERROR_INVALID_ARGUMENT; break;
        case CSDR_E_FORMAT:
        case CSDR_E_TRUNCATED: code = CORTEX_ERROR_DECOMPRESSION; break;
        case CSDR_E_HIP: code = CORTEX_ERROR_INFERENCE; break;
        case CSDR_E_WORKSPACE: code = CORTEX_ERROR_MEMORY; break;
        case CSDR_E_UNSUPPORTED: code = CORTEX_ERROR_UNSUPPORTED_FORMAT; break;
        default: break;
    }
    return fail(code, what + ": " + csdr_last_error());
}

std::string lower(std::string s) {
    for (auto& c : s) c = (char)std::tolower((unsigned char)c);
    return s;
}

enum Kind { kHsdb, kDense, kQ4k, kGguf };

struct Cached {
    Kind kind = kHsdb;
    int gguf = -1;        // kGguf: CSDR_GGUF_* format
    csdr_hsdb* seg = nullptr;
    void* dev = nullptr;  // dense fp32 W or GGUF blocks
    uint32_t R = 0, C = 0;
    size_t bytes = 0;
    uint64_t last_use = 0;
    bool pinned = false;  // held by the decoder
};

std::mutex g_mu;
std::unordered_set<const void*> g_live;

}  // namespace

struct CortexInferenceEngine {
    csdr_archive* ar = nullptr;
    hipStream_t st = nullptr;
    std::unordered_map<size_t, Cached> cache;
    uint64_t tick = 0;
    size_t cache_bytes = 0, budget = 0;
    size_t batch = 1;
    bool dropout = false, training = false, aggressive = false, prefetch = true;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    float* xd = nullptr;
    float* yd = nullptr;
    size_t xcap = 0, ycap = 0;
    std::string stats = "{}";
    csdr_decoder* dec = nullptr;
    int dec_ctx = 0;
    std::string emb_name;           // the decoder's token embedding segment
    int lazy_mode = 0;              // token choice by the CLI's lazy HSDR scoring (0 = off)
    csdr_lazy_hsdr* lazy = nullptr;
    int lazy_loaded_mode = 0;
    // aggressive memory: the decoder's blocks are host-resident segments streamed to the
    // device when they run (owned here, released with the decoder)
    std::vector<csdr_hsdb*> host_segs;
    bool dec_streamed = false;
};

namespace {

bool live(const CortexInferenceEngine* e) {
    std::lock_guard<std::mutex> g(g_mu);
    return e && g_live.count(e);
}

void release(Cached& c) {
    if (c.seg) csdr_hsdb_free(c.seg);
    if (c.dev) (void)hipFree(c.dev);
    c.seg = nullptr;
    c.dev = nullptr;
}

void evict(CortexInferenceEngine* e, size_t idx) {
    auto it = e->cache.find(idx);
    if (it == e->cache.end() || it->second.pinned) return;
    (void)hipStreamSynchronize(e->st);
    e->cache_bytes -= it->second.bytes;
    release(it->second);
    e->cache.erase(it);
}

// Least recently used unpinned segments go until `need` more bytes fit the budget.
void make_room(CortexInferenceEngine* e, size_t need) {
    while (e->budget && e->cache_bytes + need > e->budget) {
        size_t victim = (size_t)-1;
        uint64_t oldest = UINT64_MAX;
        for (auto& kv : e->cache)
            if (!kv.second.pinned && kv.second.last_use < oldest) {
                oldest = kv.second.last_use;
                victim = kv.first;
            }
        if (victim == (size_t)-1) break;
        evict(e, victim);
    }
}

int grow(void** p, size_t* cap, size_t bytes) {
    if (*cap >= bytes && *p) return CSDR_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    CSDR_HIP_CHECK(hipMalloc(p, std::max<size_t>(bytes, 256)));
    CSDR_HIP_CHECK(hipMemset(*p, 0, std::max<size_t>(bytes, 256)));
    // the fill runs on the null stream, which does not order the engine's non-blocking
    // stream: without this wait it can land after the next upload or product
    CSDR_HIP_CHECK(hipDeviceSynchronize());
    *cap = bytes;
    return CSDR_OK;
}

// Entry for `name`, else `name.weight` (applyLinearLayer's fallback).
bool resolve(const CortexInferenceEngine* e, const std::string& name, size_t* idx) {
    if (csdr_archive_find(e->ar, name.c_str(), idx) == CSDR_OK) return true;
    return csdr_archive_find(e->ar, (name + ".weight").c_str(), idx) == CSDR_OK;
}

CortexError load(CortexInferenceEngine* e, size_t idx, Cached** out) {
    auto it = e->cache.find(idx);
    if (it != e->cache.end()) {
        it->second.last_use = ++e->tick;
        *out = &it->second;
        return ok();
    }
    csdr_segment_info info;
    csdr_archive_info(e->ar, idx, &info);
    const std::string name = info.name;
    // the size is bounded by the archive file (the index reader checks every entry against it)
    std::vector<uint8_t> bytes;
    try {
        bytes.resize((size_t)info.compressed_size);
    } catch (const std::exception&) {
        return fail(CORTEX_ERROR_MEMORY, "out of host memory reading '" + name + "'");
    }
    int rc = csdr_archive_read(e->ar, idx, bytes.data(), bytes.size(), nullptr);
    if (rc) return from_csdr(rc, "load '" + name + "'");
    Cached c;
    const std::string fmt = lower(info.data_format);
    if (info.strategy_id == 5) {
        make_room(e, bytes.size());
        rc = csdr_hsdb_load(bytes.data(), bytes.size(), e->st, &c.seg);
        if (rc) return from_csdr(rc, "matmulHSDR: segment '" + name + "'");
        csdr_hsdb_info hi;
        csdr_hsdb_get_info(c.seg, &hi);
        c.kind = kHsdb;
        c.R = hi.rows;
        c.C = hi.cols;
        c.bytes = hi.device_bytes;
    } else if (info.strategy_id == 0 && (csdr_gguf_format(fmt.c_str()) >= 0 || fmt == "f32" ||
                                         fmt == "fp32" ||
                                         (fmt.empty() && info.original_type == 1))) {
        if (!info.has_metadata || info.n_dims != 2)
            return fail(CORTEX_ERROR_INFERENCE,
                        "matmulForLayer: segment '" + name +
                            "' has no 2-D tensor_metadata; cannot fall back to dense matmul");
        c.R = info.dims[0];
        c.C = info.dims[1];
        const bool q4k = (fmt == "q4_k");
        const int gg = q4k ? -1 : csdr_gguf_format(fmt.c_str());
        int bb = 4, be = 1;  // bytes per element group (fp32: 4 bytes per element)
        if (q4k) {
            bb = 144;
            be = 256;
        } else if (gg >= 0) {
            csdr_gguf_block(gg, &bb, &be);
        }
        const size_t want = (size_t)c.R * c.C / be * bb;
        if (c.C % be || bytes.size() != want)
            return fail(CORTEX_ERROR_INFERENCE, "matmulForLayer: segment '" + name + "' holds " +
                                                    std::to_string(bytes.size()) +
                                                    " bytes, expected " + std::to_string(want));
        make_room(e, want);
        if (hipMalloc(&c.dev, want) != hipSuccess)
            return fail(CORTEX_ERROR_MEMORY, "device allocation for '" + name + "' failed");
        if (hipMemcpy(c.dev, bytes.data(), want, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(c.dev);
            return fail(CORTEX_ERROR_INFERENCE, "upload of '" + name + "' failed");
        }
        c.kind = q4k ? kQ4k : (gg >= 0 ? kGguf : kDense);
        c.gguf = gg;
        c.bytes = want;
    } else {
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                    "segment '" + name + "' (strategy " + std::to_string(info.strategy_id) +
                        ", format '" + info.data_format +
                        "') is not served by the device path: strategy 5 (HSDR/HSDB), or "
                        "strategy 0 with fp32 or a GGUF block format the engine decodes");
    }
    c.last_use = ++e->tick;
    e->cache_bytes += c.bytes;
    auto res = e->cache.emplace(idx, c);
    *out = &res.first->second;
    return ok();
}

// Host floats of an uncoded vector segment (norm weights).
CortexError read_vector(CortexInferenceEngine* e, const std::string& name, size_t n,
                        std::vector<float>& out) {
    size_t idx;
    if (!resolve(e, name, &idx)) return fail(CORTEX_ERROR_INFERENCE, "Segment not found: " + name);
    csdr_segment_info info;
    csdr_archive_info(e->ar, idx, &info);
    if (info.strategy_id != 0 || info.compressed_size != n * 4)
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                    "segment '" + name + "' is not an uncoded fp32 vector of " +
                        std::to_string(n) + " floats");
    out.resize(n);
    int rc = csdr_archive_read(e->ar, idx, out.data(), n * 4, nullptr);
    if (rc) return from_csdr(rc, "read '" + name + "'");
    return ok();
}

// Every input finite and within fp16's range, so x = fp16(x) + fp16(x - fp16(x)) holds to
// about 2^-22 of each element.
bool split_ok(const float* x, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!(std::fabs(x[i]) <= 32768.0f)) return false;
    return true;
}

char* dup_c(const std::string& s) {
    char* p = static_cast<char*>(std::malloc(s.size() + 1));
    if (p) std::memcpy(p, s.c_str(), s.size() + 1);
    return p;
}

// ---- decoder discovery (discover_native_llm_paths, cortex_sdk.cpp:477-545)

struct Block {
    std::string attn_norm, q, k, v, o, ffn_norm, gate, up, down;
    bool complete() const {
        return !attn_norm.empty() && !q.empty() && !k.empty() && !v.empty() && !o.empty() &&
               !ffn_norm.empty() && !gate.empty() && !up.empty() && !down.empty();
    }
};

void free_decoder(CortexInferenceEngine* e) {
    if (e->dec) csdr_decoder_free(e->dec);
    e->dec = nullptr;
    e->dec_ctx = 0;
    for (csdr_hsdb* s : e->host_segs) csdr_hsdb_free(s);
    e->host_segs.clear();
}

// A strategy-5 segment loaded with its codes in pinned host memory (not cached on the
// device): the unit of the on-demand layer loading (loadLayerByNameAsync,
// SparseInferenceEngine.cpp:1101-1224).
CortexError load_host(CortexInferenceEngine* e, const std::string& name, csdr_hsdb** out) {
    size_t idx;
    if (!resolve(e, name, &idx)) return fail(CORTEX_ERROR_INFERENCE, "Segment not found: " + name);
    csdr_segment_info info;
    csdr_archive_info(e->ar, idx, &info);
    if (info.strategy_id != 5)
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                    "decoder: '" + name + "' must be an HSDR/HSDB (strategy 5) segment");
    std::vector<uint8_t> bytes((size_t)info.compressed_size);
    int rc = csdr_archive_read(e->ar, idx, bytes.data(), bytes.size(), nullptr);
    if (rc) return from_csdr(rc, "load '" + name + "'");
    rc = csdr_hsdb_load_host(bytes.data(), bytes.size(), e->st, out);
    if (rc) return from_csdr(rc, "decoder: segment '" + name + "'");
    e->host_segs.push_back(*out);
    return ok();
}

CortexError build_decoder(CortexInferenceEngine* e, int ctx) {
    std::string emb, out_norm, out_proj;
    std::map<size_t, Block> blocks;
    const std::regex blk(R"(blk\.(\d+)\.)");
    const size_t n = csdr_archive_count(e->ar);
    for (size_t i = 0; i < n; ++i) {
        csdr_segment_info info;
        csdr_archive_info(e->ar, i, &info);
        const std::string cand = (info.layer_name && *info.layer_name) ? info.layer_name : info.name;
        const std::string lc = lower(cand);
        if (emb.empty() && (lc.find("token_embd") != std::string::npos ||
                            lc.find("tok_embeddings") != std::string::npos ||
                            lc.find("embed_tokens") != std::string::npos))
            emb = info.name;
        if (out_norm.empty() && (lc == "output_norm" || lc == "output_norm.weight" ||
                                 lc.find("model.norm") != std::string::npos))
            out_norm = info.name;
        if (out_proj.empty() && (lc == "output" || lc == "output.weight" ||
                                 lc.find("lm_head") != std::string::npos))
            out_proj = info.name;
        std::smatch m;
        if (std::regex_search(cand, m, blk)) {
            Block& b = blocks[(size_t)std::stoull(m[1].str())];
            const std::string& nm = info.name;
            if (lc.find("attn_norm") != std::string::npos) b.attn_norm = nm;
            else if (lc.find("attn_q") != std::string::npos) b.q = nm;
            else if (lc.find("attn_k") != std::string::npos) b.k = nm;
            else if (lc.find("attn_v") != std::string::npos) b.v = nm;
            else if (lc.find("attn_output") != std::string::npos) b.o = nm;
            else if (lc.find("ffn_norm") != std::string::npos) b.ffn_norm = nm;
            else if (lc.find("ffn_gate") != std::string::npos) b.gate = nm;
            else if (lc.find("ffn_up") != std::string::npos) b.up = nm;
            else if (lc.find("ffn_down") != std::string::npos) b.down = nm;
        }
    }
    std::vector<Block> layers;
    for (auto& kv : blocks)
        if (kv.second.complete()) layers.push_back(kv.second);
    if (emb.empty() || layers.empty())
        return fail(CORTEX_ERROR_INFERENCE,
                    "No complete GGUF transformer blocks were discovered (need token_embd and "
                    "blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_output,ffn_norm,ffn_gate,"
                    "ffn_up,ffn_down})");
    auto seg_of = [&](const std::string& name, Cached** c) -> CortexError {
        size_t idx;
        if (!resolve(e, name, &idx)) return fail(CORTEX_ERROR_INFERENCE, "Segment not found: " + name);
        CortexError r = load(e, idx, c);
        if (r.code) return r;
        if ((*c)->kind != kHsdb)
            return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                        "decoder: '" + name + "' must be an HSDR/HSDB (strategy 5) segment");
        (*c)->pinned = true;
        return ok();
    };
    Cached* embc = nullptr;
    CortexError r = seg_of(emb, &embc);
    if (r.code) return r;
    const uint32_t vocab = embc->R, H = embc->C;
    Cached* lmc = embc;
    if (!out_proj.empty()) {
        Cached* c = nullptr;
        r = seg_of(out_proj, &c);
        if (r.code) return r;
        if (c->R == vocab && c->C == H) lmc = c;  // can_use_logits_projection: shape check
    }
    Cached *q0, *k0, *v0, *g0;
    if ((r = seg_of(layers[0].q, &q0)).code || (r = seg_of(layers[0].k, &k0)).code ||
        (r = seg_of(layers[0].v, &v0)).code || (r = seg_of(layers[0].gate, &g0)).code)
        return r;
    // infer_attention_layout (cortex_sdk.cpp:1311-1352): first head size in the reference's
    // preference order that divides q/k/v widths into a valid GQA split
    int hd = 0;
    for (int cand : {128, 64, 256, 32, 16}) {
        if (q0->R % cand || k0->R % cand || v0->R % cand) continue;
        const uint32_t qh = q0->R / cand, kh = k0->R / cand, vh = v0->R / cand;
        if (!qh || !kh || !vh || qh < kh || qh < vh || qh % kh || qh % vh) continue;
        hd = cand;
        break;
    }
    if (hd != 64 && hd != 128)
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                    "decoder: attention layout needs head size 64 or 128 (inferred " +
                        std::to_string(hd) + ")");
    csdr_decoder_config cfg{};
    cfg.n_layers = (int)layers.size();
    cfg.hidden = (int)H;
    cfg.head_dim = hd;
    cfg.n_heads = (int)(q0->R / hd);
    cfg.n_kv_heads = (int)(k0->R / hd);
    cfg.ffn = (int)g0->R;
    cfg.vocab = (int)vocab;
    cfg.max_ctx = ctx;
    cfg.rope_theta = 1000000.0f;  // get_rope_cache default (cortex_sdk.cpp:1363)
    cfg.rms_eps = 1e-5f;          // rms_norm default (cortex_sdk.cpp:1212)
    if (q0->R != H)
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT, "decoder: attn_q must be hidden x hidden");
    free_decoder(e);
    int rc = csdr_decoder_create(&cfg, &e->dec);
    if (rc) return from_csdr(rc, "decoder");
    // aggressive memory management: blocks are not kept on the device; each is streamed
    // from pinned host memory when it runs (runLayersOnDemand, SparseInferenceEngine.cpp:
    // 2911-3027), the next block's copy overlapping the current one when prefetch is on
    const bool streamed = e->aggressive;
    for (size_t l = 0; l < layers.size(); ++l) {
        const Block& b = layers[l];
        csdr_hsdb* w[7];
        const std::string* names[7] = {&b.q, &b.k, &b.v, &b.o, &b.gate, &b.up, &b.down};
        for (int i = 0; i < 7; ++i) {
            if (streamed) {
                if ((r = load_host(e, *names[i], &w[i])).code) return r;
            } else {
                Cached* c = nullptr;
                if ((r = seg_of(*names[i], &c)).code) return r;
                w[i] = c->seg;
            }
        }
        std::vector<float> an, fn;
        if ((r = read_vector(e, b.attn_norm, H, an)).code || (r = read_vector(e, b.ffn_norm, H, fn)).code)
            return r;
        rc = csdr_decoder_set_layer(e->dec, (int)l, w[0], w[1], w[2], w[3], w[4], w[5], w[6],
                                    an.data(), fn.data(), nullptr, nullptr, nullptr);
        if (rc) return from_csdr(rc, "decoder block " + std::to_string(l));
    }
    rc = csdr_decoder_set_layer_prefetch(e->dec, e->prefetch ? 1 : 0);
    if (rc) return from_csdr(rc, "decoder prefetch");
    e->dec_streamed = streamed;
    if (streamed)  // block 0's device copies only served the shape discovery above
        for (Cached* c : {q0, k0, v0, g0}) c->pinned = false;
    std::vector<float> onw;
    if (!out_norm.empty() && (r = read_vector(e, out_norm, H, onw)).code) return r;
    rc = csdr_decoder_set_output(e->dec, lmc->seg, onw.empty() ? nullptr : onw.data(),
                                 embc == lmc ? nullptr : embc->seg);
    if (rc) return from_csdr(rc, "decoder output");
    e->dec_ctx = ctx;
    e->emb_name = emb;
    return ok();
}

// The text CLI's lazy HSDR embedding of the decoder's token embedding (its raw strategy-5
// stream, 1-row tiles), read with the mode's code reading; applied to the decoder, or removed.
CortexError apply_lazy(CortexInferenceEngine* e) {
    if (!e->lazy_mode) {
        const int rc = csdr_decoder_set_lazy_selection(e->dec, nullptr, 0.0f);
        return rc ? from_csdr(rc, "lazy selection") : ok();
    }
    if (!e->lazy || e->lazy_loaded_mode != e->lazy_mode) {
        if (e->lazy) csdr_lazy_hsdr_free(e->lazy);
        e->lazy = nullptr;
        size_t idx;
        if (!resolve(e, e->emb_name, &idx))
            return fail(CORTEX_ERROR_INFERENCE, "Segment not found: " + e->emb_name);
        csdr_segment_info info;
        csdr_archive_info(e->ar, idx, &info);
        if (info.strategy_id != 5)
            return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                        "lazy HSDR selection: the token embedding is not HSDR-coded");
        std::vector<uint8_t> bytes((size_t)info.compressed_size);
        int rc = csdr_archive_read(e->ar, idx, bytes.data(), bytes.size(), nullptr);
        if (rc) return from_csdr(rc, "lazy HSDR selection: read '" + e->emb_name + "'");
        rc = csdr_lazy_hsdr_load(bytes.data(), bytes.size(),
                                 e->lazy_mode == 2 ? CSDR_LAZY_UNPACK_CLI : CSDR_LAZY_UNPACK_PACKED,
                                 e->st, &e->lazy);
        if (rc) return from_csdr(rc, "lazy HSDR selection: '" + e->emb_name + "'");
        e->lazy_loaded_mode = e->lazy_mode;
    }
    // select_next_token_from_lazy_hsdr's repeat penalty (cortexsdr_cli.cpp:723-725)
    const int rc = csdr_decoder_set_lazy_selection(e->dec, e->lazy, 1.0f);
    return rc ? from_csdr(rc, "lazy selection") : ok();
}

// getExecutionOrder without a graph (SparseInferenceEngine.cpp:2852-2893): the weight-like
// segments (isWeightLikeSegmentType :91-100) and executable op layers (:102-130), those with
// a layer name first by (layer index, layer name), then by name; each under its execution
// name (deriveExecutionName :529-547: the layer name, else the name without a weight/bias
// suffix), token embeddings skipped, each name once.
std::vector<std::string> execution_order(const CortexInferenceEngine* e) {
    struct Cand {
        std::string name, layer_name;
        uint32_t layer_index;
    };
    static const char* const kOps[] = {"add", "sub", "mul", "div", "relu", "sigmoid", "tanh",
                                       "softmax", "gelu", "leakyrelu", "elu", "silu", "swish",
                                       "reshape", "transpose", "flatten", "concat", "slice"};
    std::vector<Cand> cands;
    const size_t n = csdr_archive_count(e->ar);
    for (size_t i = 0; i < n; ++i) {
        csdr_segment_info info;
        csdr_archive_info(e->ar, i, &info);
        const uint32_t t = info.original_type;
        bool take = t == 1 || t == 2 || t == 3 || t == 4 || (t >= 11 && t <= 14);
        const std::string lt = lower(info.layer_type ? info.layer_type : "");
        for (const char* op : kOps) take = take || lt == op;
        if (take)
            cands.push_back({info.name, info.layer_name ? info.layer_name : "", info.layer_index});
    }
    std::stable_sort(cands.begin(), cands.end(), [](const Cand& a, const Cand& b) {
        const bool ha = !a.layer_name.empty(), hb = !b.layer_name.empty();
        if (ha != hb) return ha > hb;
        if (ha && hb) {
            if (a.layer_index != b.layer_index) return a.layer_index < b.layer_index;
            if (a.layer_name != b.layer_name) return a.layer_name < b.layer_name;
        }
        return a.name < b.name;
    });
    static const char* const kSuffixes[] = {".weight", ".weights", ".bias", "/weight",
                                            "/weights", "/bias", "_weight", "_bias"};
    std::vector<std::string> order;
    std::unordered_set<std::string> seen;
    for (const Cand& c : cands) {
        std::string x = c.layer_name;
        if (x.empty()) {
            x = c.name;
            for (const char* suf : kSuffixes) {
                const size_t k = std::strlen(suf);
                if (x.size() > k && x.compare(x.size() - k, k, suf) == 0) {
                    x.erase(x.size() - k);
                    break;
                }
            }
        }
        const std::string lx = lower(x);
        if (lx.find("token_embd") != std::string::npos ||
            lx.find("tok_embeddings") != std::string::npos ||
            lx.find("embed_tokens") != std::string::npos)
            continue;
        if (!x.empty() && seen.insert(x).second) order.push_back(x);
    }
    return order;
}

const char* path_name(const Cached* c) {
    return c->kind == kHsdb   ? "hsdb"
           : c->kind == kQ4k  ? "q4_k"
           : c->kind == kGguf ? "gguf"
                              : "dense_f32";
}

// y (M x R, host) = x (M x C, host) . W^T through the loaded segment's device path (the
// body of run_layer and of each layer of run); *dev_ms gets the device time.
CortexError run_linear(CortexInferenceEngine* e, Cached* c, const std::string& layer_name,
                       const float* input, size_t M, std::vector<float>& output, float* dev_ms) {
    const size_t R = c->R, C = c->C, input_size = M * C;
    int rc = grow((void**)&e->xd, &e->xcap, input_size * 4);
    if (!rc) rc = grow((void**)&e->yd, &e->ycap, M * R * 4);
    if (rc) return from_csdr(rc, "staging");
    std::vector<float> host;
    bool split = false;  // Q4_K / GGUF batch through the matrix cores (fp16 hi + lo inputs)
    hipEvent_t ev0, ev1;
    (void)hipEventCreate(&ev0);
    (void)hipEventCreate(&ev1);
    struct Events {
        hipEvent_t a, b;
        ~Events() {
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
        }
    } evs{ev0, ev1};
    if (c->kind == kHsdb) {
        // M x C token-major in, the coded product takes C x M feature-major
        const float* xin = input;
        if (M > 1) {
            host.resize(input_size);
            for (size_t m = 0; m < M; ++m)
                for (size_t k = 0; k < C; ++k) host[k * M + m] = input[m * C + k];
            xin = host.data();
        }
        if (hipMemcpyAsync(e->xd, xin, input_size * 4, hipMemcpyHostToDevice, e->st) != hipSuccess)
            return fail(CORTEX_ERROR_INFERENCE, "input upload failed");
        const size_t need = csdr_hsdb_workspace_bytes(c->seg, (int)M);
        if ((rc = grow(&e->ws, &e->ws_bytes, need))) return from_csdr(rc, "workspace");
        (void)hipEventRecord(ev0, e->st);
        rc = csdr_hsdb_matmul(c->seg, e->xd, CSDR_F32, (int)M, e->yd, e->ws, e->ws_bytes, e->st);
    } else {
        const bool tc = (c->kind == kQ4k || c->kind == kGguf) && M > 1 &&
                        split_ok(input, input_size) && (c->kind == kQ4k || C % 16 == 0);
        if (!tc) {
            if (hipMemcpyAsync(e->xd, input, input_size * 4, hipMemcpyHostToDevice, e->st) !=
                hipSuccess)
                return fail(CORTEX_ERROR_INFERENCE, "input upload failed");
            (void)hipEventRecord(ev0, e->st);
        }
        if (tc) {
            // the matrix-core form for the whole batch: it reads fp16 activations, so the fp32
            // input goes in as two exact fp16 parts, hi = fp16(x) and lo = fp16(x - hi), whose
            // products are added in fp32 on the way out (x to about 2^-22, the weights read
            // twice instead of M times)
            split = true;
            std::vector<_Float16> parts(2 * input_size);
            for (size_t i = 0; i < input_size; ++i) {
                const _Float16 h = (_Float16)input[i];
                parts[i] = h;
                parts[input_size + i] = (_Float16)(input[i] - (float)h);
            }
            // the fp32 staging holds both fp16 parts; the second product's output follows y
            if ((rc = grow((void**)&e->yd, &e->ycap, 2 * M * R * 4)))
                return from_csdr(rc, "staging");
            (void)hipEventRecord(ev0, e->st);
            if (hipMemcpyAsync(e->xd, parts.data(), 2 * input_size * 2, hipMemcpyHostToDevice,
                               e->st) != hipSuccess)
                return fail(CORTEX_ERROR_INFERENCE, "input upload failed");
            const _Float16* xh = reinterpret_cast<const _Float16*>(e->xd);
            for (int part = 0; part < 2 && rc == CSDR_OK; ++part) {
                const _Float16* xp = xh + part * input_size;
                float* yp = e->yd + part * M * R;
                rc = c->kind == kQ4k
                         ? csdr_q4k_linear(c->dev, (int)R, (int)C, CSDR_Q4K_GGML, xp, CSDR_F16,
                                           (int)M, yp, e->st)
                         : csdr_gguf_linear(c->dev, c->gguf, (int)R, (int)C, xp, CSDR_F16,
                                            (int)M, yp, e->st);
            }
        } else if (c->kind == kQ4k || c->kind == kGguf) {
            // M == 1 (or inputs beyond fp16's range): the GEMV form on fp32 x, row by row
            rc = CSDR_OK;
            for (size_t m = 0; m < M && rc == CSDR_OK; ++m)
                rc = c->kind == kQ4k
                         ? csdr_q4k_linear(c->dev, (int)R, (int)C, CSDR_Q4K_GGML, e->xd + m * C,
                                           CSDR_F32, 1, e->yd + m * R, e->st)
                         : csdr_gguf_linear(c->dev, c->gguf, (int)R, (int)C, e->xd + m * C,
                                            CSDR_F32, 1, e->yd + m * R, e->st);
        } else {
            rc = csdr_dense_linear(static_cast<const float*>(c->dev), (int)R, (int)C, e->xd,
                                   (int)M, e->yd, e->st);
        }
    }
    (void)hipEventRecord(ev1, e->st);
    if (rc) return from_csdr(rc, "run_layer '" + layer_name + "'");
    host.resize((split ? 2 : 1) * M * R);
    if (hipMemcpyAsync(host.data(), e->yd, host.size() * 4, hipMemcpyDeviceToHost, e->st) !=
            hipSuccess ||
        hipStreamSynchronize(e->st) != hipSuccess)
        return fail(CORTEX_ERROR_INFERENCE, "output download failed");
    *dev_ms = 0.f;
    (void)hipEventElapsedTime(dev_ms, ev0, ev1);
    output.resize(M * R);
    if (c->kind == kHsdb && M > 1) {
        for (size_t r2 = 0; r2 < R; ++r2)
            for (size_t m = 0; m < M; ++m) output[m * R + r2] = host[r2 * M + m];
    } else if (split) {
        for (size_t i = 0; i < M * R; ++i) output[i] = host[i] + host[M * R + i];
    } else {
        std::memcpy(output.data(), host.data(), M * R * 4);
    }
    return ok();
}

}  // namespace

extern "C" {

CSDR_API CortexError cortex_inference_engine_create(const char* path,
                                                    CortexInferenceEngineHandle* handle) {
    CORTEX_GUARD_BEGIN
    if (!path || !handle)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid arguments (null pointers)");
    *handle = nullptr;
    auto* e = new (std::nothrow) CortexInferenceEngine();
    if (!e) return fail(CORTEX_ERROR_MEMORY, "out of host memory");
    int rc = csdr_archive_open(path, &e->ar);
    if (rc) {
        delete e;
        return fail(rc == CSDR_E_INVALID ? CORTEX_ERROR_FILE_IO : CORTEX_ERROR_DECOMPRESSION,
                    csdr_last_error());
    }
    if (hipStreamCreateWithFlags(&e->st, hipStreamNonBlocking) != hipSuccess) {
        csdr_archive_close(e->ar);
        delete e;
        return fail(CORTEX_ERROR_INFERENCE, "HIP stream creation failed (no device?)");
    }
    {
        std::lock_guard<std::mutex> g(g_mu);
        g_live.insert(e);
    }
    *handle = e;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_create")
}

CSDR_API CortexError cortex_inference_engine_free(CortexInferenceEngineHandle e) {
    CORTEX_GUARD_BEGIN
    {
        std::lock_guard<std::mutex> g(g_mu);
        if (!e || !g_live.erase(e)) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid handle");
    }
    (void)hipStreamSynchronize(e->st);
    free_decoder(e);
    if (e->lazy) csdr_lazy_hsdr_free(e->lazy);
    for (auto& kv : e->cache) release(kv.second);
    if (e->ws) (void)hipFree(e->ws);
    if (e->xd) (void)hipFree(e->xd);
    if (e->yd) (void)hipFree(e->yd);
    (void)hipStreamDestroy(e->st);
    csdr_archive_close(e->ar);
    delete e;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_free")
}

#define CHECK_HANDLE(e) \
    if (!live(e)) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid handle")

CSDR_API CortexError cortex_inference_engine_set_batch_size(CortexInferenceEngineHandle e,
                                                            size_t batch_size) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (batch_size == 0) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "batch size must be > 0");
    e->batch = batch_size;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_set_batch_size")
}

CSDR_API CortexError cortex_inference_engine_enable_dropout(CortexInferenceEngineHandle e,
                                                            int enable) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    e->dropout = enable != 0;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_enable_dropout")
}

CSDR_API CortexError cortex_inference_engine_set_mode(CortexInferenceEngineHandle e,
                                                      int training_mode) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    e->training = training_mode != 0;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_set_mode")
}

CSDR_API CortexError cortex_inference_engine_init_memory_pool(CortexInferenceEngineHandle e,
                                                              size_t max_memory_mb) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    e->budget = max_memory_mb * 1024 * 1024;
    make_room(e, 0);
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_init_memory_pool")
}

CSDR_API CortexError cortex_inference_engine_enable_aggressive_memory(
    CortexInferenceEngineHandle e, int enable) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    e->aggressive = enable != 0;
    // the decoder's blocks change residency: rebuilt at the next generate_text
    if (e->dec && e->dec_streamed != e->aggressive) free_decoder(e);
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_enable_aggressive_memory")
}

CSDR_API CortexError cortex_inference_engine_get_memory_usage(CortexInferenceEngineHandle e,
                                                              size_t* bytes) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!bytes) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "null output");
    *bytes = e->cache_bytes;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_get_memory_usage")
}

CSDR_API CortexError cortex_inference_engine_enable_layer_prefetch(CortexInferenceEngineHandle e,
                                                                   int enable) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    e->prefetch = enable != 0;
    if (e->dec) {
        const int rc = csdr_decoder_set_layer_prefetch(e->dec, e->prefetch ? 1 : 0);
        if (rc) return from_csdr(rc, "layer prefetch");
    }
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_enable_layer_prefetch")
}

CSDR_API CortexError cortex_inference_engine_get_last_run_stats_json(CortexInferenceEngineHandle e,
                                                                     char** out_json) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!out_json) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "null output");
    *out_json = dup_c(e->stats);
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_get_last_run_stats_json")
}

CSDR_API void cortex_free_string(char* s) { std::free(s); }

CSDR_API void cortex_error_free(CortexError* error) {
    if (error) error->message = nullptr;  // messages are library-owned (thread-local)
}

CSDR_API const char* cortex_sdk_version(void) { return "1.0.0-mi355x"; }

CSDR_API CortexError cortex_inference_engine_run(CortexInferenceEngineHandle e,
                                                 const float* input, size_t input_size,
                                                 float* output, size_t output_size,
                                                 size_t* actual_output_size) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!input || !output || !actual_output_size)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid arguments (null pointers)");
    *actual_output_size = 0;
    const auto t0 = std::chrono::steady_clock::now();
    // SDRInferenceEngine::run (SparseInferenceEngine.cpp:2220-2262) -> runLayersOnDemand
    // (:2911-3027): the archive's layers in execution order, each output the next input
    std::vector<float> cur(input, input + input_size), next;
    std::string layers_json;
    for (const std::string& name : execution_order(e)) {
        size_t idx;
        if (!resolve(e, name, &idx))
            return fail(CORTEX_ERROR_INFERENCE, "Segment info not found for layer: " + name);
        csdr_segment_info info;
        csdr_archive_info(e->ar, idx, &info);
        const auto l0 = std::chrono::steady_clock::now();
        Cached* c = nullptr;
        CortexError r = load(e, idx, &c);
        if (r.code == CORTEX_ERROR_UNSUPPORTED_FORMAT || r.code == CORTEX_ERROR_INFERENCE)
            return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                        "run: layer '" + name + "' is not a linear layer of the device path " +
                            "(strategy-5 HSDR/HSDB, fp32, q4_k or GGUF 2-D weights): " +
                            std::string(r.message ? r.message : ""));
        if (r.code) return r;
        const auto l1 = std::chrono::steady_clock::now();
        if (cur.empty() || cur.size() % c->C)
            return fail(CORTEX_ERROR_INFERENCE,
                        "run: layer '" + name + "' takes " + std::to_string(c->C) +
                            " input features; its input has " + std::to_string(cur.size()) +
                            " values");
        const size_t M = cur.size() / c->C;
        float ms = 0.f;
        r = run_linear(e, c, name, cur.data(), M, next, &ms);
        if (r.code) return r;
        if (c->kind != kHsdb) {
            // a loaded layer carries its bias segment (name.bias, loadLayerByName :1128-1137);
            // the HSDR stub of runLayersOnDemand (:2931-2955) carries only the shapes
            size_t bidx;
            if (csdr_archive_find(e->ar, (name + ".bias").c_str(), &bidx) == CSDR_OK) {
                std::vector<float> bias;
                r = read_vector(e, name + ".bias", c->R, bias);
                if (r.code) return r;
                for (size_t m = 0; m < M; ++m)
                    for (size_t j = 0; j < c->R; ++j) next[m * c->R + j] += bias[j];
            }
        }
        cur.swap(next);
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s{\"name\":\"%s\",\"path\":\"%s\",\"load_ms\":%.4f,"
                      "\"device_ms\":%.4f,\"output_size\":%zu}",
                      layers_json.empty() ? "" : ",", name.c_str(), path_name(c),
                      std::chrono::duration<double, std::milli>(l1 - l0).count(), ms,
                      cur.size());
        layers_json += buf;
        if (e->aggressive) evict(e, idx);
    }
    *actual_output_size = cur.size();
    if (cur.size() > output_size) return fail(CORTEX_ERROR_MEMORY, "Output buffer too small");
    std::copy(cur.begin(), cur.end(), output);
    char head[128];
    std::snprintf(head, sizeof head, "{\"total_ms\":%.4f,\"layers\":[",
                  std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                      .count());
    e->stats = std::string(head) + layers_json + "]}";
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_run")
}

CSDR_API CortexError cortex_inference_engine_run_layer(CortexInferenceEngineHandle e,
                                                       const char* layer_name,
                                                       const float* input, size_t input_size,
                                                       float* output, size_t output_size,
                                                       size_t* actual_output_size) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!layer_name || !input || !output || !actual_output_size)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid arguments (null pointers)");
    size_t idx;
    if (!resolve(e, layer_name, &idx))
        return fail(CORTEX_ERROR_INFERENCE, std::string("Segment not found: ") + layer_name);
    const auto t0 = std::chrono::steady_clock::now();
    Cached* c = nullptr;
    CortexError r = load(e, idx, &c);
    if (r.code) return r;
    const auto t1 = std::chrono::steady_clock::now();
    const size_t R = c->R, C = c->C;
    if (input_size == 0 || input_size % C)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT,
                    "input size " + std::to_string(input_size) + " is not a multiple of the "
                    "layer's " + std::to_string(C) + " input features");
    const size_t M = input_size / C;
    if (M > (size_t)1 << 20) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "batch too large");
    *actual_output_size = M * R;
    if (output_size < M * R) return fail(CORTEX_ERROR_MEMORY, "Output buffer too small");
    std::vector<float> y;
    float dev_ms = 0.f;
    r = run_linear(e, c, layer_name, input, M, y, &dev_ms);
    if (r.code) return r;
    std::memcpy(output, y.data(), M * R * 4);
    const auto t2 = std::chrono::steady_clock::now();
    char buf[512];
    std::snprintf(buf, sizeof buf,
                  "{\"layer\":\"%s\",\"path\":\"%s\",\"rows\":%zu,\"cols\":%zu,\"batch\":%zu,"
                  "\"load_ms\":%.4f,\"device_ms\":%.4f,\"total_ms\":%.4f,\"cached_bytes\":%zu}",
                  layer_name, path_name(c), R, C, M,
                  std::chrono::duration<double, std::milli>(t1 - t0).count(), dev_ms,
                  std::chrono::duration<double, std::milli>(t2 - t0).count(), e->cache_bytes);
    e->stats = buf;
    if (e->aggressive) evict(e, idx);
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_run_layer")
}

CSDR_API CortexError cortex_inference_engine_matmul_device(CortexInferenceEngineHandle e,
                                                           const char* layer_name, const void* x,
                                                           int x_dtype, int M, float* y,
                                                           void* hip_stream) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!layer_name || !x || !y || M <= 0)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid arguments");
    size_t idx;
    if (!resolve(e, layer_name, &idx))
        return fail(CORTEX_ERROR_INFERENCE,
                    std::string("matmulHSDR: segment not found: ") + layer_name);
    csdr_segment_info info;
    csdr_archive_info(e->ar, idx, &info);
    if (info.strategy_id != 5)
        return fail(CORTEX_ERROR_UNSUPPORTED_FORMAT,
                    std::string("matmulHSDR: segment '") + layer_name +
                        "' is not HSDR-encoded (strategy_id=" + std::to_string(info.strategy_id) +
                        ")");
    Cached* c = nullptr;
    CortexError r = load(e, idx, &c);
    if (r.code) return r;
    (void)hipStreamSynchronize(e->st);  // the segment upload ran on the engine stream
    int rc = grow(&e->ws, &e->ws_bytes, csdr_hsdb_workspace_bytes(c->seg, M));
    if (rc) return from_csdr(rc, "workspace");
    rc = csdr_hsdb_matmul(c->seg, x, x_dtype, M, y, e->ws, e->ws_bytes, hip_stream);
    if (rc) return from_csdr(rc, std::string("matmulHSDR '") + layer_name + "'");
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_matmul_device")
}

CSDR_API CortexError cortex_inference_engine_set_lazy_hsdr_selection(CortexInferenceEngineHandle e,
                                                                     int mode) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (mode < 0 || mode > 2)
        return fail(CORTEX_ERROR_INVALID_ARGUMENT, "lazy HSDR selection mode must be 0, 1 or 2");
    e->lazy_mode = mode;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_set_lazy_hsdr_selection")
}

CSDR_API CortexError cortex_inference_engine_generate_text(CortexInferenceEngineHandle e,
                                                           const char* prompt, int max_new_tokens,
                                                           char** out_text) {
    CORTEX_GUARD_BEGIN
    CHECK_HANDLE(e);
    if (!prompt || !out_text) return fail(CORTEX_ERROR_INVALID_ARGUMENT, "Invalid argument(s)");
    *out_text = nullptr;
    std::vector<int32_t> ids;
    const char* p = prompt;
    while (*p) {
        while (*p && std::isspace((unsigned char)*p)) ++p;
        if (!*p) break;
        char* end = nullptr;
        const long v = std::strtol(p, &end, 10);
        if (end == p || v < 0 || v > INT32_MAX || (*end && !std::isspace((unsigned char)*end)))
            return fail(CORTEX_ERROR_INVALID_ARGUMENT,
                        "prompt must be whitespace-separated token ids (no tokenizer on this path)");
        ids.push_back((int32_t)v);
        p = end;
    }
    if (ids.empty())
        return fail(CORTEX_ERROR_INFERENCE, "Prompt tokenization produced no tokens");
    const int steps = std::max(1, max_new_tokens);
    const int ctx = (int)((ids.size() + steps + 255) / 256 * 256);
    const auto t0 = std::chrono::steady_clock::now();
    if (!e->dec || e->dec_ctx < (int)ids.size() + steps) {
        CortexError r = build_decoder(e, ctx);
        if (r.code) return r;
    }
    {
        CortexError r = apply_lazy(e);
        if (r.code) return r;
    }
    const auto t1 = std::chrono::steady_clock::now();
    // generate_text's sampling: temperature 0.8, repeat penalty 1.5 on generated tokens (the
    // lazy HSDR choice applies its own penalty of 1.0)
    const float temperature = 0.8f, penalty = 1.5f;
    int rc = csdr_decoder_prefill(e->dec, ids.data(), (int)ids.size(), temperature, penalty);
    if (rc) return from_csdr(rc, "prefill");
    const auto t2 = std::chrono::steady_clock::now();
    rc = csdr_decoder_decode(e->dec, steps - 1, temperature, penalty);
    if (rc) return from_csdr(rc, "decode");
    const auto t3 = std::chrono::steady_clock::now();
    std::vector<int32_t> out(steps);
    rc = csdr_decoder_tokens(e->dec, (int)ids.size(), steps, out.data());
    if (rc) return from_csdr(rc, "tokens");
    std::string text;
    for (int i = 0; i < steps; ++i) {
        if (out[i] < 0)
            return fail(CORTEX_ERROR_INFERENCE, "Failed to sample next token (no finite score)");
        if (i) text += ' ';
        text += std::to_string(out[i]);
    }
    *out_text = dup_c(text);
    const double build_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    const double pre_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    const double dec_ms = std::chrono::duration<double, std::milli>(t3 - t2).count();
    char buf[512];
    std::snprintf(buf, sizeof buf,
                  "{\"prompt_tokens\":%zu,\"generated_tokens\":%d,\"setup_ms\":%.3f,"
                  "\"prefill_ms\":%.3f,\"decode_ms\":%.3f,\"tokens_per_sec\":%.2f,"
                  "\"cached_bytes\":%zu}",
                  ids.size(), steps, build_ms, pre_ms, dec_ms,
                  steps > 1 ? (steps - 1) / (dec_ms * 1e-3) : 0.0, e->cache_bytes);
    e->stats = buf;
    return ok();
    CORTEX_GUARD_END("cortex_inference_engine_generate_text")
}

}  // extern "C"
