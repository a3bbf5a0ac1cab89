// ref_shim.cpp — C-ABI driver over the cortexSDR reference sources, compiled from where
// they lie under the reference tree by oracle/Makefile into oracle/_ref/libcsdr_ref.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ (and tests/golden/make_fixtures.py) to check the
// oracle restatement against the reference's own code. No reference source is copied here;
// this file only calls the reference's public entry points:
//   HierarchicalSDRStrategy::{compress, decompress, matmulRowMajor, dequantizeToFP32}
//     (strategies/HierarchicalSDRStrategy.hpp:170-181, :333)
//   HierarchicalSDRStrategy::compressGroupedSegments + SharedDictArchive::writeToStream
//     and HSDAReader::{matmul, decompress} (HierarchicalSDRStrategy.hpp:289-346, 368-405)
//   Kernels::multi_head_attention (kernels/attention_kernels.hpp:26)
//   Kernels::flash_attention_forward (kernels/flash_attention.hpp:43)
#include "strategies/HierarchicalSDRStrategy.hpp"
#include "kernels/attention_kernels.hpp"
#include "kernels/flash_attention.hpp"

#include <cstdlib>
#include <cstring>
#include <sstream>
#include <exception>
#include <string>
#include <vector>

using namespace CortexAICompression;

namespace {
thread_local std::string g_err;

int fail(const std::exception& e, int code) {
    g_err = e.what();
    return code;
}

std::vector<std::byte> as_bytes(const void* p, size_t n) {
    std::vector<std::byte> v(n);
    if (n) std::memcpy(v.data(), p, n);
    return v;
}
}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

void ref_free(void* p) { std::free(p); }

// Compress an R x C fp32 matrix with the reference V4b fit. The same config is installed
// for the attention and MLP roles, so configFor() picks it regardless of the name (it still
// widens tile_cols to C when tile_rows == 1, HierarchicalSDRStrategy.cpp:1024-1046).
int ref_hsdr_compress(const float* w, uint32_t R, uint32_t C, uint16_t tile_rows,
                      uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages, uint8_t k_per_stage,
                      uint8_t ksvd_iters, float stage_decay, uint8_t** out, size_t* out_n) {
    try {
        HierarchicalSDRConfig cfg;
        cfg.tile_rows = tile_rows;
        cfg.tile_cols = tile_cols;
        cfg.n_atoms = n_atoms;
        cfg.n_stages = n_stages;
        cfg.active_bits_per_stage = k_per_stage;
        cfg.ksvd_iters = ksvd_iters;
        cfg.stage_decay = stage_decay;
        HierarchicalSDRStrategy strat(cfg, cfg);
        ModelSegment seg(SegmentType::WEIGHTS_FP32, "ref.weight",
                         as_bytes(w, sizeof(float) * size_t(R) * C));
        TensorMetadata meta;
        meta.dimensions = {R, C};
        seg.tensor_metadata = meta;
        seg.data_format = "f32";
        std::vector<std::byte> bytes = strat.compress(seg);
        *out_n = bytes.size();
        *out = static_cast<uint8_t*>(std::malloc(bytes.size() ? bytes.size() : 1));
        std::memcpy(*out, bytes.data(), bytes.size());
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

int ref_hsdr_decompress(const uint8_t* stream, size_t n, float* out, size_t out_floats) {
    try {
        HierarchicalSDRStrategy strat;
        std::vector<std::byte> bytes =
            strat.decompress(as_bytes(stream, n), SegmentType::WEIGHTS_FP32, out_floats * 4);
        std::memcpy(out, bytes.data(), bytes.size());
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

int ref_hsdr_matmul_row_major(const uint8_t* stream, size_t n, const float* x, size_t batch,
                              float* y, size_t y_floats) {
    try {
        HierarchicalSDRStrategy strat;
        std::vector<float> Y = strat.matmulRowMajor(as_bytes(stream, n), x, batch);
        if (Y.size() > y_floats) return -2;
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

// dequantizeToFP32 on a one-segment byte stream tagged with `fmt` ("q4_k", "q5_k", ...).
int ref_dequant(const uint8_t* data, size_t n, const char* fmt, uint32_t R, uint32_t C,
                float* out, size_t out_floats) {
    try {
        ModelSegment seg(SegmentType::WEIGHTS_INT8, "ref.kquant", as_bytes(data, n));
        seg.data_format = fmt;
        TensorMetadata meta;
        meta.dimensions = {R, C};
        seg.tensor_metadata = meta;
        std::vector<float> v = HierarchicalSDRStrategy::dequantizeToFP32(seg);
        if (v.size() > out_floats) return -2;
        std::memcpy(out, v.data(), v.size() * sizeof(float));
        return static_cast<int>(v.size());
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

// n row-major fp32 matrices (R_i x C, names[i]) -> HSDA bytes through the reference's
// shared-dictionary pipeline with 1-row tiles (one dictionary for the group).
int ref_hsda_build(uint32_t n, const char* const* names, const float* const* ws,
                   const uint32_t* rows, uint32_t C, uint16_t n_atoms, uint8_t n_stages,
                   uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay, uint8_t** out,
                   size_t* out_n) {
    try {
        HierarchicalSDRConfig cfg;
        cfg.tile_rows = 1;
        cfg.tile_cols = static_cast<uint16_t>(C);
        cfg.n_atoms = n_atoms;
        cfg.n_stages = n_stages;
        cfg.active_bits_per_stage = k_per_stage;
        cfg.ksvd_iters = ksvd_iters;
        cfg.stage_decay = stage_decay;
        HierarchicalSDRStrategy strat(cfg, cfg);
        std::vector<ModelSegment> segs;
        for (uint32_t i = 0; i < n; ++i) {
            ModelSegment seg(SegmentType::WEIGHTS_FP32, names[i],
                             as_bytes(ws[i], sizeof(float) * size_t(rows[i]) * C));
            TensorMetadata meta;
            meta.dimensions = {rows[i], C};
            seg.tensor_metadata = meta;
            seg.data_format = "f32";
            segs.push_back(std::move(seg));
        }
        std::vector<std::string> skipped;
        auto archive = strat.compressGroupedSegments(segs, &skipped);
        if (!skipped.empty()) {
            g_err = "segment skipped by the reference pipeline: " + skipped[0];
            return -3;
        }
        std::ostringstream os;
        archive.writeToStream(os);
        const std::string b = os.str();
        *out_n = b.size();
        *out = static_cast<uint8_t*>(std::malloc(b.size() ? b.size() : 1));
        std::memcpy(*out, b.data(), b.size());
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

// compressGroupedSegments with per-segment widths, a tile geometry and the fit-pool cap:
// skipped[i] = 1 for the segments the pipeline skipped (out_skipped_names).
int ref_hsda_build_ex(uint32_t n, const char* const* names, const float* const* ws,
                      const uint32_t* rows, const uint32_t* cols, uint16_t tile_rows,
                      uint16_t tile_cols, uint16_t n_atoms, uint8_t n_stages,
                      uint8_t k_per_stage, uint8_t ksvd_iters, float stage_decay,
                      uint32_t max_tiles_for_fit, uint8_t* skipped, uint8_t** out,
                      size_t* out_n) {
    try {
        HierarchicalSDRConfig cfg;
        cfg.tile_rows = tile_rows;
        cfg.tile_cols = tile_cols;
        cfg.n_atoms = n_atoms;
        cfg.n_stages = n_stages;
        cfg.active_bits_per_stage = k_per_stage;
        cfg.ksvd_iters = ksvd_iters;
        cfg.stage_decay = stage_decay;
        cfg.max_tiles_for_fit = max_tiles_for_fit;
        HierarchicalSDRStrategy strat(cfg, cfg);
        std::vector<ModelSegment> segs;
        for (uint32_t i = 0; i < n; ++i) {
            ModelSegment seg(SegmentType::WEIGHTS_FP32, names[i],
                             as_bytes(ws[i], sizeof(float) * size_t(rows[i]) * cols[i]));
            TensorMetadata meta;
            meta.dimensions = {rows[i], cols[i]};
            seg.tensor_metadata = meta;
            seg.data_format = "f32";
            segs.push_back(std::move(seg));
        }
        std::vector<std::string> sk;
        auto archive = strat.compressGroupedSegments(segs, &sk);
        for (uint32_t i = 0; i < n; ++i) {
            skipped[i] = 0;
            for (const auto& nm : sk)
                if (nm == names[i]) skipped[i] = 1;
        }
        std::ostringstream os;
        archive.writeToStream(os);
        const std::string b = os.str();
        *out_n = b.size();
        *out = static_cast<uint8_t*>(std::malloc(b.size() ? b.size() : 1));
        std::memcpy(*out, b.data(), b.size());
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

int ref_hsda_matmul(const uint8_t* data, size_t n, const char* name, const float* x,
                    size_t batch, float* y, size_t y_floats) {
    try {
        std::istringstream is(std::string(reinterpret_cast<const char*>(data), n));
        HSDAReader reader(HierarchicalSDRStrategy::SharedDictArchive::readFromStream(is));
        std::vector<float> Y = reader.matmul(name, x, batch);
        if (Y.size() > y_floats) return -2;
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

int ref_hsda_decompress(const uint8_t* data, size_t n, const char* name, float* w,
                        size_t w_floats) {
    try {
        std::istringstream is(std::string(reinterpret_cast<const char*>(data), n));
        HSDAReader reader(HierarchicalSDRStrategy::SharedDictArchive::readFromStream(is));
        std::vector<std::byte> b = reader.decompress(name);
        if (b.size() > w_floats * 4) return -2;
        std::memcpy(w, b.data(), b.size());
        return 0;
    } catch (const std::exception& e) {
        return fail(e, -1);
    }
}

void ref_mha(const float* q, const float* k, const float* v, float* out, size_t B, size_t T,
             size_t hidden, size_t heads, int causal) {
    Kernels::multi_head_attention(q, k, v, out, B, T, hidden, heads, causal != 0);
}

void ref_flash_attention(const float* q, const float* k, const float* v, float* out, size_t B,
                         size_t T, size_t hidden, size_t heads, int causal) {
    Kernels::FlashAttentionConfig cfg;
    cfg.use_causal_mask = causal != 0;
    Kernels::flash_attention_forward(q, k, v, out, B, T, hidden, heads, cfg);
}

}  // extern "C"
