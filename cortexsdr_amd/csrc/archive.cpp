// archive.cpp — host readers for the containers that carry coded weights to the device:
// the .sdr archive index and payloads, HSDR codes-only streams with an external dictionary
// (HSDC), and the shared-dictionary archive (HSDA).
//
// Reference formats (cortexSDR tree):
//   .sdr   AIDecompressor::readArchiveIndex (core/AIDecompressor.cpp:78-262), payload reads
//          readCompressedBytes (:418-435), writer AICompressor.cpp:233-309, magic/version
//          ArchiveConstants.cpp:10-11. Little-endian, strings = u32 length + bytes,
//          bool = 1 byte.
//   HSDC   HSDRCodesHeader (strategies/HierarchicalSDRStrategy.cpp:675-691) + u16 codes;
//          parseCodesStream's geometry checks against the dictionary config (:1766-1801).
//   HSDA   SharedDictArchive::readFromStream (:1937-2081): per dictionary the raw
//          HierarchicalSDRConfig (20 bytes: u16 tile_rows, tile_cols, n_atoms; u8 n_stages,
//          k, ksvd_iters, pad; 2 padding bytes; f32 stage_decay; u32 max_tiles_for_fit),
//          stage scales and atoms; per segment name, dict index, sizes and an HSDC stream.
//
// The reference re-opens the .sdr file for every payload read; here the archive keeps one
// open file and the device segments built from it are cached by the engine (engine.cpp).
// A codes-only stream plus its dictionary is turned into the equivalent HSDR v2 stream
// (stage scales from the dictionary, zero edge strips where the shape is not a multiple of
// the tile, as reassembleTiles leaves them) and loaded through csdr_hsdb_load.
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cortexsdr_hip.h"
#include "common.hpp"

using csdr::set_error;

namespace {

struct Entry {
    std::string name, data_format, layer_type, layer_name;
    uint8_t type = 0, strategy = 0;
    uint64_t orig = 0, comp = 0, offset = 0;
    uint32_t layer_index = 0;
    bool has_meta = false, sorted = false, has_scale = false, has_zp = false;
    std::vector<uint32_t> dims, in_shape, out_shape;
    float sparsity = 0.f, scale = 0.f, zp = 0.f;
};

// Bounds-checked little-endian reader over a byte range.
struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if (!ok || (size_t)(end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint32_t n = get<uint32_t>();
        if (!ok || (size_t)(end - p) < n) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char*>(p), n);
        p += n;
        return s;
    }
    bool bytes(void* dst, size_t n) {
        if (!ok || (size_t)(end - p) < n) return ok = false;
        std::memcpy(dst, p, n);
        p += n;
        return true;
    }
};

int read_file(const char* path, std::vector<uint8_t>& out) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return set_error(CSDR_E_INVALID, std::string("cannot open ") + path);
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    if (n < 0) {
        std::fclose(f);
        return set_error(CSDR_E_INVALID, std::string("cannot size ") + path);
    }
    out.resize((size_t)n);
    const size_t got = n ? std::fread(out.data(), 1, (size_t)n, f) : 0;
    std::fclose(f);
    if (got != (size_t)n) return set_error(CSDR_E_TRUNCATED, std::string("short read of ") + path);
    return CSDR_OK;
}

struct Dict {
    uint16_t tile_rows = 0, tile_cols = 0, n_atoms = 0;
    uint8_t n_stages = 0, k = 0;
    float stage_decay = 0.f;
    std::vector<float> scales, atoms;
};

// HSDC stream + dictionary -> equivalent HSDR v2 stream (see file comment).
int codes_to_hsdr(const uint8_t* buf, size_t n, const Dict& d, std::vector<uint8_t>& out) {
    Cursor c{buf, buf + n};
    char magic[4];
    c.bytes(magic, 4);
    const uint32_t version = c.get<uint32_t>();
    const uint32_t R = c.get<uint32_t>(), C = c.get<uint32_t>(), n_tiles = c.get<uint32_t>();
    const uint16_t tr = c.get<uint16_t>(), tc = c.get<uint16_t>(), K = c.get<uint16_t>();
    const uint8_t S = c.get<uint8_t>(), k = c.get<uint8_t>();
    const float decay = c.get<float>();
    if (!c.ok) return set_error(CSDR_E_TRUNCATED, "HSDC: stream shorter than its header");
    if (std::memcmp(magic, "HSDC", 4) != 0)
        return set_error(CSDR_E_FORMAT, "HSDR shared: bad codes-stream magic");
    if (version != 1) return set_error(CSDR_E_FORMAT, "HSDR shared: unsupported codes-stream version");
    if (tr != d.tile_rows || tc != d.tile_cols || K != d.n_atoms || S != d.n_stages || k != d.k)
        return set_error(CSDR_E_FORMAT,
                         "HSDR shared: stream geometry doesn't match dictionary config");
    if (tr == 0 || tc == 0) return set_error(CSDR_E_FORMAT, "HSDC: zero tile geometry");
    const size_t slots = (size_t)S * k;
    const size_t n_codes = (size_t)n_tiles * slots;
    if ((size_t)(c.end - c.p) < 2 * n_codes)
        return set_error(CSDR_E_TRUNCATED, "HSDR decompress: truncated stream");
    const size_t tile_dim = (size_t)tr * tc;
    if (d.atoms.size() != (size_t)K * tile_dim)
        return set_error(CSDR_E_FORMAT, "HSDC: dictionary has " + std::to_string(d.atoms.size()) +
                                            " atom floats, expected " +
                                            std::to_string((size_t)K * tile_dim));
    if (d.scales.size() < S) return set_error(CSDR_E_FORMAT, "HSDC: dictionary lacks stage scales");
    const uint32_t R_full = R / tr * tr, C_full = C / tc * tc;
    // the header's shape must describe exactly n_tiles tiles, and the zero edge strips the
    // equivalent stream carries must fit its u32 byte count (a corrupt R or C would otherwise
    // size an allocation from unchecked fields)
    if ((uint64_t)(R / tr) * (C / tc) != n_tiles)
        return set_error(CSDR_E_FORMAT, "HSDC: tile count does not match the stream's shape");
    const uint64_t edge_floats = (uint64_t)R_full * (C - C_full) + (uint64_t)(R - R_full) * C;
    if (edge_floats * 4 > 0xFFFFFFFFull || edge_floats > (uint64_t)R * C)
        return set_error(CSDR_E_FORMAT, "HSDC: edge strips exceed the stream format's limits");
    out.clear();
    out.reserve(36 + 4 * S + 4 * d.atoms.size() + 2 * n_codes + 4 * edge_floats);
    auto put = [&](const void* p, size_t b) {
        const uint8_t* q = static_cast<const uint8_t*>(p);
        out.insert(out.end(), q, q + b);
    };
    const uint32_t ver2 = 2, eb = (uint32_t)(edge_floats * 4);
    put("HSDR", 4);
    put(&ver2, 4);
    put(&R, 4);
    put(&C, 4);
    put(&n_tiles, 4);
    put(&tr, 2);
    put(&tc, 2);
    put(&K, 2);
    put(&S, 1);
    put(&k, 1);
    put(&decay, 4);
    put(&eb, 4);
    put(d.scales.data(), 4 * (size_t)S);
    put(d.atoms.data(), 4 * d.atoms.size());
    put(c.p, 2 * n_codes);
    out.resize(out.size() + 4 * edge_floats, 0);
    return CSDR_OK;
}

// Exceptions (allocation failures of a large but well-formed stream) stay inside: the caller
// gets a status, as from every entry point of this library.
int load_codes(const uint8_t* buf, size_t n, const Dict& d, void* hip_stream, csdr_hsdb** out) {
    try {
        std::vector<uint8_t> hsdr;
        int rc = codes_to_hsdr(buf, n, d, hsdr);
        if (rc) return rc;
        return csdr_hsdb_load(hsdr.data(), hsdr.size(), hip_stream, out);
    } catch (const std::exception& ex) {
        return set_error(CSDR_E_FORMAT, std::string("HSDC: cannot build the segment: ") + ex.what());
    }
}

}  // namespace

struct csdr_archive {
    std::string path;
    FILE* f = nullptr;
    uint32_t version = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> by_name;
    ~csdr_archive() {
        if (f) std::fclose(f);
    }
};

struct csdr_hsda {
    std::vector<Dict> dicts;
    struct Seg {
        std::string name;
        uint32_t dict = 0;
        uint64_t orig = 0;
        uint8_t type = 0;
        std::vector<uint8_t> codes;
    };
    std::vector<Seg> segs;
    std::unordered_map<std::string, size_t> by_name;
};

namespace {

int parse_index(csdr_archive* a) {
    FILE* f = a->f;
    uint8_t head[28];
    if (std::fread(head, 1, sizeof head, f) != sizeof head)
        return set_error(CSDR_E_FORMAT, "Invalid or missing archive magic number.");
    if (std::memcmp(head, "CORTEXSR", 8) != 0)
        return set_error(CSDR_E_FORMAT, "Invalid or missing archive magic number.");
    uint64_t nseg = 0, index_off = 0;
    std::memcpy(&a->version, head + 8, 4);
    std::memcpy(&nseg, head + 12, 8);
    std::memcpy(&index_off, head + 20, 8);
    if (a->version == 0 || a->version > 2)
        return set_error(CSDR_E_FORMAT, "Unsupported archive version.");
    std::fseek(f, 0, SEEK_END);
    const long fsize = std::ftell(f);
    if (fsize < 0 || index_off > (uint64_t)fsize)
        return set_error(CSDR_E_TRUNCATED, "archive index offset beyond the end of the file");
    std::vector<uint8_t> idx((size_t)((uint64_t)fsize - index_off));
    std::fseek(f, (long)index_off, SEEK_SET);
    if (!idx.empty() && std::fread(idx.data(), 1, idx.size(), f) != idx.size())
        return set_error(CSDR_E_TRUNCATED, "short read of the archive index");
    Cursor c{idx.data(), idx.data() + idx.size()};
    // every entry takes at least 50 bytes: bounds the reservation for a corrupt count
    if (nseg > idx.size() / 50 + 1)
        return set_error(CSDR_E_FORMAT, "Failed to read segment count.");
    a->entries.reserve((size_t)nseg);
    for (uint64_t i = 0; i < nseg; ++i) {
        Entry e;
        e.name = c.str();
        if (a->version >= 2) e.data_format = c.str();
        e.layer_type = c.str();
        e.type = c.get<uint8_t>();
        e.strategy = c.get<uint8_t>();
        e.orig = c.get<uint64_t>();
        e.comp = c.get<uint64_t>();
        e.offset = c.get<uint64_t>();
        e.layer_name = c.str();
        e.layer_index = c.get<uint32_t>();
        e.has_meta = c.get<uint8_t>() != 0;
        if (e.has_meta) {
            const uint8_t nd = c.get<uint8_t>();
            for (uint8_t d = 0; d < nd && c.ok; ++d) e.dims.push_back(c.get<uint32_t>());
            e.sparsity = c.get<float>();
            e.sorted = c.get<uint8_t>() != 0;
            e.has_scale = c.get<uint8_t>() != 0;
            if (e.has_scale) e.scale = c.get<float>();
            e.has_zp = c.get<uint8_t>() != 0;
            if (e.has_zp) e.zp = c.get<float>();
        }
        if (c.get<uint8_t>()) {
            const uint8_t nd = c.get<uint8_t>();
            for (uint8_t d = 0; d < nd && c.ok; ++d) e.in_shape.push_back(c.get<uint32_t>());
        }
        if (c.get<uint8_t>()) {
            const uint8_t nd = c.get<uint8_t>();
            for (uint8_t d = 0; d < nd && c.ok; ++d) e.out_shape.push_back(c.get<uint32_t>());
        }
        if (!c.ok)
            return set_error(CSDR_E_TRUNCATED, "Failed to read segment header information from "
                                               "index (entry " + std::to_string(i) + ").");
        if (e.comp > index_off || e.offset > index_off - e.comp)
            return set_error(CSDR_E_FORMAT, "segment '" + e.name + "' payload overlaps the index");
        a->by_name.emplace(e.name, a->entries.size());  // first entry of a name wins
        a->entries.push_back(std::move(e));
    }
    return CSDR_OK;
}

void fill_info(const Entry& e, csdr_segment_info* info) {
    std::memset(info, 0, sizeof *info);
    info->name = e.name.c_str();
    info->data_format = e.data_format.c_str();
    info->layer_type = e.layer_type.c_str();
    info->layer_name = e.layer_name.c_str();
    info->original_type = e.type;
    info->strategy_id = e.strategy;
    info->original_size = e.orig;
    info->compressed_size = e.comp;
    info->data_offset = e.offset;
    info->layer_index = e.layer_index;
    info->has_metadata = e.has_meta;
    info->n_dims = (uint32_t)std::min<size_t>(e.dims.size(), 8);
    for (uint32_t i = 0; i < info->n_dims; ++i) info->dims[i] = e.dims[i];
    info->sparsity_ratio = e.sparsity;
    info->n_input_dims = (uint32_t)std::min<size_t>(e.in_shape.size(), 8);
    for (uint32_t i = 0; i < info->n_input_dims; ++i) info->input_shape[i] = e.in_shape[i];
    info->n_output_dims = (uint32_t)std::min<size_t>(e.out_shape.size(), 8);
    for (uint32_t i = 0; i < info->n_output_dims; ++i) info->output_shape[i] = e.out_shape[i];
}

int parse_hsda(const uint8_t* buf, size_t n, csdr_hsda* h) {
    Cursor c{buf, buf + n};
    char magic[4];
    if (!c.bytes(magic, 4) || std::memcmp(magic, "HSDA", 4) != 0)
        return set_error(CSDR_E_FORMAT, "HSDA read: bad magic - not an HSDA stream");
    const uint32_t version = c.get<uint32_t>();
    if (c.ok && version != 1) return set_error(CSDR_E_FORMAT, "HSDA read: unsupported version");
    const uint32_t nd = c.get<uint32_t>(), ns = c.get<uint32_t>();
    if (!c.ok) return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated stream");
    if ((uint64_t)nd * 28 > n || (uint64_t)ns * 21 > n)
        return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated stream");
    h->dicts.resize(nd);
    for (auto& d : h->dicts) {
        uint8_t cfg[20];
        if (!c.bytes(cfg, 20)) break;
        std::memcpy(&d.tile_rows, cfg + 0, 2);
        std::memcpy(&d.tile_cols, cfg + 2, 2);
        std::memcpy(&d.n_atoms, cfg + 4, 2);
        d.n_stages = cfg[6];
        d.k = cfg[7];
        std::memcpy(&d.stage_decay, cfg + 12, 4);
        const uint32_t nsc = c.get<uint32_t>();
        if (!c.ok || (size_t)(c.end - c.p) / 4 < nsc) return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated array");
        d.scales.resize(nsc);
        c.bytes(d.scales.data(), 4 * (size_t)nsc);
        const uint32_t na = c.get<uint32_t>();
        if (!c.ok || (size_t)(c.end - c.p) / 4 < na) return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated array");
        d.atoms.resize(na);
        c.bytes(d.atoms.data(), 4 * (size_t)na);
    }
    if (!c.ok) return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated stream");
    h->segs.resize(ns);
    for (size_t i = 0; i < ns; ++i) {
        auto& s = h->segs[i];
        s.name = c.str();
        s.dict = c.get<uint32_t>();
        s.orig = c.get<uint64_t>();
        s.type = c.get<uint8_t>();
        const uint32_t cl = c.get<uint32_t>();
        if (!c.ok || (size_t)(c.end - c.p) < cl)
            return set_error(CSDR_E_TRUNCATED, "HSDA read: truncated array");
        s.codes.assign(c.p, c.p + cl);
        c.p += cl;
        if (s.dict >= nd) return set_error(CSDR_E_FORMAT, "HSDA read: dict_index out of range");
        h->by_name[s.name] = i;
    }
    return CSDR_OK;
}

}  // namespace

extern "C" {

CSDR_API int csdr_archive_open(const char* path, csdr_archive** out) {
    if (!path || !out) return set_error(CSDR_E_INVALID, "archive_open: null argument");
    *out = nullptr;
    auto a = std::unique_ptr<csdr_archive>(new (std::nothrow) csdr_archive());
    if (!a) return set_error(CSDR_E_INVALID, "archive_open: out of host memory");
    a->path = path;
    a->f = std::fopen(path, "rb");
    if (!a->f)
        return set_error(CSDR_E_INVALID, std::string("Failed to open archive: ") + path);
    int rc;
    try {
        rc = parse_index(a.get());
    } catch (const std::bad_alloc&) {
        rc = set_error(CSDR_E_FORMAT, "archive_open: index too large");
    }
    if (rc) return rc;
    *out = a.release();
    return CSDR_OK;
}

CSDR_API int csdr_archive_close(csdr_archive* a) {
    delete a;
    return CSDR_OK;
}

CSDR_API size_t csdr_archive_count(const csdr_archive* a) { return a ? a->entries.size() : 0; }

CSDR_API int csdr_archive_info(const csdr_archive* a, size_t i, csdr_segment_info* info) {
    if (!a || !info || i >= a->entries.size())
        return set_error(CSDR_E_INVALID, "archive_info: bad argument");
    fill_info(a->entries[i], info);
    return CSDR_OK;
}

CSDR_API int csdr_archive_find(const csdr_archive* a, const char* name, size_t* index) {
    if (!a || !name || !index) return set_error(CSDR_E_INVALID, "archive_find: bad argument");
    auto it = a->by_name.find(name);
    if (it == a->by_name.end())
        return set_error(CSDR_E_INVALID, std::string("Segment not found: ") + name);
    *index = it->second;
    return CSDR_OK;
}

CSDR_API int csdr_archive_read(const csdr_archive* a, size_t i, void* buf, size_t cap,
                               size_t* n) {
    if (!a || i >= a->entries.size()) return set_error(CSDR_E_INVALID, "archive_read: bad argument");
    const Entry& e = a->entries[i];
    if (n) *n = e.comp;
    if (!buf) return CSDR_OK;  // size query
    if (cap < e.comp)
        return set_error(CSDR_E_INVALID, "archive_read: buffer holds " + std::to_string(cap) +
                                             " bytes, segment '" + e.name + "' has " +
                                             std::to_string(e.comp));
    if (std::fseek(a->f, (long)e.offset, SEEK_SET) != 0 ||
        std::fread(buf, 1, (size_t)e.comp, a->f) != e.comp)
        return set_error(CSDR_E_TRUNCATED,
                         "Failed to read compressed data for segment: " + e.name);
    return CSDR_OK;
}

CSDR_API int csdr_hsdb_load_codes(const void* codes, size_t nbytes, const csdr_dictionary* dict,
                                  void* hip_stream, csdr_hsdb** out) {
    if (!codes || !dict || !out || !dict->atoms || !dict->stage_scales)
        return set_error(CSDR_E_INVALID, "hsdb_load_codes: null argument");
    if (dict->n_atom_floats > ((size_t)1 << 34) || dict->n_stage_scales > 255)
        return set_error(CSDR_E_INVALID, "hsdb_load_codes: dictionary sizes out of range");
    Dict d;
    d.tile_rows = (uint16_t)dict->tile_rows;
    d.tile_cols = (uint16_t)dict->tile_cols;
    d.n_atoms = (uint16_t)dict->n_atoms;
    d.n_stages = (uint8_t)dict->n_stages;
    d.k = (uint8_t)dict->k_per_stage;
    d.stage_decay = dict->stage_decay;
    try {
        d.scales.assign(dict->stage_scales, dict->stage_scales + dict->n_stage_scales);
        d.atoms.assign(dict->atoms, dict->atoms + dict->n_atom_floats);
    } catch (const std::bad_alloc&) {
        return set_error(CSDR_E_INVALID, "hsdb_load_codes: out of host memory");
    }
    return load_codes(static_cast<const uint8_t*>(codes), nbytes, d, hip_stream, out);
}

CSDR_API int csdr_hsda_open(const char* path, csdr_hsda** out) {
    if (!path || !out) return set_error(CSDR_E_INVALID, "hsda_open: null argument");
    std::vector<uint8_t> buf;
    int rc = read_file(path, buf);
    if (rc) return rc;
    return csdr_hsda_open_memory(buf.data(), buf.size(), out);
}

CSDR_API int csdr_hsda_open_memory(const void* data, size_t nbytes, csdr_hsda** out) {
    if (!data || !out) return set_error(CSDR_E_INVALID, "hsda_open: null argument");
    *out = nullptr;
    auto h = std::unique_ptr<csdr_hsda>(new (std::nothrow) csdr_hsda());
    if (!h) return set_error(CSDR_E_INVALID, "hsda_open: out of host memory");
    int rc;
    try {
        rc = parse_hsda(static_cast<const uint8_t*>(data), nbytes, h.get());
    } catch (const std::bad_alloc&) {
        rc = set_error(CSDR_E_TRUNCATED, "HSDA read: truncated stream");
    }
    if (rc) return rc;
    *out = h.release();
    return CSDR_OK;
}

CSDR_API int csdr_hsda_close(csdr_hsda* h) {
    delete h;
    return CSDR_OK;
}

CSDR_API size_t csdr_hsda_count(const csdr_hsda* h) { return h ? h->segs.size() : 0; }
CSDR_API size_t csdr_hsda_dictionary_count(const csdr_hsda* h) { return h ? h->dicts.size() : 0; }

CSDR_API int csdr_hsda_segment(const csdr_hsda* h, size_t i, const char** name,
                               uint32_t* dict_index, uint64_t* original_size) {
    if (!h || i >= h->segs.size()) return set_error(CSDR_E_INVALID, "hsda_segment: bad argument");
    if (name) *name = h->segs[i].name.c_str();
    if (dict_index) *dict_index = h->segs[i].dict;
    if (original_size) *original_size = h->segs[i].orig;
    return CSDR_OK;
}

CSDR_API int csdr_hsda_load(const csdr_hsda* h, const char* name, void* hip_stream,
                            csdr_hsdb** out) {
    if (!h || !name || !out) return set_error(CSDR_E_INVALID, "hsda_load: null argument");
    auto it = h->by_name.find(name);
    if (it == h->by_name.end())
        return set_error(CSDR_E_INVALID,
                         std::string("HSDAReader::matmul: segment not found: ") + name);
    const auto& s = h->segs[it->second];
    return load_codes(s.codes.data(), s.codes.size(), h->dicts[s.dict], hip_stream, out);
}

}  // extern "C"
