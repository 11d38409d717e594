// XorSparse container ("XORSPARE1") reader / writer and the HF-checkpoint
// converter, host side (include/xtern.h).
//
// Layout (SPARSE_FORMAT.md:30-50, as SparseFile::serialize writes it,
// src/loader/sparse_loader.rs:124-139), little-endian:
//   bytes 0..9   magic "XORSPARE1"
//   bytes 9..13  version u32 = 1
//   bytes 13..17 num_tensors u32
//   then per tensor: name_len u32, name, out_dim u32, in_dim u32,
//                    w_scale f32, blob_len u32, blob (XorSparse row blobs).
// The reference's reader (sparse_loader.rs:48-55) takes the version from
// bytes 8..12 and the directory from byte 16, one byte early, so it rejects
// every file its own writer produces; this reader follows the writer.
#include <stdint.h>
#include <string.h>

#include <map>
#include <new>
#include <string>
#include <vector>

#include "../../include/xtern.h"
#include "xtern_layout.h"

namespace {

const char kMagic[9] = {'X', 'O', 'R', 'S', 'P', 'A', 'R', 'E', '1'};
constexpr uint32_t kVersion = 1;

inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
inline void wr32(uint8_t* p, uint32_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
    p[2] = (uint8_t)(v >> 16);
    p[3] = (uint8_t)(v >> 24);
}

struct Entry {
    std::string name;
    uint32_t out_dim, in_dim;
    float w_scale;
    size_t blob_off, blob_len;
};

// Ternary value of (row o, column i) of HF striped bytes [N/f][K]: digit j of
// byte [p][i] with o = j*R + p (destripe), or -- the reference converter's
// reading (convert_sparse.rs:104) -- value k = o*K + i of the linear unpack,
// digit k % f of byte k / f.
inline int hf_value(const uint8_t* stored, int fmt, int64_t K, int64_t N, int64_t o, int64_t i,
                    bool destripe) {
    const int64_t f = fmt == XT_PACK5 ? 5 : 4;
    int64_t byte, j;
    if (destripe) {
        const int64_t R = N / f;
        j = o / R;
        byte = (o % R) * K + i;
    } else {
        const int64_t k = o * K + i;
        byte = k / f;
        j = k % f;
    }
    const unsigned x = stored[byte];
    if (fmt == XT_PACK5) {
        static const unsigned pw[5] = {1, 3, 9, 27, 81};
        return (int)((x / pw[j]) % 3u) - 1;
    }
    const unsigned fld = (x >> (2 * j)) & 3u;
    return fld == 0 ? -1 : (fld == 2 ? 1 : 0);
}

}  // namespace

struct xt_sparse_file {
    std::vector<uint8_t> data;
    std::vector<Entry> entries;
    std::map<std::string, size_t> by_name;  // last entry of a name wins, as a HashMap insert
};

// xtern_api.cpp owns the thread-local error string.
int xt_internal_fail(int code, const std::string& msg);

extern "C" {

int xt_sparse_file_open(const void* data, size_t len, xt_sparse_file** out) {
    if (!out) return xt_internal_fail(XT_ERR_INVALID, "out is NULL");
    *out = nullptr;
    if (!data && len) return xt_internal_fail(XT_ERR_INVALID, "NULL data");
    const uint8_t* d = static_cast<const uint8_t*>(data);
    if (len < 17) return xt_internal_fail(XT_ERR_INVALID, "XorSparse file too small");
    if (memcmp(d, kMagic, 9) != 0)
        return xt_internal_fail(XT_ERR_INVALID, "XorSparse bad magic (expected XORSPARE1)");
    const uint32_t version = rd32(d + 9);
    if (version != kVersion)
        return xt_internal_fail(XT_ERR_INVALID,
                                "XorSparse unsupported version " + std::to_string(version));
    const uint32_t count = rd32(d + 13);
    xt_sparse_file* f = new (std::nothrow) xt_sparse_file();
    if (!f) return xt_internal_fail(XT_ERR_NOMEM, "container handle");
    try {
        f->data.assign(d, d + len);
        size_t p = 17;
        for (uint32_t t = 0; t < count; ++t) {
            const std::string where = "XorSparse tensor " + std::to_string(t) + ": ";
            if (p + 4 > len) throw std::string(where + "truncated name length");
            const uint32_t nl = rd32(d + p);
            p += 4;
            if (nl > len - p) throw std::string(where + "truncated name");
            Entry e;
            e.name.assign(reinterpret_cast<const char*>(d + p), nl);
            p += nl;
            if (16 > len - p) throw std::string(where + "truncated header");
            e.out_dim = rd32(d + p);
            e.in_dim = rd32(d + p + 4);
            const uint32_t sb = rd32(d + p + 8);
            memcpy(&e.w_scale, &sb, 4);
            const uint32_t bl = rd32(d + p + 12);
            p += 16;
            if (bl > len - p) throw std::string(where + "blob runs past the end of the file");
            e.blob_off = p;
            e.blob_len = bl;
            p += bl;
            f->by_name[e.name] = f->entries.size();
            f->entries.push_back(std::move(e));
        }
    } catch (const std::string& msg) {
        delete f;
        return xt_internal_fail(XT_ERR_INVALID, msg);
    } catch (...) {
        delete f;
        return xt_internal_fail(XT_ERR_NOMEM, "container copy");
    }
    *out = f;
    return XT_OK;
}

int xt_sparse_file_close(xt_sparse_file* f) {
    delete f;
    return XT_OK;
}

int xt_sparse_file_count(const xt_sparse_file* f, int64_t* n) {
    if (!f || !n) return xt_internal_fail(XT_ERR_INVALID, "NULL argument");
    *n = (int64_t)f->entries.size();
    return XT_OK;
}

int xt_sparse_file_entry(const xt_sparse_file* f, int64_t idx, const char** name, int64_t* out_dim,
                         int64_t* in_dim, float* w_scale, const void** blob, size_t* blob_len) {
    if (!f) return xt_internal_fail(XT_ERR_INVALID, "container is NULL");
    if (idx < 0 || idx >= (int64_t)f->entries.size())
        return xt_internal_fail(XT_ERR_INVALID, "tensor index out of range");
    const Entry& e = f->entries[(size_t)idx];
    if (name) *name = e.name.c_str();
    if (out_dim) *out_dim = e.out_dim;
    if (in_dim) *in_dim = e.in_dim;
    if (w_scale) *w_scale = e.w_scale;
    if (blob) *blob = f->data.data() + e.blob_off;
    if (blob_len) *blob_len = e.blob_len;
    return XT_OK;
}

int xt_sparse_file_find(const xt_sparse_file* f, const char* name, int64_t* idx) {
    if (!f || !name || !idx) return xt_internal_fail(XT_ERR_INVALID, "NULL argument");
    auto it = f->by_name.find(name);
    if (it == f->by_name.end())
        return xt_internal_fail(XT_ERR_INVALID,
                                std::string("XorSparse: tensor '") + name + "' not found");
    *idx = (int64_t)it->second;
    return XT_OK;
}

int xt_weights_create_from_sparse_file(const xt_sparse_file* f, const char* name, int64_t in_dim,
                                       int64_t out_dim, xt_weights** out) {
    if (!out) return xt_internal_fail(XT_ERR_INVALID, "out is NULL");
    *out = nullptr;
    int64_t idx = 0;
    if (int rc = xt_sparse_file_find(f, name, &idx)) return rc;
    const Entry& e = f->entries[(size_t)idx];
    if ((int64_t)e.in_dim != in_dim || (int64_t)e.out_dim != out_dim)
        return xt_internal_fail(XT_ERR_INVALID,
                                std::string("XorSparse '") + name + "' shape mismatch: expected [" +
                                    std::to_string(out_dim) + ", " + std::to_string(in_dim) +
                                    "], got [" + std::to_string(e.out_dim) + ", " +
                                    std::to_string(e.in_dim) + "]");
    std::vector<float> ws;
    try {
        ws.assign((size_t)out_dim, e.w_scale);
    } catch (...) {
        return xt_internal_fail(XT_ERR_NOMEM, "scale buffer");
    }
    return xt_weights_create(XT_XORSPARSE, in_dim, out_dim, f->data.data() + e.blob_off,
                             e.blob_len, ws.data(), out);
}

size_t xt_sparse_file_serialized_size(int64_t n, const char* const* names, const size_t* blob_lens) {
    if (n < 0 || (n > 0 && (!names || !blob_lens))) return 0;
    size_t total = 17;
    for (int64_t t = 0; t < n; ++t) {
        if (!names[t]) return 0;
        total += 4 + strlen(names[t]) + 16 + blob_lens[t];
    }
    return total;
}

int xt_sparse_file_serialize(int64_t n, const char* const* names, const int64_t* out_dims,
                             const int64_t* in_dims, const float* w_scales,
                             const void* const* blobs, const size_t* blob_lens, void* out,
                             size_t out_len) {
    if (n < 0 || n > 0xffffffffLL) return xt_internal_fail(XT_ERR_INVALID, "bad tensor count");
    if (n > 0 && (!names || !out_dims || !in_dims || !w_scales || !blobs || !blob_lens))
        return xt_internal_fail(XT_ERR_INVALID, "NULL argument");
    const size_t need = xt_sparse_file_serialized_size(n, names, blob_lens);
    if (!need) return xt_internal_fail(XT_ERR_INVALID, "NULL tensor name");
    if (!out || out_len < need)
        return xt_internal_fail(XT_ERR_INVALID, "output buffer holds " + std::to_string(out_len) +
                                                    " bytes, need " + std::to_string(need));
    uint8_t* o = static_cast<uint8_t*>(out);
    memcpy(o, kMagic, 9);
    wr32(o + 9, kVersion);
    wr32(o + 13, (uint32_t)n);
    size_t p = 17;
    for (int64_t t = 0; t < n; ++t) {
        const size_t nl = strlen(names[t]);
        if (nl > 0xffffffffu || blob_lens[t] > 0xffffffffu || out_dims[t] < 0 || in_dims[t] < 0 ||
            out_dims[t] > 0xffffffffLL || in_dims[t] > 0xffffffffLL || (blob_lens[t] && !blobs[t]))
            return xt_internal_fail(XT_ERR_INVALID, "tensor " + std::to_string(t) +
                                                        " does not fit the u32 fields");
        wr32(o + p, (uint32_t)nl);
        memcpy(o + p + 4, names[t], nl);
        p += 4 + nl;
        wr32(o + p, (uint32_t)out_dims[t]);
        wr32(o + p + 4, (uint32_t)in_dims[t]);
        uint32_t sb;
        memcpy(&sb, &w_scales[t], 4);
        wr32(o + p + 8, sb);
        wr32(o + p + 12, (uint32_t)blob_lens[t]);
        p += 16;
        if (blob_lens[t]) memcpy(o + p, blobs[t], blob_lens[t]);
        p += blob_lens[t];
    }
    return XT_OK;
}

int xt_hf_to_sparse_blob(int fmt, int64_t in_dim, int64_t out_dim, const void* stored,
                         size_t nbytes, int destripe, void* blob_out, size_t cap,
                         size_t* blob_len) {
    if (!stored || !blob_len) return xt_internal_fail(XT_ERR_INVALID, "NULL argument");
    if (fmt != XT_PACK4 && fmt != XT_PACK5)
        return xt_internal_fail(XT_ERR_INVALID, "HF prepacked weights are Pack4 or Pack5 only");
    const int64_t f = fmt == XT_PACK5 ? 5 : 4;
    if (in_dim <= 0 || out_dim <= 0 || out_dim % f != 0 ||
        (uint64_t)nbytes != (uint64_t)(in_dim * (out_dim / f)))
        return xt_internal_fail(
            XT_ERR_INVALID, "Tensor is not in pre-packed U8 ternary format: expected [" +
                                std::to_string(out_dim / f) + "][" + std::to_string(in_dim) +
                                "] bytes for out_dim " + std::to_string(out_dim) + ", got " +
                                std::to_string(nbytes));
    const uint8_t* st = static_cast<const uint8_t*>(stored);
    const int64_t nb = (in_dim + 63) / 64;
    // sparse.rs:61-86 per row: num_blocks, then per block mask + set-order signs
    size_t total = 0;
    for (int64_t o = 0; o < out_dim; ++o) {
        total += 4;
        for (int64_t b = 0; b < nb; ++b) {
            int nnz = 0;
            for (int64_t l = 0; l < 64 && b * 64 + l < in_dim; ++l)
                nnz += hf_value(st, fmt, in_dim, out_dim, o, b * 64 + l, destripe != 0) != 0;
            total += 8 + (size_t)(nnz + 7) / 8;
        }
    }
    *blob_len = total;
    if (!blob_out) return XT_OK;
    if (cap < total)
        return xt_internal_fail(XT_ERR_INVALID, "blob buffer holds " + std::to_string(cap) +
                                                    " bytes, need " + std::to_string(total));
    uint8_t* w = static_cast<uint8_t*>(blob_out);
    size_t p = 0;
    for (int64_t o = 0; o < out_dim; ++o) {
        wr32(w + p, (uint32_t)nb);
        p += 4;
        for (int64_t b = 0; b < nb; ++b) {
            uint64_t mask = 0;
            uint8_t signs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int nz = 0;
            for (int64_t l = 0; l < 64 && b * 64 + l < in_dim; ++l) {
                const int v = hf_value(st, fmt, in_dim, out_dim, o, b * 64 + l, destripe != 0);
                if (!v) continue;
                mask |= 1ull << l;
                if (v < 0) signs[nz >> 3] |= (uint8_t)(1u << (nz & 7));
                ++nz;
            }
            for (int t = 0; t < 8; ++t) w[p + t] = (uint8_t)(mask >> (8 * t));
            p += 8;
            const int sbytes = (nz + 7) / 8;
            memcpy(w + p, signs, (size_t)sbytes);
            p += (size_t)sbytes;
        }
    }
    return XT_OK;
}

}  // extern "C"
