// Mutation fuzzing of the host-side parsers, built with AddressSanitizer and
// UndefinedBehaviorSanitizer from the host-only sources (xtern_layout.cpp,
// xtern_container.cpp; no device code):
//   * XorSparse row blobs (the repack of format XT_XORSPARSE), valid ones and
//     byte-flipped / truncated / extended copies;
//   * the XORSPARE1 container reader, on mutated serialised files;
//   * the Pack4 / Pack5 / Int8 / Int4 repacks and the HF destripe with short
//     or oversized inputs;
//   * the HF -> XorSparse blob step, sizes only.
// Every call must return normally (0 or an error code); any out-of-bounds
// access or undefined behaviour aborts the program under the sanitizers.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>
#include <string>
#include <vector>

#include "../../include/xtern.h"
#include "../../xor-net_amd/csrc/xtern_layout.h"

// The two library entry points the container source calls outside itself:
// the error setter and the device upload (never reached with valid inputs
// here; it reports "unsupported" without touching a device).
int xt_internal_fail(int code, const std::string&) { return code; }
extern "C" int xt_weights_create(int, int64_t, int64_t, const void*, size_t, const float*,
                                 xt_weights** out) {
    if (out) *out = nullptr;
    return XT_ERR_UNSUPPORTED;
}

namespace {

std::mt19937_64 rng(12345);

// sparse.rs:61-86 layout: per row u32 num_blocks, per 64-block u64 lane mask
// then ceil(popcount / 8) sign bytes in set order (bit j: j-th non-zero is -1).
std::vector<uint8_t> encode_sparse(const std::vector<int8_t>& t, int64_t K, int64_t N) {
    std::vector<uint8_t> out;
    const int64_t nb = (K + 63) / 64;
    for (int64_t o = 0; o < N; ++o) {
        const uint32_t n32 = (uint32_t)nb;
        for (int b = 0; b < 4; ++b) out.push_back((uint8_t)(n32 >> (8 * b)));
        for (int64_t b = 0; b < nb; ++b) {
            uint64_t mask = 0;
            std::vector<int> signs;
            for (int l = 0; l < 64 && b * 64 + l < K; ++l) {
                const int8_t v = t[o * K + b * 64 + l];
                if (v) {
                    mask |= 1ull << l;
                    signs.push_back(v < 0);
                }
            }
            for (int k = 0; k < 8; ++k) out.push_back((uint8_t)(mask >> (8 * k)));
            for (size_t s0 = 0; s0 < signs.size(); s0 += 8) {
                uint8_t byte = 0;
                for (size_t s = s0; s < signs.size() && s < s0 + 8; ++s)
                    byte |= (uint8_t)(signs[s] << (s - s0));
                out.push_back(byte);
            }
        }
    }
    return out;
}

void mutate(std::vector<uint8_t>& v) {
    const int kind = (int)(rng() % 4);
    if (kind == 0 && !v.empty()) {  // flip bytes
        const int n = 1 + (int)(rng() % 4);
        for (int i = 0; i < n; ++i) v[rng() % v.size()] ^= (uint8_t)(1 + rng() % 255);
    } else if (kind == 1 && !v.empty()) {  // truncate
        v.resize(rng() % v.size());
    } else if (kind == 2) {  // extend with garbage
        const int n = 1 + (int)(rng() % 64);
        for (int i = 0; i < n; ++i) v.push_back((uint8_t)rng());
    } else if (!v.empty()) {  // overwrite a 4-byte field with an extreme value
        const size_t at = rng() % v.size();
        const uint32_t vals[] = {0u, 1u, 0x7fffffffu, 0xffffffffu, 0x10000u};
        const uint32_t x = vals[rng() % 5];
        for (int b = 0; b < 4 && at + b < v.size(); ++b) v[at + b] = (uint8_t)(x >> (8 * b));
    }
}

int fuzz_sparse_blob(int iters) {
    int ok = 0;
    for (int it = 0; it < iters; ++it) {
        const int64_t K = 1 + (int64_t)(rng() % 300), N = 1 + (int64_t)(rng() % 40);
        std::vector<int8_t> t((size_t)(K * N));
        for (auto& v : t) v = (int8_t)((int)(rng() % 3) - 1);
        std::vector<uint8_t> blob = encode_sparse(t, K, N);
        if (it % 4) mutate(blob);
        std::vector<uint8_t> tiles(xt::tile_bytes(XT_XORSPARSE, K, N));
        std::string err;
        if (xt::repack(XT_XORSPARSE, K, N, blob.data(), blob.size(), tiles.data(), &err) == 0) ++ok;
    }
    return ok;
}

int fuzz_container(int iters) {
    int opened = 0;
    for (int it = 0; it < iters; ++it) {
        const int n = 1 + (int)(rng() % 3);
        std::vector<std::string> names;
        std::vector<std::vector<uint8_t>> blobs;
        std::vector<int64_t> outs, ins;
        std::vector<float> scales;
        for (int e = 0; e < n; ++e) {
            const int64_t K = 1 + (int64_t)(rng() % 130), N = 1 + (int64_t)(rng() % 9);
            std::vector<int8_t> t((size_t)(K * N));
            for (auto& v : t) v = (int8_t)((int)(rng() % 3) - 1);
            names.push_back("layer." + std::to_string(e) + ".w");
            blobs.push_back(encode_sparse(t, K, N));
            outs.push_back(N);
            ins.push_back(K);
            scales.push_back(0.5f + e);
        }
        std::vector<const char*> np;
        std::vector<const void*> bp;
        std::vector<size_t> bl;
        for (int e = 0; e < n; ++e) {
            np.push_back(names[e].c_str());
            bp.push_back(blobs[e].data());
            bl.push_back(blobs[e].size());
        }
        const size_t sz = xt_sparse_file_serialized_size(n, np.data(), bl.data());
        std::vector<uint8_t> file(sz);
        if (xt_sparse_file_serialize(n, np.data(), outs.data(), ins.data(), scales.data(), bp.data(),
                                     bl.data(), file.data(), file.size()) != XT_OK) {
            fprintf(stderr, "serialize failed\n");
            return -1;
        }
        if (it % 4) mutate(file);
        xt_sparse_file* f = nullptr;
        if (xt_sparse_file_open(file.data(), file.size(), &f) != XT_OK) continue;
        ++opened;
        int64_t cnt = 0;
        xt_sparse_file_count(f, &cnt);
        for (int64_t e = 0; e < cnt; ++e) {
            const char* name = nullptr;
            int64_t od = 0, id = 0;
            float ws = 0;
            const void* blob = nullptr;
            size_t blen = 0;
            if (xt_sparse_file_entry(f, e, &name, &od, &id, &ws, &blob, &blen) != XT_OK) continue;
            // the entry's blob through the parser, at the entry's shape when small
            if (od > 0 && id > 0 && od <= (1 << 16) && id <= (1 << 16) && od * id <= (1 << 16)) {
                std::vector<uint8_t> tiles(xt::tile_bytes(XT_XORSPARSE, id, od));
                std::string err;
                xt::repack(XT_XORSPARSE, id, od, blob, blen, tiles.data(), &err);
            }
            int64_t idx = -1;
            xt_sparse_file_find(f, name, &idx);
        }
        xt_sparse_file_close(f);
    }
    return opened;
}

int fuzz_dense(int iters) {
    int ok = 0;
    const int fmts[] = {XT_PACK4, XT_PACK5, XT_INT8, XT_INT4};
    for (int it = 0; it < iters; ++it) {
        const int fmt = fmts[rng() % 4];
        const int64_t K = 1 + (int64_t)(rng() % 700), N = 1 + (int64_t)(rng() % 40);
        const int64_t bpr = fmt == XT_PACK4 ? (K + 3) / 4
                            : fmt == XT_PACK5 ? (K + 4) / 5
                            : fmt == XT_INT8  ? K
                                              : (K + 1) / 2;
        size_t nbytes = (size_t)(bpr * N);
        if (it % 3 == 1) nbytes = rng() % (nbytes + 1);             // short
        if (it % 3 == 2) nbytes += 1 + rng() % 17;                  // oversized
        std::vector<uint8_t> src(nbytes);
        for (auto& b : src) b = (uint8_t)rng();
        std::vector<uint8_t> tiles(xt::tile_bytes(fmt, K, N));
        std::string err;
        if (xt::repack(fmt, K, N, src.data(), src.size(), tiles.data(), &err) == 0) ++ok;
        if (fmt == XT_PACK4 || fmt == XT_PACK5) {
            const int64_t f = fmt == XT_PACK5 ? 5 : 4;
            const int64_t Nh = f * (1 + (int64_t)(rng() % 8));
            size_t hb = (size_t)((Nh / f) * K);
            if (it % 3 == 1) hb = rng() % (hb + 1);
            std::vector<uint8_t> stored(hb);
            for (auto& b : stored) b = (uint8_t)rng();
            std::vector<uint8_t> rows((size_t)(Nh * bpr));
            xt::hf_destripe(fmt, K, Nh, stored.data(), stored.size(), rows.data(), &err);
            size_t blen = 0;
            if (xt_hf_to_sparse_blob(fmt, K, Nh, stored.data(), stored.size(), it & 1, nullptr, 0,
                                     &blen) == XT_OK &&
                blen < (1u << 20)) {
                std::vector<uint8_t> blob(blen);
                xt_hf_to_sparse_blob(fmt, K, Nh, stored.data(), stored.size(), it & 1, blob.data(),
                                     blob.size(), &blen);
                std::vector<uint8_t> st2(xt::tile_bytes(XT_XORSPARSE, K, Nh));
                xt::repack(XT_XORSPARSE, K, Nh, blob.data(), blob.size(), st2.data(), &err);
            }
        }
    }
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 3000;
    const int a = fuzz_sparse_blob(iters);
    const int b = fuzz_container(iters);
    const int c = fuzz_dense(iters);
    if (a < 0 || b < 0 || c < 0) return 1;
    // the unmutated quarter must parse
    if (a < iters / 4 || b < iters / 4) {
        fprintf(stderr, "valid inputs rejected: sparse %d container %d of %d\n", a, b, iters);
        return 1;
    }
    printf("fuzz ok: sparse blobs parsed %d/%d, containers opened %d/%d, dense repacks %d/%d\n", a,
           iters, b, iters, c, iters);
    return 0;
}
