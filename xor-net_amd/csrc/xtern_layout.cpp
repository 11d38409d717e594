// Host-side repack of the reference's weight byte layouts into the xtern
// device tile layout (geometry documented in xtern_internal.h).
//
// Input formats (paths relative to xor-net):
//   Pack4      src/bit1_58/quantization.rs:7-46   ([N][ceil(K/4)] bytes)
//   Pack5      src/bit1_58/quantization.rs:48-91  ([N][ceil(K/5)] bytes)
//   XorSparse  src/bit1_58/sparse.rs:9-17, :135-194 (row blobs)
#include <math.h>
#include <string.h>

#include <string>
#include <vector>

#include "xtern_layout.h"

namespace xt {

size_t tile_bytes(int fmt, int64_t K, int64_t N) {
    const int64_t ch = chunk_cols(fmt);
    const int64_t nch = (K + ch - 1) / ch;
    const int64_t ng = (N + 15) / 16;
    return (size_t)(ng * nch * tiles_per_chunk(fmt) * kTileBytes);
}

namespace {

// Place the code of (row o, column k) into a Pack4 tile buffer.
inline void put4(uint8_t* tiles, int64_t nch, int64_t o, int64_t k, unsigned code) {
    const int64_t G = o >> 4, j = o & 15;
    const int64_t c = k >> 8, kk = k & 255;
    const int64_t s = kk >> 6, g = (kk & 63) >> 4, b = kk & 15;
    const int64_t jj = b >> 2, d = b & 3;
    uint8_t* p = tiles + ((G * nch + c) * 64 + g * 16 + j) * 16 + s * 4 + d;
    const int sh = (int)(2 * jj);
    *p = (uint8_t)((*p & ~(3u << sh)) | (code << sh));
}

// Pack4 code of a reference byte field: 00 -> -1, 10 -> +1, 01 and 11 -> 0
// (quantization.rs:36-41).  Canonical device code = weight + 1.
inline unsigned canon4(unsigned field) { return field == 0 ? 0u : (field == 2 ? 2u : 1u); }

int repack_pack4(int64_t K, int64_t N, const uint8_t* src, size_t nbytes, uint8_t* tiles,
                 std::string* err) {
    const int64_t bpr = (K + 3) / 4;
    if ((uint64_t)nbytes < (uint64_t)(bpr * N)) {
        *err = "Pack4 weights: expected " + std::to_string(bpr * N) + " bytes ([out_dim][ceil(in_dim/4)]), got " +
               std::to_string(nbytes);
        return -1;
    }
    const int64_t nch = (K + 255) / 256;
    for (int64_t o = 0; o < N; ++o) {
        const uint8_t* row = src + o * bpr;
        for (int64_t k = 0; k < K; ++k)
            put4(tiles, nch, o, k, canon4((row[k >> 2] >> (2 * (k & 3))) & 3u));
    }
    return 0;
}

// XorSparse row blobs -> Pack4 tiles (lossless; same weights as the dense
// Pack4 encoding of the rows).
int repack_sparse(int64_t K, int64_t N, const uint8_t* blob, size_t nbytes, uint8_t* tiles,
                  std::string* err) {
    const int64_t nch = (K + 255) / 256;
    const int64_t want_nb = (K + 63) / 64;
    size_t p = 0;
    for (int64_t o = 0; o < N; ++o) {
        if (p + 4 > nbytes) {
            *err = "XorSparse blob truncated at row " + std::to_string(o);
            return -1;
        }
        const uint32_t nb = (uint32_t)blob[p] | ((uint32_t)blob[p + 1] << 8) |
                            ((uint32_t)blob[p + 2] << 16) | ((uint32_t)blob[p + 3] << 24);
        p += 4;
        if ((int64_t)nb != want_nb) {
            *err = "XorSparse row " + std::to_string(o) + ": num_blocks " + std::to_string(nb) +
                   " != ceil(in_dim/64) = " + std::to_string(want_nb);
            return -1;
        }
        for (int64_t b = 0; b < want_nb; ++b) {
            if (p + 8 > nbytes) {
                *err = "XorSparse blob truncated at row " + std::to_string(o);
                return -1;
            }
            uint64_t mask = 0;
            for (int t = 0; t < 8; ++t) mask |= (uint64_t)blob[p + t] << (8 * t);
            p += 8;
            const int nnz = __builtin_popcountll(mask);
            const size_t sbytes = (size_t)(nnz + 7) / 8;
            if (p + sbytes > nbytes) {
                *err = "XorSparse blob truncated at row " + std::to_string(o);
                return -1;
            }
            if (b * 64 + 64 > K && (mask >> (K - b * 64)) != 0) {
                *err = "XorSparse row " + std::to_string(o) + ": mask sets lanes beyond in_dim";
                return -1;
            }
            uint64_t sb = 0;
            for (size_t t = 0; t < sbytes; ++t) sb |= (uint64_t)blob[p + t] << (8 * t);
            p += sbytes;
            unsigned si = 0;
            for (int lane = 0; lane < 64; ++lane) {
                if (!((mask >> lane) & 1u)) continue;
                const unsigned neg = (unsigned)((sb >> si) & 1u);
                ++si;
                put4(tiles, nch, o, b * 64 + lane, neg ? 0u : 2u);
            }
        }
    }
    return 0;
}

int repack_pack5(int64_t K, int64_t N, const uint8_t* src, size_t nbytes, uint8_t* tiles,
                 std::string* err) {
    const int64_t bpr = (K + 4) / 5;
    if ((uint64_t)nbytes < (uint64_t)(bpr * N)) {
        *err = "Pack5 weights: expected " + std::to_string(bpr * N) + " bytes ([out_dim][ceil(in_dim/5)]), got " +
               std::to_string(nbytes);
        return -1;
    }
    const int64_t nch = (K + 319) / 320;
    const int64_t ng = (N + 15) / 16;
    for (int64_t G = 0; G < ng; ++G) {
        // trits (weight + 1) of the 16 rows of this group; 1 = padding
        std::vector<uint8_t> rows((size_t)(16 * K), 1);
        for (int64_t j = 0; j < 16; ++j) {
            const int64_t o = G * 16 + j;
            if (o >= N) break;
            const uint8_t* row = src + o * bpr;
            // quantization.rs:72-91 / simd.rs:388-414: repeated %3 and /3.
            for (int64_t c = 0; c < bpr; ++c) {
                unsigned b = row[c];
                for (int t = 0; t < 5 && c * 5 + t < K; ++t) {
                    rows[(size_t)(j * K + c * 5 + t)] = (uint8_t)(b % 3);
                    b /= 3;
                }
            }
        }
        for (int64_t c = 0; c < nch; ++c) {
            uint8_t* out = tiles + (G * nch + c) * kTileBytes;
            for (int lane = 0; lane < 64; ++lane) {
                const int g = lane >> 4, j = lane & 15;
                for (int b = 0; b < 16; ++b) {
                    unsigned v = 0;
                    for (int s = 0; s < 5; ++s) {
                        const int64_t k = c * 320 + s * 64 + g * 16 + b;
                        const unsigned t = (k < K) ? rows[(size_t)(j * K + k)] : 1u;
                        v = v * 3 + t;
                    }
                    out[lane * 16 + b] = (uint8_t)((v * 256 + 242) / 243);
                }
            }
        }
    }
    return 0;
}

// Int8Linear weight_i8 [N][K] (dynamic_linear.rs:236-258) -> Int8 tiles.
int repack_int8(int64_t K, int64_t N, const uint8_t* src, size_t nbytes, uint8_t* tiles,
                std::string* err) {
    if ((uint64_t)nbytes < (uint64_t)(K * N)) {
        *err = "Int8 weights: expected " + std::to_string(K * N) + " bytes ([out_dim][in_dim]), got " +
               std::to_string(nbytes);
        return -1;
    }
    const int64_t nch = (K + 255) / 256;
    memset(tiles, 0, tile_bytes(3, K, N));
    for (int64_t o = 0; o < N; ++o) {
        const int64_t G = o >> 4, j = o & 15;
        for (int64_t k = 0; k < K; ++k) {
            const int64_t c = k >> 8, kk = k & 255, s = kk >> 6, g = (kk & 63) >> 4, b = kk & 15;
            tiles[(((G * nch + c) * 4 + s) * 64 + g * 16 + j) * 16 + b] = src[o * K + k];
        }
    }
    return 0;
}

// Int4Linear weight_i4 [N][ceil(K/2)] (dynamic_linear.rs:389-410: column 2c
// in the low nibble, 2c+1 in the high one, two's complement) -> Int4 tiles
// of codes q + 8.  Int4Linear's dot pairs the bytes with
// quantized_in.chunks_exact(2) (:442-449), so for odd K the last column never
// contributes: it is stored as q = 0.
int repack_int4(int64_t K, int64_t N, const uint8_t* src, size_t nbytes, uint8_t* tiles,
                std::string* err) {
    const int64_t bpr = (K + 1) / 2;
    if ((uint64_t)nbytes < (uint64_t)(bpr * N)) {
        *err = "Int4 weights: expected " + std::to_string(bpr * N) +
               " bytes ([out_dim][ceil(in_dim/2)]), got " + std::to_string(nbytes);
        return -1;
    }
    const int64_t nch = (K + 255) / 256;
    memset(tiles, 0x88, tile_bytes(4, K, N));  // code 8 = weight 0 everywhere
    const int64_t kuse = K & ~(int64_t)1;       // columns the reference's dot reads
    for (int64_t o = 0; o < N; ++o) {
        const int64_t G = o >> 4, j = o & 15;
        for (int64_t k = 0; k < kuse; ++k) {
            const unsigned byte = src[o * bpr + (k >> 1)];
            const unsigned nib = (k & 1) ? (byte >> 4) : (byte & 15u);
            const unsigned code = nib ^ 8u;  // q + 8 for the two's-complement nibble q
            const int64_t c = k >> 8, kk = k & 255, s = kk >> 6, g = (kk & 63) >> 4, b = kk & 15;
            uint8_t* p = tiles + (((G * nch + c) * 2 + (s >> 1)) * 64 + g * 16 + j) * 16 + b;
            const int sh = (s & 1) ? 4 : 0;
            *p = (uint8_t)((*p & ~(15u << sh)) | (code << sh));
        }
    }
    return 0;
}

}  // namespace

int build_xs_stream(int64_t K, int64_t N, const uint8_t* blob, size_t nbytes,
                    std::vector<uint8_t>* out, XsLayout* lay, std::string* err) {
    const int64_t nb = (K + 63) / 64, ng = (N + 15) / 16;
    std::vector<uint64_t> mask, sgn;
    try {
        mask.assign((size_t)(ng * 16 * nb), 0);
        sgn.assign((size_t)(ng * 16 * nb), 0);
    } catch (...) {
        *err = "host buffer for the XorSparse stream";
        return -1;
    }
    // the blob, validated as for the tile layout (sparse.rs:135-194)
    size_t p = 0;
    uint64_t bits = 0;
    for (int64_t o = 0; o < N; ++o) {
        if (p + 4 > nbytes) {
            *err = "XorSparse blob truncated at row " + std::to_string(o);
            return -1;
        }
        const uint32_t nbr = (uint32_t)blob[p] | ((uint32_t)blob[p + 1] << 8) |
                             ((uint32_t)blob[p + 2] << 16) | ((uint32_t)blob[p + 3] << 24);
        p += 4;
        if ((int64_t)nbr != nb) {
            *err = "XorSparse row " + std::to_string(o) + ": num_blocks " + std::to_string(nbr) +
                   " != ceil(in_dim/64) = " + std::to_string(nb);
            return -1;
        }
        for (int64_t b = 0; b < nb; ++b) {
            if (p + 8 > nbytes) {
                *err = "XorSparse blob truncated at row " + std::to_string(o);
                return -1;
            }
            uint64_t m = 0;
            for (int t = 0; t < 8; ++t) m |= (uint64_t)blob[p + t] << (8 * t);
            p += 8;
            const int nnz = __builtin_popcountll(m);
            const size_t sbytes = (size_t)(nnz + 7) / 8;
            if (p + sbytes > nbytes) {
                *err = "XorSparse blob truncated at row " + std::to_string(o);
                return -1;
            }
            if (b * 64 + 64 > K && (m >> (K - b * 64)) != 0) {
                *err = "XorSparse row " + std::to_string(o) + ": mask sets lanes beyond in_dim";
                return -1;
            }
            uint64_t sb = 0;
            for (size_t t = 0; t < sbytes; ++t) sb |= (uint64_t)blob[p + t] << (8 * t);
            p += sbytes;
            if (nnz < 64) sb &= ((uint64_t)1 << nnz) - 1;
            mask[(size_t)(o * nb + b)] = m;
            sgn[(size_t)(o * nb + b)] = sb;
            bits += (uint64_t)nnz;
        }
    }
    // Sections (each within a 32-bit buffer range; the kernel adds offsets
    // below 2^31)
    const uint64_t words = (bits + 31) / 32 + 3;  // + the window the last lane reads
    XsLayout L;
    L.nb = nb;
    L.ng = ng;
    L.seg_off = 0;
    const uint64_t seg_b = (uint64_t)(ng * nb) * 4, mask_b = (uint64_t)(ng * nb) * 128;
    L.mask_off = (size_t)((seg_b + 255) / 256 * 256);
    L.sign_off = (size_t)((L.mask_off + mask_b + 255) / 256 * 256);
    L.sign_bytes = (size_t)(words * 4);
    L.total = L.sign_off + L.sign_bytes;
    if (bits >= ((uint64_t)1 << 32) - 256 || mask_b >= ((uint64_t)1 << 31) ||
        words * 4 >= ((uint64_t)1 << 31)) {
        *err = "XorSparse stream above 2 GiB per section is not supported";
        return -1;
    }
    try {
        out->assign(L.total, 0);
    } catch (...) {
        *err = "host buffer for the XorSparse stream";
        return -1;
    }
    uint8_t* base = out->data();
    uint32_t* seg = reinterpret_cast<uint32_t*>(base + L.seg_off);
    uint64_t* msk = reinterpret_cast<uint64_t*>(base + L.mask_off);
    uint32_t* sw = reinterpret_cast<uint32_t*>(base + L.sign_off);
    uint64_t pos = 0;
    for (int64_t G = 0; G < ng; ++G)
        for (int64_t b = 0; b < nb; ++b) {
            seg[G * nb + b] = (uint32_t)pos;
            for (int j = 0; j < 16; ++j) {
                const int64_t o = G * 16 + j;
                const uint64_t m = o < N ? mask[(size_t)(o * nb + b)] : 0;
                const uint64_t sb = o < N ? sgn[(size_t)(o * nb + b)] : 0;
                msk[(G * nb + b) * 16 + j] = m;
                const int n = __builtin_popcountll(m);
                for (int i = 0; i < n; ++i, ++pos)
                    if ((sb >> i) & 1) sw[pos >> 5] |= 1u << (pos & 31);
            }
        }
    *lay = L;
    return 0;
}

// Int8Linear::new / Int4Linear::new (dynamic_linear.rs:236-258, :389-410).
int int_quantize(int bits, const float* w, int64_t N, int64_t K, uint8_t* out, float* scales) {
    const float qmax = bits == 8 ? 127.0f : 7.0f;
    const int64_t bpr = bits == 8 ? K : (K + 1) / 2;
    for (int64_t o = 0; o < N; ++o) {
        const float* row = w + o * K;
        float mx = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const float a = fabsf(row[k]);
            mx = (a > mx) ? a : mx;  // f32::max fold: NaN never replaces the max
        }
        const float scale = mx > 0.0f ? mx / qmax : 1.0f;
        scales[o] = scale;
        auto q_of = [&](float v) {
            // (v / scale).round().max(lo).min(hi) as i8; NaN -> lo
            float r = roundf(v / scale);
            const float lo = bits == 8 ? -127.0f : -8.0f, hi = bits == 8 ? 127.0f : 7.0f;
            r = (r != r) ? lo : (r < lo ? lo : r);
            r = r > hi ? hi : r;
            return (int)r;
        };
        uint8_t* dst = out + o * bpr;
        if (bits == 8) {
            for (int64_t k = 0; k < K; ++k) dst[k] = (uint8_t)(int8_t)q_of(row[k]);
        } else {
            for (int64_t c = 0; c < bpr; ++c) {
                const int q0 = q_of(row[2 * c]);
                const int q1 = 2 * c + 1 < K ? q_of(row[2 * c + 1]) : q_of(0.0f);
                dst[c] = (uint8_t)(((unsigned)q0 & 15u) | ((unsigned)q1 << 4));
            }
        }
    }
    return 0;
}

// loader/mod.rs:351-390 without the f32 round trip: the value of (row o,
// column i) is digit j of stored byte [p][i] with o = j*R + p, R = N/f; it
// is re-emitted in input-dim order exactly as pack_1_58bit_{4,5}pack at
// scale 1.0 would (quantization.rs:7-70): Pack4 code 11 becomes 01, unused
// high fields / digits of a row's last byte stay 0.
int hf_destripe(int fmt, int64_t K, int64_t N, const uint8_t* stored, size_t nbytes,
                uint8_t* out, std::string* err) {
    if (fmt != 0 && fmt != 1) {
        *err = "HF prepacked weights are Pack4 or Pack5 only";
        return -1;
    }
    const int64_t f = fmt == 1 ? 5 : 4;
    if (K <= 0 || N <= 0 || N % f != 0 || (uint64_t)nbytes != (uint64_t)(K * (N / f))) {
        *err = "Tensor is not in pre-packed U8 ternary format: expected [" + std::to_string(N / f) +
               "][" + std::to_string(K) + "] bytes for out_dim " + std::to_string(N) +
               " (a multiple of " + std::to_string(f) + "), got " + std::to_string(nbytes);
        return -1;
    }
    const int64_t R = N / f, bpr = (K + f - 1) / f;
    static const unsigned pow3[5] = {1, 3, 9, 27, 81};
    for (int64_t o = 0; o < N; ++o) {
        const int64_t j = o / R, p = o % R;
        const uint8_t* src = stored + p * K;
        uint8_t* dst = out + o * bpr;
        for (int64_t c = 0; c < bpr; ++c) {
            unsigned b = 0;
            for (int64_t t = 0; t < f && c * f + t < K; ++t) {
                const unsigned x = src[c * f + t];
                if (fmt == 0) {
                    const unsigned code = canon4((x >> (2 * j)) & 3u);
                    b |= code << (2 * t);
                } else {
                    b += ((x / pow3[j]) % 3u) * pow3[t];
                }
            }
            dst[c] = (uint8_t)b;
        }
    }
    return 0;
}

int repack(int fmt, int64_t K, int64_t N, const void* src, size_t nbytes, void* dst,
           std::string* err) {
    if (K <= 0 || N <= 0) {
        *err = "in_dim and out_dim must be positive";
        return -1;
    }
    if (K > (int64_t)1 << 30 || N > (int64_t)1 << 30) {
        *err = "in_dim/out_dim above 2^30 are not supported";
        return -1;
    }
    if (fmt < 0 || fmt > 4) {
        *err = "unknown weight format " + std::to_string(fmt);
        return -1;
    }
    if (fmt == 3) return repack_int8(K, N, static_cast<const uint8_t*>(src), nbytes,
                                     static_cast<uint8_t*>(dst), err);
    if (fmt == 4) return repack_int4(K, N, static_cast<const uint8_t*>(src), nbytes,
                                     static_cast<uint8_t*>(dst), err);
    const size_t tb = tile_bytes(fmt, K, N);
    uint8_t* tiles = static_cast<uint8_t*>(dst);
    if (fmt == 1) return repack_pack5(K, N, static_cast<const uint8_t*>(src), nbytes, tiles, err);
    memset(tiles, 0x55, tb);  // code 1 (weight 0) in every 2-bit field
    if (fmt == 0) return repack_pack4(K, N, static_cast<const uint8_t*>(src), nbytes, tiles, err);
    return repack_sparse(K, N, static_cast<const uint8_t*>(src), nbytes, tiles, err);
}

}  // namespace xt
