/*
 * xtern oracle — CPU restatement of xor-net's ternary linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and bench.py's cpu_baseline leg);
 * never linked into or called by the product library.  Built with
 * -ffp-contract=off so every f32 expression rounds exactly as the reference's
 * Rust code does (Rust never contracts a*b*c into an FMA).
 *
 * Paths in citations are relative to the xor-net source tree.
 */
#include "xtern_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* Pack4 / Pack5 codecs                                                      */
/* ------------------------------------------------------------------------ */

/* Per-weight ternarisation used by both packers (quantization.rs:12-21 and
 * :54-63): q = clamp(round_half_away(w / s), -1, 1) with s <= 0 giving 0,
 * then q < -0.5 -> -1, q > 0.5 -> +1, else 0.  Returns the ternary value. */
static int ternarise(float w, float w_scale) {
    float scaled = (w_scale > 0.0f) ? w / w_scale : 0.0f;
    float q = roundf(scaled);
    /* Rust's f32::max(NaN, -1) is -1, so a NaN weight ternarises to -1. */
    if (isnan(q)) q = -1.0f;
    if (q < -1.0f) q = -1.0f;
    if (q > 1.0f) q = 1.0f;
    if (q < -0.5f) return -1;
    if (q > 0.5f) return 1;
    return 0;
}

/* quantization.rs:7-27 — 2-bit codes 00=-1, 01=0, 10=+1, weight j of a byte in
 * bits 2j..2j+1, last byte zero-padded in its unused high bits. */
void or_pack4(const float* w, int64_t n, float w_scale, uint8_t* out) {
    for (int64_t c = 0; c * 4 < n; ++c) {
        uint8_t b = 0;
        for (int j = 0; j < 4 && c * 4 + j < n; ++j) {
            int t = ternarise(w[c * 4 + j], w_scale);
            uint8_t code = (t < 0) ? 0u : (t > 0) ? 2u : 1u;
            b |= (uint8_t)(code << (2 * j));
        }
        out[c] = b;
    }
}

/* quantization.rs:29-46 — code 00 -> -1, 10 -> +1, 01 and 11 -> 0. */
void or_unpack4(const uint8_t* packed, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        unsigned code = (packed[i / 4] >> (2 * (i % 4))) & 3u;
        out[i] = (code == 0) ? -1.0f : (code == 2) ? 1.0f : 0.0f;
    }
}

/* quantization.rs:48-70 — byte = sum_j t_j * 3^j, t = 0(-1), 1(0), 2(+1); the
 * first weight of a group is the least-significant trit.  A short last group
 * only holds the trits it has (higher trits are 0, i.e. not "weight 0"). */
void or_pack5(const float* w, int64_t n, float w_scale, uint8_t* out) {
    for (int64_t c = 0; c * 5 < n; ++c) {
        unsigned b = 0, mul = 1;
        for (int j = 0; j < 5 && c * 5 + j < n; ++j) {
            int t = ternarise(w[c * 5 + j], w_scale);
            unsigned v = (t < 0) ? 0u : (t > 0) ? 2u : 1u;
            b += v * mul;
            mul *= 3;
        }
        out[c] = (uint8_t)b;
    }
}

/* quantization.rs:72-91 — repeated %3, /3; digit 0 -> -1, 2 -> +1, 1 -> 0. */
void or_unpack5(const uint8_t* packed, int64_t n, float* out) {
    for (int64_t c = 0; c * 5 < n; ++c) {
        unsigned b = packed[c];
        for (int j = 0; j < 5 && c * 5 + j < n; ++j) {
            unsigned v = b % 3;
            b /= 3;
            out[c * 5 + j] = (v == 0) ? -1.0f : (v == 2) ? 1.0f : 0.0f;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Activation quantiser                                                      */
/* ------------------------------------------------------------------------ */

/* quantization.rs:95-145.  The absmax keeps 16 lane maxima updated with the
 * x86 MAXPS rule m = (m > v) ? m : v, then folds them and the scalar tail
 * with `if v > max`.  Main lanes: scaled = x*scale, clamp with MINPS/MAXPS
 * operand order (127 < s ? 127 : s, then -127 > t ? -127 : t), convert with
 * round-half-even (CVTPS2DQ under the default MXCSR), truncate to i8 (a NaN
 * becomes INT_MIN whose low byte is 0).  Tail: round half away from zero,
 * clamp after, `as i8` (NaN -> 0). */
float or_quantize_avx512(const float* x, int64_t n, int8_t* q) {
    int64_t chunks = n / 16;
    float lane[16];
    for (int j = 0; j < 16; ++j) lane[j] = 0.0f;
    for (int64_t c = 0; c < chunks; ++c)
        for (int j = 0; j < 16; ++j) {
            float v = fabsf(x[c * 16 + j]);
            lane[j] = (lane[j] > v) ? lane[j] : v;
        }
    float max_abs = 0.0f;
    for (int j = 0; j < 16; ++j)
        if (lane[j] > max_abs) max_abs = lane[j];
    for (int64_t i = chunks * 16; i < n; ++i) {
        float v = fabsf(x[i]);
        if (v > max_abs) max_abs = v;
    }
    float scale = (max_abs > 0.0f) ? 127.0f / max_abs : 1.0f;
    float inv_scale = (max_abs > 0.0f) ? max_abs / 127.0f : 1.0f;
    for (int64_t i = 0; i < chunks * 16; ++i) {
        float s = x[i] * scale;
        float t = (127.0f < s) ? 127.0f : s;
        t = (-127.0f > t) ? -127.0f : t;
        q[i] = isnan(t) ? (int8_t)0 : (int8_t)(int)nearbyintf(t);
    }
    for (int64_t i = chunks * 16; i < n; ++i) {
        float r = roundf(x[i] * scale);
        float c = (r > 127.0f) ? 127.0f : (r < -127.0f) ? -127.0f : r;
        q[i] = isnan(c) ? (int8_t)0 : (int8_t)(int)c;
    }
    return inv_scale;
}

/* quantization.rs:179-194 — scalar path: `if |x| > max`, round half away,
 * then Rust max(-127)/min(127) (which map NaN to -127). */
float or_quantize_scalar(const float* x, int64_t n, int8_t* q) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < n; ++i)
        if (fabsf(x[i]) > max_abs) max_abs = fabsf(x[i]);
    float scale = (max_abs > 0.0f) ? 127.0f / max_abs : 1.0f;
    float inv_scale = (max_abs > 0.0f) ? max_abs / 127.0f : 1.0f;
    for (int64_t i = 0; i < n; ++i) {
        float r = roundf(x[i] * scale);
        if (isnan(r)) r = -127.0f;
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        q[i] = (int8_t)(int)r;
    }
    return inv_scale;
}

/* ------------------------------------------------------------------------ */
/* Dot kernels                                                               */
/* ------------------------------------------------------------------------ */

/* simd.rs:372-381 — scalar Pack4 dot, exact i32. */
int32_t or_dot_pack4(const int8_t* a, const uint8_t* w, int64_t n) {
    int32_t acc = 0;
    for (int64_t i = 0; i < n; ++i) {
        unsigned code = (w[i / 4] >> (2 * (i % 4))) & 3u;
        int wt = (code == 0) ? -1 : (code == 2) ? 1 : 0;
        acc += (int32_t)a[i] * wt;
    }
    return acc;
}

/* simd.rs:388-414 — scalar Pack5 dot; a partial last byte decodes only the
 * trits it covers. */
int32_t or_dot_pack5(const int8_t* a, const uint8_t* w, int64_t n) {
    int32_t acc = 0;
    for (int64_t c = 0; c * 5 < n; ++c) {
        unsigned b = w[c];
        for (int j = 0; j < 5 && c * 5 + j < n; ++j) {
            unsigned v = b % 3;
            b /= 3;
            int wt = (v == 0) ? -1 : (v == 2) ? 1 : 0;
            acc += (int32_t)a[c * 5 + j] * wt;
        }
    }
    return acc;
}

/* simd.rs:425-459 — per 64-block: +a where mask & ~sign, -a where mask & sign. */
int32_t or_dot_sparse(const int8_t* a, const uint64_t* masks, const uint64_t* signs,
                      int64_t num_blocks, int64_t in_dim) {
    int32_t acc = 0;
    for (int64_t b = 0; b < num_blocks; ++b) {
        int64_t start = b * 64;
        int64_t end = start + 64 < in_dim ? start + 64 : in_dim;
        uint64_t m = masks[b], s = signs[b];
        for (int64_t i = start; i < end; ++i) {
            int lane = (int)(i - start);
            if ((m >> lane) & 1u) acc += ((s >> lane) & 1u) ? -(int32_t)a[i] : (int32_t)a[i];
        }
    }
    return acc;
}

int or_cpu_has_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
}
int or_cpu_has_avx512f(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f");
}

/* AVX-512 VNNI Pack4 dot, the reference's first-choice kernel
 * (simd.rs:256-356): per 16 packed bytes (64 weights) widen each byte to a
 * 32-bit lane, pull the four 2-bit fields into the four bytes of the lane,
 * map codes through a byte shuffle table (0->-1, 1->0, 2->+1, 3->0), form the
 * signed activation (+a / 0 / -a, computed as 0-a with i8 wrap like the
 * reference), and accumulate with vpdpbusd(acc, 1u8, sa) over 16 independent
 * accumulators; NTA prefetch 256 bytes ahead; scalar tail. */
__attribute__((target("avx512f,avx512bw,avx512vnni")))
int32_t or_dot_pack4_vnni(const int8_t* a, const uint8_t* w, int64_t n) {
    const __m512i zero = _mm512_setzero_si512();
    const __m512i one_u8 = _mm512_set1_epi8(1);
    const __m512i m3 = _mm512_set1_epi32(3);
    /* byte table indexed by the 2-bit code in each 128-bit lane */
    const __m512i table = _mm512_broadcast_i32x4(_mm_setr_epi8(-1, 0, 1, 0, 0, 0, 0, 0,
                                                                0, 0, 0, 0, 0, 0, 0, 0));
    __m512i acc[16];
    for (int k = 0; k < 16; ++k) acc[k] = zero;
    int64_t blocks = n / 64, full = blocks / 16 * 16, b = 0;
#define XT_BLOCK(ACC, IDX)                                                              \
    do {                                                                                \
        __m512i act = _mm512_loadu_si512((const void*)(a + (IDX) * 64));                \
        __m512i wide = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i*)(w + (IDX) * 16))); \
        __m512i f = _mm512_or_si512(                                                    \
            _mm512_or_si512(_mm512_and_si512(wide, m3),                                 \
                            _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(wide, 2), m3), 8)), \
            _mm512_or_si512(_mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(wide, 4), m3), 16), \
                            _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(wide, 6), m3), 24))); \
        __m512i wt = _mm512_shuffle_epi8(table, f);                                     \
        __mmask64 pos = _mm512_cmpgt_epi8_mask(wt, zero);                               \
        __mmask64 nul = _mm512_cmpeq_epi8_mask(wt, zero);                               \
        __m512i sa = _mm512_mask_blend_epi8(pos, _mm512_sub_epi8(zero, act), act);      \
        sa = _mm512_mask_mov_epi8(sa, nul, zero);                                       \
        ACC = _mm512_dpbusd_epi32(ACC, one_u8, sa);                                     \
    } while (0)
    for (; b < full; b += 16) {
        _mm_prefetch((const char*)(w + b * 16 + 256), _MM_HINT_NTA);
        for (int k = 0; k < 16; ++k) XT_BLOCK(acc[k], b + k);
    }
    __m512i sum = acc[0];
    for (int k = 1; k < 16; ++k) sum = _mm512_add_epi32(sum, acc[k]);
    for (; b < blocks; ++b) {
        _mm_prefetch((const char*)(w + b * 16 + 256), _MM_HINT_NTA);
        XT_BLOCK(sum, b);
    }
#undef XT_BLOCK
    int32_t total = _mm512_reduce_add_epi32(sum);
    for (int64_t i = blocks * 64; i < n; ++i) {
        unsigned code = (w[i / 4] >> (2 * (i % 4))) & 3u;
        int wt = (code == 0) ? -1 : (code == 2) ? 1 : 0;
        total += (int32_t)a[i] * wt;
    }
    return total;
}

/* ------------------------------------------------------------------------ */
/* XorSparse codec                                                           */
/* ------------------------------------------------------------------------ */

static uint64_t rd_u64(const uint8_t* p) {
    uint64_t v = 0;
    for (int k = 0; k < 8; ++k) v |= (uint64_t)p[k] << (8 * k);
    return v;
}
static uint32_t rd_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

int64_t or_sparse_row_bytes(const int8_t* vals, int64_t in_dim) {
    int64_t nb = (in_dim + 63) / 64, bytes = 4;
    for (int64_t b = 0; b < nb; ++b) {
        int nnz = 0;
        for (int64_t i = b * 64; i < in_dim && i < b * 64 + 64; ++i) nnz += vals[i] != 0;
        bytes += 8 + (nnz + 7) / 8;
    }
    return bytes;
}

/* sparse.rs:61-86 — u32 num_blocks, then per block u64 mask (bit i: lane i
 * non-zero) and ceil(nnz/8) bytes of set-order sign bits (bit j: j-th
 * non-zero is -1), all little-endian. */
int64_t or_sparse_encode_row(const int8_t* vals, int64_t in_dim, uint8_t* out) {
    int64_t nb = (in_dim + 63) / 64, p = 0;
    for (int k = 0; k < 4; ++k) out[p++] = (uint8_t)((uint64_t)nb >> (8 * k));
    for (int64_t b = 0; b < nb; ++b) {
        uint64_t mask = 0, sgn = 0;
        unsigned si = 0;
        for (int64_t i = b * 64; i < in_dim && i < b * 64 + 64; ++i) {
            if (vals[i] != 0) {
                mask |= 1ull << (i - b * 64);
                if (vals[i] < 0) sgn |= 1ull << si;
                ++si;
            }
        }
        for (int k = 0; k < 8; ++k) out[p++] = (uint8_t)(mask >> (8 * k));
        for (unsigned k = 0; k < (si + 7) / 8; ++k) out[p++] = (uint8_t)(sgn >> (8 * k));
    }
    return p;
}

/* sparse.rs:135-194 — per block: read the mask and ceil(popcnt/8) sign bytes,
 * then scatter the set-order sign bits to the lanes of the mask's set bits. */
int64_t or_sparse_from_blob(const uint8_t* blob, int64_t blob_len, int64_t out_dim,
                            uint64_t* masks, uint64_t* signs, int64_t max_blocks_total) {
    int64_t p = 0, first_nb = 0, w = 0;
    for (int64_t r = 0; r < out_dim; ++r) {
        if (p + 4 > blob_len) return -1;
        int64_t nb = rd_u32(blob + p);
        p += 4;
        if (r == 0) first_nb = nb;
        for (int64_t b = 0; b < nb; ++b) {
            if (p + 8 > blob_len || w >= max_blocks_total) return -1;
            uint64_t mask = rd_u64(blob + p);
            p += 8;
            int nnz = __builtin_popcountll(mask), sbytes = (nnz + 7) / 8;
            if (p + sbytes > blob_len) return -1;
            uint64_t sb = 0;
            for (int k = 0; k < sbytes; ++k) sb |= (uint64_t)blob[p + k] << (8 * k);
            p += sbytes;
            uint64_t lane_sign = 0;
            unsigned si = 0;
            for (int lane = 0; lane < 64; ++lane)
                if ((mask >> lane) & 1u) {
                    if ((sb >> si) & 1u) lane_sign |= 1ull << lane;
                    ++si;
                }
            masks[w] = mask;
            signs[w] = lane_sign;
            ++w;
        }
    }
    return first_nb;
}

/* sparse.rs:207-249 */
void or_sparse_decode_row(const uint8_t* blob, int64_t off, int64_t in_dim, int8_t* out) {
    int64_t nb = rd_u32(blob + off), p = off + 4;
    memset(out, 0, (size_t)in_dim);
    for (int64_t b = 0; b < nb; ++b) {
        uint64_t mask = rd_u64(blob + p);
        p += 8;
        int nnz = __builtin_popcountll(mask), sbytes = (nnz + 7) / 8;
        uint64_t sb = 0;
        for (int k = 0; k < sbytes; ++k) sb |= (uint64_t)blob[p + k] << (8 * k);
        p += sbytes;
        unsigned si = 0;
        for (int64_t i = b * 64; i < in_dim && i < b * 64 + 64; ++i)
            if ((mask >> (i - b * 64)) & 1u) {
                out[i] = ((sb >> si) & 1u) ? -1 : 1;
                ++si;
            }
    }
}

/* ------------------------------------------------------------------------ */
/* TernaryLinear forward                                                     */
/* ------------------------------------------------------------------------ */

/* layers.rs:216-231 — TernaryLinear::dot_row. */
static int32_t dot_row(int fmt, const uint8_t* wbytes, const uint64_t* masks,
                       const uint64_t* signs, int64_t K, int64_t o, const int8_t* q,
                       int kernel) {
    if (fmt == 0) {
        const uint8_t* row = wbytes + o * ((K + 3) / 4);
        return kernel ? or_dot_pack4_vnni(q, row, K) : or_dot_pack4(q, row, K);
    }
    if (fmt == 1) return or_dot_pack5(q, wbytes + o * ((K + 4) / 5), K);
    int64_t nb = (K + 63) / 64;
    return or_dot_sparse(q, masks + o * nb, signs + o * nb, nb, K);
}

/* src/lib.rs:25-46: 0 threads -> min(available_parallelism, 8). */
static int resolve_threads(int threads) {
    if (threads > 0) return threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    return n < 8 ? (int)n : 8;
}

/* layers.rs:262-313.  M == 1: quantise once on the calling thread, then
 * parallel chunks of max(ceil(N/T), 128) output rows.  M > 1: one task per
 * token; each quantises its own row and runs all N rows serially. */
void or_linear_forward(int fmt, const uint8_t* wbytes, const uint64_t* masks,
                       const uint64_t* signs, const float* w_scales, int64_t K, int64_t N,
                       const float* x, int64_t M, float* y, int8_t* q, float* inv,
                       int32_t* acc, int quant_mode, int threads, int kernel) {
    int T = resolve_threads(threads);
    if (kernel && !(fmt == 0 && or_cpu_has_vnni())) kernel = 0;
    if (M == 1) {
        float s = quant_mode ? or_quantize_scalar(x, K, q) : or_quantize_avx512(x, K, q);
        if (inv) inv[0] = s;
        int64_t chunk = (N + T - 1) / T;
        if (chunk < 128) chunk = 128;
        int64_t nchunks = (N + chunk - 1) / chunk;
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
        for (int64_t c = 0; c < nchunks; ++c) {
            int64_t end = (c + 1) * chunk < N ? (c + 1) * chunk : N;
            for (int64_t o = c * chunk; o < end; ++o) {
                int32_t d = dot_row(fmt, wbytes, masks, signs, K, o, q, kernel);
                if (acc) acc[o] = d;
                float t = (float)d * s;
                y[o] = t * w_scales[o];
            }
        }
        return;
    }
#pragma omp parallel for num_threads(T) schedule(dynamic, 1)
    for (int64_t m = 0; m < M; ++m) {
        int8_t* qm = q + m * K;
        float s = quant_mode ? or_quantize_scalar(x + m * K, K, qm)
                             : or_quantize_avx512(x + m * K, K, qm);
        if (inv) inv[m] = s;
        for (int64_t o = 0; o < N; ++o) {
            int32_t d = dot_row(fmt, wbytes, masks, signs, K, o, qm, kernel);
            if (acc) acc[m * N + o] = d;
            float t = (float)d * s;
            y[m * N + o] = t * w_scales[o];
        }
    }
}

/* layers.rs:315-345 applied row by row. */
void or_linear_forward_q(int fmt, const uint8_t* wbytes, const uint64_t* masks,
                         const uint64_t* signs, const float* w_scales, int64_t K, int64_t N,
                         const int8_t* q, const float* inv, int64_t M, float* y,
                         int32_t* acc) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t o = 0; o < N; ++o) {
            int32_t d = dot_row(fmt, wbytes, masks, signs, K, o, q + m * K, 0);
            if (acc) acc[m * N + o] = d;
            float t = (float)d * inv[m];
            y[m * N + o] = t * w_scales[o];
        }
}

/* loader/mod.rs:355-389: unpack the whole stored stream linearly
 * (unpack_1_58bit_{4,5}pack), scatter value k to row j*stored_rows + p,
 * column i (byte k/f = p*in_dim + i, j = k % f), then pack each row at
 * scale 1.0. */
int or_hf_destripe(int fmt, int64_t in_dim, int64_t out_dim, const uint8_t* stored,
                   uint8_t* out_packed) {
    const int64_t f = fmt == 1 ? 5 : 4;
    if (out_dim % f) return -1;
    const int64_t n = in_dim * out_dim, stored_rows = out_dim / f;
    float* flat = (float*)malloc((size_t)n * sizeof(float));
    float* rows = (float*)malloc((size_t)n * sizeof(float));
    if (!flat || !rows) {
        free(flat);
        free(rows);
        return -1;
    }
    if (fmt == 1) or_unpack5(stored, n, flat);
    else or_unpack4(stored, n, flat);
    for (int64_t k = 0; k < n; ++k) {
        const int64_t byte_idx = k / f, j = k % f;
        const int64_t row_p = byte_idx / in_dim, col = byte_idx % in_dim;
        rows[(j * stored_rows + row_p) * in_dim + col] = flat[k];
    }
    const int64_t bpr = (in_dim + f - 1) / f;
    for (int64_t o = 0; o < out_dim; ++o) {
        if (fmt == 1) or_pack5(rows + o * in_dim, in_dim, 1.0f, out_packed + o * bpr);
        else or_pack4(rows + o * in_dim, in_dim, 1.0f, out_packed + o * bpr);
    }
    free(flat);
    free(rows);
    return 0;
}

static inline float silu_scalar(float g, float u) {
    /* quantization.rs:213 / :280: g * (1.0 / (1.0 + (-g).exp())) * u */
    const float e = expf(-g);
    const float sig = 1.0f / (1.0f + e);
    const float a = g * sig;
    return a * u;
}

static inline float relu2_mul(float g, float u) {
    /* :215-216 / :282-283 and tensor.rs:223-224: r = max(g, 0); r * r * u.
     * MAXPS(g, 0) returns 0 for NaN g, as does Rust's f32::max. */
    const float r = (g > 0.0f) ? g : 0.0f;
    const float rr = r * r;
    return rr * u;
}

/* One lane of silu_inplace_avx512's vector body (quantization.rs:243-272):
 * MINPS/MAXPS return their second operand unless the comparison holds
 * (so NaN clamps to the bound), ROUNDSCALE imm 0 rounds half to even,
 * the polynomial uses fused multiply-adds, 2^n is built from the bits
 * ((n + 127) << 23) with 32-bit wrap, and 1 / (1 + e) is an IEEE division. */
static inline float silu_avx512_lane(float g, float u) {
    const float inv_ln2 = 1.44269504088896341f, ln2 = 0.693147180559945309f;
    const float hi = 88.3762626647949f, lo = -88.3762626647949f;
    float x = 0.0f - g;
    x = (x < hi) ? x : hi;
    x = (x > lo) ? x : lo;
    const float fx = x * inv_ln2;
    const float n_f = nearbyintf(fx); /* default rounding mode: to nearest even */
    const float t = x - n_f * ln2;
    float e = fmaf(1.0f / 24.0f, t, 1.0f / 6.0f);
    e = fmaf(e, t, 0.5f);
    e = fmaf(e, t, 1.0f);
    e = fmaf(e, t, 1.0f);
    const int32_t ni = (int32_t)n_f; /* n_f is integral and in [-128, 128] */
    const uint32_t bits = ((uint32_t)ni + 127u) << 23;
    float pow2n;
    memcpy(&pow2n, &bits, 4);
    const float exp_x = e * pow2n;
    const float sig = 1.0f / (1.0f + exp_x);
    const float act = g * sig;
    return act * u;
}

void or_silu_inplace(float* gate, const float* up, int64_t n, int use_silu, int avx512) {
    const int64_t nmain = avx512 ? (n / 16) * 16 : 0;
    for (int64_t i = 0; i < n; ++i) {
        const float g = gate[i], u = up[i];
        if (!use_silu) gate[i] = relu2_mul(g, u);
        else gate[i] = i < nmain ? silu_avx512_lane(g, u) : silu_scalar(g, u);
    }
}

void or_act_mul_inplace(float* x, const float* up, int64_t n, int use_silu) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = x[i], u = up[i];
        if (use_silu) {
            const float d = 1.0f + expf(-g);
            const float s = g / d;
            x[i] = s * u;
        } else {
            x[i] = relu2_mul(g, u);
        }
    }
}

float or_rms_norm(float* x, const float* w, int64_t n, float eps) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float sq = x[i] * x[i];
        sum += sq;
    }
    const float rms = sqrtf(sum / (float)n + eps);
    const float inv = 1.0f / rms;
    for (int64_t i = 0; i < n; ++i) {
        const float a = x[i] * inv;
        x[i] = a * w[i];
    }
    return sum;
}

void or_int_new(int bits, const float* w, int64_t N, int64_t K, uint8_t* out, float* scales) {
    const float qmax = bits == 8 ? 127.0f : 7.0f;
    const float lo = bits == 8 ? -127.0f : -8.0f, hi = bits == 8 ? 127.0f : 7.0f;
    const int64_t bpr = bits == 8 ? K : (K + 1) / 2;
    for (int64_t o = 0; o < N; ++o) {
        const float* row = w + o * K;
        float mx = 0.0f; /* row.iter().map(abs).fold(0.0, f32::max) */
        for (int64_t k = 0; k < K; ++k) mx = fmaxf(mx, fabsf(row[k]));
        const float scale = mx > 0.0f ? mx / qmax : 1.0f;
        scales[o] = scale;
        for (int64_t c = 0; c < bpr; ++c) {
            int q[2];
            const int per = bits == 8 ? 1 : 2;
            for (int t = 0; t < per; ++t) {
                const int64_t k = c * per + t;
                const float v = k < K ? row[k] : 0.0f;
                float r = roundf(v / scale);
                r = fmaxf(r, lo); /* Rust max: NaN -> lo */
                r = fminf(r, hi);
                q[t] = (int)r;
            }
            out[o * bpr + c] = bits == 8 ? (uint8_t)(int8_t)q[0]
                                         : (uint8_t)(((unsigned)q[0] & 15u) | ((unsigned)q[1] << 4));
        }
    }
}

void or_int_forward(int bits, const uint8_t* wbytes, const float* scales, int64_t K, int64_t N,
                    const float* x, int64_t M, float* y, int32_t* acc, int quant_mode) {
    int8_t* q = (int8_t*)malloc((size_t)K);
    const int64_t bpr = bits == 8 ? K : (K + 1) / 2;
    for (int64_t m = 0; m < M; ++m) {
        const float inv = quant_mode == 1 ? or_quantize_scalar(x + m * K, K, q)
                                          : or_quantize_avx512(x + m * K, K, q);
        for (int64_t o = 0; o < N; ++o) {
            const uint8_t* wr = wbytes + o * bpr;
            int32_t dot = 0;
            if (bits == 8) {
                for (int64_t k = 0; k < K; ++k) dot += (int32_t)q[k] * (int32_t)(int8_t)wr[k];
            } else {
                for (int64_t c = 0; c < K / 2; ++c) { /* zip with chunks_exact(2) */
                    const int q0 = (int8_t)(uint8_t)(wr[c] << 4) >> 4;
                    const int q1 = (int8_t)(wr[c] & 0xF0) >> 4;
                    dot += (int32_t)q[2 * c] * q0 + (int32_t)q[2 * c + 1] * q1;
                }
            }
            if (acc) acc[m * N + o] = dot;
            const float a = (float)dot * inv;
            y[m * N + o] = a * scales[o];
        }
    }
    free(q);
}

/* simd.rs:556-565: x = x*6364136223846793005 + 1442695040888963407; x >> 33. */
uint64_t or_lcg_next(uint64_t* state) {
    *state = *state * 6364136223846793005ull + 1442695040888963407ull;
    return *state >> 33;
}
