/*
 * xtern oracle — CPU restatement of xor-net's ternary linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path and the timed CPU baseline ("port") in bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (libxtern) never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the xor-net source tree).  All functions are plain C with explicit-width
 * integer types; sizes are int64_t element counts.
 */
#ifndef XTERN_ORACLE_H
#define XTERN_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Pack4 / Pack5 codecs: src/bit1_58/quantization.rs:7-91 ---- */
void or_pack4(const float* w, int64_t n, float w_scale, uint8_t* out);      /* :7-27  */
void or_unpack4(const uint8_t* packed, int64_t n, float* out);             /* :29-46 */
void or_pack5(const float* w, int64_t n, float w_scale, uint8_t* out);      /* :48-70 */
void or_unpack5(const uint8_t* packed, int64_t n, float* out);             /* :72-91 */

/* ---- activation quantiser: src/bit1_58/quantization.rs:95-195 ----
 * or_quantize_avx512 restates the AVX-512F path (:95-145): lanes below
 * floor(n/16)*16 are clamped to [-127,127] and then rounded half-to-even, the
 * tail is rounded half-away-from-zero and clamped after.  or_quantize_scalar
 * restates the non-AVX-512 path (:179-194).  Both return inv_scale. */
float or_quantize_avx512(const float* x, int64_t n, int8_t* q);
float or_quantize_scalar(const float* x, int64_t n, int8_t* q);

/* ---- dot kernels: src/bit1_58/simd.rs ---- */
int32_t or_dot_pack4(const int8_t* a, const uint8_t* w, int64_t n);         /* :372-381 scalar */
int32_t or_dot_pack5(const int8_t* a, const uint8_t* w, int64_t n);         /* :388-414 */
int32_t or_dot_sparse(const int8_t* a, const uint64_t* masks, const uint64_t* signs,
                      int64_t num_blocks, int64_t in_dim);                  /* :425-459 */
/* AVX-512 VNNI restatement of simd.rs:256-356 (the reference's dispatch-first
 * kernel).  Returns the same value as or_dot_pack4 for every valid input.
 * Only callable when or_cpu_has_vnni() is true. */
int32_t or_dot_pack4_vnni(const int8_t* a, const uint8_t* w, int64_t n);
int or_cpu_has_vnni(void);
int or_cpu_has_avx512f(void);

/* ---- XorSparse codec: src/bit1_58/sparse.rs ---- */
/* Bytes the row encoding of one ternary row takes (sparse.rs:61-86). */
int64_t or_sparse_row_bytes(const int8_t* vals, int64_t in_dim);
/* Encode one row, returns bytes written (sparse.rs:61-86). */
int64_t or_sparse_encode_row(const int8_t* vals, int64_t in_dim, uint8_t* out);
/* Walk the blob and produce lane-order masks/signs, [out_dim][num_blocks]
 * (sparse.rs:135-194).  Returns num_blocks of the first row, or -1 when the
 * blob is shorter than its own headers claim. */
int64_t or_sparse_from_blob(const uint8_t* blob, int64_t blob_len, int64_t out_dim,
                            uint64_t* masks, uint64_t* signs, int64_t max_blocks_total);
/* Decode one row starting at byte offset `off` to {-1,0,1} (sparse.rs:207-249). */
void or_sparse_decode_row(const uint8_t* blob, int64_t off, int64_t in_dim, int8_t* out);

/* ---- TernaryLinear::forward: src/bit1_58/layers.rs:262-313 ----
 * fmt: 0 = Pack4, 1 = Pack5 (dense bytes [N][bpr]); 2 = XorSparse (lane-order
 * masks/signs [N][nb]).  y[m*N+o] = (float)dot * inv_scale[m] * w_scales[o]
 * with two separately rounded f32 multiplies.  q (M*K) / inv (M) / acc (M*N)
 * receive the quantised activations, the per-row inverse scales and the i32
 * dot products when non-NULL.  quant_mode 0 = AVX-512 semantics, 1 = scalar.
 * threads: 0 = the reference default min(nproc, 8) (src/lib.rs:25-46);
 * kernel: 0 = scalar dots, 1 = the VNNI Pack4 dot (fmt 0 only). */
void or_linear_forward(int fmt, const uint8_t* wbytes, const uint64_t* masks,
                       const uint64_t* signs, const float* w_scales,
                       int64_t K, int64_t N, const float* x, int64_t M, float* y,
                       int8_t* q, float* inv, int32_t* acc, int quant_mode,
                       int threads, int kernel);

/* TernaryLinear::forward_with_quantized (layers.rs:315-345), for every row m
 * of an [M][K] i8 input with per-row inv_scale. */
void or_linear_forward_q(int fmt, const uint8_t* wbytes, const uint64_t* masks,
                         const uint64_t* signs, const float* w_scales, int64_t K,
                         int64_t N, const int8_t* q, const float* inv, int64_t M,
                         float* y, int32_t* acc);

/* ---- HF prepacked weights: src/loader/mod.rs:301-394 ----
 * `stored` is the checkpoint's U8 tensor [out_dim/f][in_dim] (f = 4 for Pack4,
 * 5 for Pack5) whose byte [p][i] holds output rows j*(out_dim/f) + p for
 * j < f.  Writes the input-dim packed rows get_prepacked_ternary returns
 * ([out_dim][ceil(in_dim/f)] bytes, packed at scale 1.0).  Returns 0, or -1
 * when out_dim is not a multiple of f. */
int or_hf_destripe(int fmt, int64_t in_dim, int64_t out_dim, const uint8_t* stored,
                   uint8_t* out_packed);

/* ---- MLP activations and RMSNorm ----
 * or_silu_inplace: quantization::silu_inplace (src/bit1_58/quantization.rs:
 * 201-286), the activation of the fused MLP (layers.rs:563).  gate[i] becomes
 * silu(gate)*up or relu(gate)^2*up.  avx512 != 0 restates the AVX-512F path
 * (:225-286: lanes below floor(n/16)*16 take the vectorised exp polynomial,
 * the tail takes the scalar formula), avx512 == 0 the portable path
 * (:208-218).  The scalar formula is g * (1 / (1 + expf(-g))) * u with the C
 * library's expf, as Rust's f32::exp calls it. */
void or_silu_inplace(float* gate, const float* up, int64_t n, int use_silu, int avx512);
/* FastTensor::silu_mul_inplace / relu2_mul_inplace (src/tensor.rs:170-238),
 * the activation of the unfused MLP (models/llama/mlp.rs:118-121):
 * (x / (1 + expf(-x))) * u, or relu(x)^2 * u. */
void or_act_mul_inplace(float* x, const float* up, int64_t n, int use_silu);
/* rms_norm (src/nn/fast_attention_simd.rs:458-516; every ISA path sums x*x
 * sequentially in index order): rms = sqrtf(sum / n + eps), inv = 1 / rms,
 * x[i] = x[i] * inv * w[i].  In place.  Returns sum. */
float or_rms_norm(float* x, const float* w, int64_t n, float eps);

/* ---- Int8 / Int4 LM head: src/nn/dynamic_linear.rs:229-535 ----
 * or_int_new: Int8Linear::new (bits 8, :236-258) / Int4Linear::new (bits 4,
 * :389-410): per row scale = max|w| / 127 (/ 7), 1.0 for a zero row;
 * q = round(w / scale) clamped; writes [N][K] i8 or [N][ceil(K/2)] nibbles.
 * or_int_forward: Int8Linear::forward / Int4Linear::forward (:260-375,
 * :412-535): per row absmax quantisation (quant_mode as or_linear_forward),
 * exact i32 dot (Int4: bytes paired with chunks_exact(2) of the activations,
 * so an odd in_dim's last column is skipped), y = (f32)dot * inv * scale[o].
 * acc (nullable) receives the dots. */
void or_int_new(int bits, const float* w, int64_t N, int64_t K, uint8_t* out, float* scales);
void or_int_forward(int bits, const uint8_t* wbytes, const float* scales, int64_t K, int64_t N,
                    const float* x, int64_t M, float* y, int32_t* acc, int quant_mode);

/* ---- the reference's deterministic test RNG: simd.rs:556-565 ---- */
uint64_t or_lcg_next(uint64_t* state);

#ifdef __cplusplus
}
#endif
#endif
