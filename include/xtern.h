/*
 * xtern — MI355X (gfx950) ternary linear-layer library, C ABI.
 *
 * This header is the drop-in boundary for xor-net's bit1_58 ternary linear
 * path.  Every entry point is plain C: plain pointers and sizes, no exceptions
 * cross it, every call returns an int status (XT_OK = 0, negative = error) and
 * leaves a thread-local message readable with xt_last_error().
 *
 * Device pointers are HIP device pointers on the current device; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  All compute calls
 * are asynchronous on `stream`; the library only synchronises inside
 * xt_weights_create / xt_weights_destroy / xt_workspace_release.
 *
 * Threads: every call may be made from several host threads at once, also
 * on one shared stream and with one shared weight handle (the reference's
 * forward(&self) is shared across threads through Arc).  The device
 * workspaces of the f32 entry points belong to one (device, stream, host
 * thread) each, so concurrent callers never share one; a workspace that has
 * to grow is replaced, and the old one is kept (not freed) until
 * xt_workspace_release, because queued launches or a captured HIP graph may
 * still use it.
 *
 * HIP graphs: the compute calls can be captured.  No call allocates,
 * synchronises or clears memory while its stream is being captured: a call
 * whose workspace would have to grow fails with XT_ERR_UNSUPPORTED instead.
 * Make one eager call of the largest shape on the capturing stream and
 * thread first.  A graph uses the workspace of the thread and stream it was
 * captured on; replay it on that stream, or order it against eager calls of
 * that thread on that stream.
 *
 * Reference paths below are relative to the xor-net source tree.
 */
#ifndef XTERN_H
#define XTERN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    XT_OK = 0,
    XT_ERR_INVALID = -1,     /* bad argument / shape (reference: anyhow::bail!) */
    XT_ERR_HIP = -2,         /* a HIP runtime call failed */
    XT_ERR_NOMEM = -3,       /* device or host allocation failed */
    XT_ERR_UNSUPPORTED = -4  /* valid request this build does not handle */
};

/* Weight storage formats.  Values match the on-disk/host byte layouts the
 * reference keeps:
 *   XT_PACK4     TernaryPackType::Pack4, [out_dim][ceil(in_dim/4)] bytes,
 *                2-bit codes 00=-1 01=0 10=+1 (11 reads as 0)
 *                (src/bit1_58/quantization.rs:7-46)
 *   XT_PACK5     TernaryPackType::Pack5, [out_dim][ceil(in_dim/5)] bytes,
 *                base-3 digits 0=-1 1=0 2=+1, first weight least significant
 *                (src/bit1_58/quantization.rs:48-91)
 *   XT_XORSPARSE the XorSparse row blob: per row u32 num_blocks, then per
 *                64-block u64 mask + ceil(popcount/8) set-order sign bytes
 *                (src/bit1_58/sparse.rs:9-17, :61-86)                        */
/*   XT_INT8      Int8Linear::weight_i8, [out_dim][in_dim] i8 with per-row
 *                scales (src/nn/dynamic_linear.rs:229-258)
 *   XT_INT4      Int4Linear::weight_i4, [out_dim][ceil(in_dim/2)] bytes, two
 *                two's-complement nibbles per byte, column 2c low
 *                (dynamic_linear.rs:382-410).  As in Int4Linear's dot, the
 *                last column of an odd in_dim contributes nothing. */
/*   XT_XORSPARSE_STREAM  the same XorSparse row blob as XT_XORSPARSE, kept
 *                on the device in its compact form (block masks and set-order
 *                sign bits, no expansion to 2-bit tiles): products read about
 *                0.77x the tile bytes and expand the signs in registers.
 *                in_dim up to 16384; products only (not the fused MLP or the
 *                decode stack). */
enum { XT_PACK4 = 0, XT_PACK5 = 1, XT_XORSPARSE = 2, XT_INT8 = 3, XT_INT4 = 4,
       XT_XORSPARSE_STREAM = 5 };

/* Activation rounding: which of the reference's two quantiser paths to
 * reproduce bit for bit (src/bit1_58/quantization.rs:170-195).
 *   XT_QUANT_AVX512  the path taken on AVX-512F hosts (:95-145): clamp then
 *                    round half to even for the first floor(K/16)*16 lanes,
 *                    round half away from zero for the tail.
 *   XT_QUANT_SCALAR  the portable path (:179-194): round half away, clamp. */
enum { XT_QUANT_AVX512 = 0, XT_QUANT_SCALAR = 1 };

/* Elementwise activations of the MLP, each reproducing one reference
 * function bit for bit (out = act(gate) * up):
 *   XT_ACT_RELU2_MUL            max(g, 0)^2 * u (quantization.rs:215-216,
 *                               tensor.rs:206-238)
 *   XT_ACT_SILU_INPLACE_AVX512  silu_inplace on an AVX-512F host
 *                               (quantization.rs:225-286): exp polynomial for
 *                               the first floor(n/16)*16 lanes of each row,
 *                               g * (1 / (1 + expf(-g))) * u for the tail
 *   XT_ACT_SILU_INPLACE_SCALAR  silu_inplace elsewhere (:208-218)
 *   XT_ACT_SILU_MUL             FastTensor::silu_mul_inplace
 *                               (tensor.rs:170-204): (g / (1 + expf(-g))) * u
 * expf is the C library's (glibc) expf, reproduced exactly. */
enum {
    XT_ACT_RELU2_MUL = 0,
    XT_ACT_SILU_INPLACE_AVX512 = 1,
    XT_ACT_SILU_INPLACE_SCALAR = 2,
    XT_ACT_SILU_MUL = 3
};

/* Opaque device-resident weights: the packed ternary matrix in the GPU tile
 * layout plus the per-output-row f32 scales.  Owns its device memory.
 * Replaces TernaryLinear { rep, in_dim, out_dim, pack_type, w_scales }
 * (src/bit1_58/layers.rs:34-41, TernaryRep :23-27). */
typedef struct xt_weights xt_weights;

/* Library version string. */
const char* xt_version(void);

/* Message for the last failed call on this host thread ("" if none). */
const char* xt_last_error(void);

/* Upload packed weights.  `host_bytes`/`nbytes` hold the matrix in `fmt`'s
 * host layout (see the enum above); `w_scales` holds out_dim floats (one per
 * output row, as TernaryLinear::w_scales).  The bytes are repacked once into
 * the device tile layout on the calling thread and copied to the current
 * device.  XT_INT8 / XT_INT4 handles (the LM head's Int8Linear / Int4Linear)
 * work with the same product entry points (xt_ternary_linear_q / _f32),
 * computing (f32)dot_i32 * inv_scale * scale[o] as Int8Linear::forward /
 * Int4Linear::forward do (dynamic_linear.rs:260-375, :412-535).  Replaces DynamicLinear::new_ternary_direct
 * (src/nn/dynamic_linear.rs:670-680), TernaryLinear::new_sparse_from_packed
 * (src/bit1_58/layers.rs:183-210) and, for XT_XORSPARSE,
 * SparseTernary::from_blob (src/bit1_58/sparse.rs:135-194). */
int xt_weights_create(int fmt, int64_t in_dim, int64_t out_dim, const void* host_bytes,
                      size_t nbytes, const float* w_scales, xt_weights** out);

/* HF prepacked checkpoints (U8, output-dim striped): `stored` holds the
 * [out_dim/f][in_dim] bytes of the safetensors tensor, f = 4 (XT_PACK4) or
 * 5 (XT_PACK5); digit j of byte [p][i] is the weight of output row
 * j*(out_dim/f) + p at input column i.
 *
 * xt_hf_destripe writes the input-dim packed rows, out_dim * ceil(in_dim/f)
 * bytes, byte-identical to what get_prepacked_ternary returns
 * (src/loader/mod.rs:301-394, the unpack/transpose/repack of :351-390), so
 * they can be passed to xt_weights_create or kept on the host.
 *
 * xt_weights_create_hf uploads the striped bytes and builds the device tiles
 * on the GPU (no host transpose); w_scales are out_dim copies of
 * `weight_scale`, or of 1.0f / weight_scale when is_inverted_scale != 0
 * (:340-347, :392).  Together with xt_weights_create it replaces the
 * get_prepacked_ternary -> DynamicLinear::new_ternary_direct chain of
 * DynamicLinear::load (src/nn/dynamic_linear.rs:729-741).  Both reject a byte
 * count other than in_dim * out_dim / f, or out_dim not a multiple of f, as
 * the loader's is_packed check does (:324-331). */
int xt_hf_destripe(int fmt, int64_t in_dim, int64_t out_dim, const void* stored, size_t nbytes,
                   void* packed_out);
int xt_weights_create_hf(int fmt, int64_t in_dim, int64_t out_dim, const void* stored,
                         size_t nbytes, float weight_scale, int is_inverted_scale,
                         xt_weights** out);

/* ---- XorSparse container ("XORSPARE1", SPARSE_FORMAT.md:30-50) ----
 * Layout as SparseFile::serialize writes it (src/loader/sparse_loader.rs:
 * 124-139): magic "XORSPARE1" (9 bytes), version u32 = 1 at byte 9,
 * num_tensors u32 at byte 13, then per tensor name_len u32, name, out_dim
 * u32, in_dim u32, w_scale f32, blob_len u32, blob (XorSparse row blobs).
 * The reference's reader reads the version at byte 8 and so rejects every
 * file; these entry points read what the writer writes. */
typedef struct xt_sparse_file xt_sparse_file;

/* Parse a container held in memory (copied; the caller may free `data`).
 * Replaces SparseFile::from_bytes / open (sparse_loader.rs:41-104); every
 * length is bounds-checked.  A repeated name resolves to its last entry, as
 * the reference's HashMap insert does. */
int xt_sparse_file_open(const void* data, size_t len, xt_sparse_file** out);
int xt_sparse_file_close(xt_sparse_file* f);
int xt_sparse_file_count(const xt_sparse_file* f, int64_t* n);
/* Directory entry `idx`; the name and blob pointers stay valid until close. */
int xt_sparse_file_entry(const xt_sparse_file* f, int64_t idx, const char** name, int64_t* out_dim,
                         int64_t* in_dim, float* w_scale, const void** blob, size_t* blob_len);
int xt_sparse_file_find(const xt_sparse_file* f, const char* name, int64_t* idx);
/* SparseFile::get_sparse (sparse_loader.rs:106-122) plus the sparse arm of
 * DynamicLinear::load (src/nn/dynamic_linear.rs:697-716): shape check with
 * the reference's message, w_scales = out_dim copies of the entry's scale,
 * upload as XT_XORSPARSE. */
int xt_weights_create_from_sparse_file(const xt_sparse_file* f, const char* name, int64_t in_dim,
                                       int64_t out_dim, xt_weights** out);
/* SparseFile::serialize (sparse_loader.rs:124-139) into `out`; the size is
 * xt_sparse_file_serialized_size(n, names, blob_lens) (0 on bad input). */
size_t xt_sparse_file_serialized_size(int64_t n, const char* const* names, const size_t* blob_lens);
int xt_sparse_file_serialize(int64_t n, const char* const* names, const int64_t* out_dims,
                             const int64_t* in_dims, const float* w_scales,
                             const void* const* blobs, const size_t* blob_lens, void* out,
                             size_t out_len);
/* The per-tensor step of convert_sparse (src/bin/convert_sparse.rs:86-126):
 * HF striped U8 bytes [out_dim/f][in_dim] -> XorSparse row blob
 * (encode_sparse_tensor, src/bit1_58/sparse.rs:61-103).  destripe != 0 maps
 * rows as get_prepacked_ternary does (row j*(out_dim/f) + p from digit j of
 * byte [p][i]), so the blob's rows are the engine's dense rows; destripe == 0
 * reproduces the reference converter, which unpacks the bytes linearly
 * (convert_sparse.rs:104) and so permutes the rows.  *blob_len receives the
 * size; with blob_out NULL nothing else is written. */
int xt_hf_to_sparse_blob(int fmt, int64_t in_dim, int64_t out_dim, const void* stored,
                         size_t nbytes, int destripe, void* blob_out, size_t cap,
                         size_t* blob_len);

/* Copy a handle's device tiles (xt_tile_bytes() bytes) to host memory, after
 * waiting for the device.  No reference counterpart: lets tests compare
 * tiles built on the device with xt_repack_host's. */
int xt_weights_read_tiles(const xt_weights* w, void* host_out, size_t nbytes);

/* Int8Linear::new (bits = 8, dynamic_linear.rs:236-258) / Int4Linear::new
 * (bits = 4, :389-410) on the host: per output row scale = absmax / 127
 * (or / 7; 1.0 for an all-zero row) and q = round(w / scale) clamped to
 * [-127, 127] ([-8, 7]).  `out` receives out_dim * in_dim (Int8) or
 * out_dim * ceil(in_dim / 2) (Int4) bytes in the XT_INT8 / XT_INT4 host
 * layout, `scales` out_dim floats. */
int xt_int_quantize_host(int bits, const float* w, int64_t out_dim, int64_t in_dim, void* out,
                         float* scales);

/* Free every device workspace the library holds (live and retired), after
 * waiting for the current device.  No reference counterpart.  The caller
 * guarantees that no captured graph using them is replayed afterwards; later
 * calls allocate new workspaces. */
int xt_workspace_release(void);

/* Free a handle (NULL is a no-op).  Waits for the device first. */
int xt_weights_destroy(xt_weights* w);

/* Shape / format / device-footprint queries. */
int xt_weights_info(const xt_weights* w, int* fmt, int64_t* in_dim, int64_t* out_dim,
                    size_t* device_bytes);

/* Host-side repack into the device tile layout, exposed so the layout can be
 * checked (or precomputed) without a GPU.  Writes xt_tile_bytes() bytes. */
size_t xt_tile_bytes(int fmt, int64_t in_dim, int64_t out_dim);
int xt_repack_host(int fmt, int64_t in_dim, int64_t out_dim, const void* host_bytes,
                   size_t nbytes, void* tiles_out);

/* The device layout of XT_XORSPARSE_STREAM weights, built on the host (no
 * GPU): *len = its size; with out (cap >= *len) the bytes, and sections[3]
 * = byte offsets of the segment offsets (u32 [ceil(out/16)][ceil(in/64)]:
 * bit offset of each 16-row group's block in the sign stream), the masks
 * (u64 [group][block][16 rows], rows past out_dim 0) and the sign stream
 * (u32 words; per group and block the 16 rows' set-order sign bits in row
 * order, bit 1 = negative).  No reference counterpart: lets tests check the
 * layout without a GPU. */
int xt_xorsparse_stream_host(int64_t in_dim, int64_t out_dim, const void* blob, size_t nbytes,
                             void* out, size_t cap, size_t* len, uint64_t* sections);

/* Per-row absmax quantisation of x [M][K] f32 (device) into q [M][K] i8 and
 * inv_scale [M] f32 (device).  Bit-exact with quantize_f32_to_i8
 * (src/bit1_58/quantization.rs:170-195) in the selected rounding mode. */
int xt_quantize_i8(const float* x, int64_t M, int64_t K, int8_t* q, float* inv_scale,
                   int mode, void* stream);

/* xt_quantize_i8 that also writes rowsum [M] i32 = sum_k q[m][k] (nullable).
 * No reference counterpart: the row sums let xt_ternary_linear_q_rowsum skip
 * its own summing pass when one quantised input feeds several products. */
int xt_quantize_i8_rowsum(const float* x, int64_t M, int64_t K, int8_t* q, float* inv_scale,
                          int32_t* rowsum, int mode, void* stream);

/* y[M][out_dim] = (f32)dot_i32(q[m], row o) * inv_scale[m] * w_scales[o]
 * given already-quantised activations q [M][in_dim] i8 and inv_scale [M].
 * `acc` (nullable, [M][out_dim] i32) receives the exact i32 dot products.
 * Replaces TernaryLinear::forward_with_quantized (src/bit1_58/layers.rs:315-345)
 * — which the reference only defines for one row — for any M. */
int xt_ternary_linear_q(const xt_weights* w, const int8_t* q, const float* inv_scale,
                        int64_t M, float* y, int32_t* acc, void* stream);

/* xt_ternary_linear_q with caller-provided exact row sums of q (from
 * xt_quantize_i8_rowsum).  No reference counterpart; a wrong rowsum gives
 * wrong outputs (it is subtracted from the code-domain dot product). */
int xt_ternary_linear_q_rowsum(const xt_weights* w, const int8_t* q, const float* inv_scale,
                               const int32_t* rowsum, int64_t M, float* y, int32_t* acc,
                               void* stream);

/* Full forward: quantise x [M][in_dim] f32 per row (mode as above), then the
 * ternary product, y [M][out_dim] f32.  Replaces TernaryLinear::forward
 * (src/bit1_58/layers.rs:262-313) and DynamicLinear::forward's Ternary arm
 * (src/nn/dynamic_linear.rs:625-633).  Uses a per-stream device workspace
 * owned by the library. */
int xt_ternary_linear_f32(const xt_weights* w, const float* x, int64_t M, float* y,
                          int mode, void* stream);

/* xt_ternary_linear_f32 without any device allocation: no reference
 * counterpart.  For callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * quantised rows go to a static device scratch of 8 MiB per GPU (held until
 * the process ends) instead of a workspace: A + 2 * B bytes must fit, with
 * A = M * ceil(in_dim / chunk) * chunk (chunk = 256, Pack5 320) and B = 4 * M,
 * each rounded up to a multiple of 256, or the call fails with
 * XT_ERR_INVALID.  A forced split-K configuration (XTERN_CONFIG) fails with
 * XT_ERR_UNSUPPORTED.  Every call on one GPU shares that
 * scratch: calls that overlap on one GPU (other streams, other threads) race;
 * the caller serialises them.  Results equal xt_ternary_linear_f32's. */
int xt_ternary_linear_f32_noalloc(const xt_weights* w, const float* x, int64_t M, float* y,
                                  int mode, void* stream);

/* Several projections that share one input (same in_dim and format) in one
 * launch: ys[p] [M][out_dim(p)] for p < n (n <= 4).  The input is quantised
 * once.  Replaces TernaryLinear::fused_forward_qkv (src/bit1_58/layers.rs:347-424)
 * and fused_forward_mlp (:426-486).  q/inv_scale variant: */
int xt_ternary_linear_multi_q(const xt_weights* const* ws, int n, const int8_t* q,
                              const float* inv_scale, int64_t M, float* const* ys,
                              void* stream);
int xt_ternary_linear_multi_f32(const xt_weights* const* ws, int n, const float* x,
                                int64_t M, float* const* ys, int mode, void* stream);

/* out[m][i] = act(gate[m][i]) * up[m][i] for M rows of n (device, f32),
 * act one of XT_ACT_*.  Replaces quantization::silu_inplace
 * (src/bit1_58/quantization.rs:201-286; call once per row, as the reference
 * applies it to one row) and FastTensor::silu_mul_inplace /
 * relu2_mul_inplace (src/tensor.rs:170-238).  n <= 16384. */
int xt_activation_mul(int act, const float* gate, const float* up, int64_t M, int64_t n,
                      float* out, void* stream);

/* y[m] = rms_norm(x[m]) for M rows of n (device, f32), bit-exact with
 * rms_norm (src/nn/fast_attention_simd.rs:458-516: the sum of squares is
 * accumulated in index order in f32; rms = sqrt(sum / n + eps); y = x * (1 /
 * rms) * weight).  Replaces FastRmsNorm::forward / FastTensor::rmsnorm
 * (src/tensor.rs:242-265).  n <= 16384. */
int xt_rms_norm(const float* x, const float* weight, int64_t M, int64_t n, float eps, float* y,
                void* stream);

/* The ternary MLP block: gate = x Wg, up = x Wu (one quantised input, one
 * launch), mid = act(gate) * up, optional RMSNorm of mid (norm_weight [I]
 * device f32, or NULL), requantisation of mid, y = down(mid) [M][out_dim].
 * gate/up share in_dim and format; down's in_dim is the intermediate size
 * I <= 16384.  use_silu = 0 selects ReLU^2.
 *
 * xt_ternary_mlp_q takes the quantised input (q [M][in_dim] i8, inv_scale
 * [M]) and applies TernaryLinear::fused_mlp_all (src/bit1_58/layers.rs:
 * 497-645) to every row: SiLU is silu_inplace's AVX-512 path when mode is
 * XT_QUANT_AVX512, its portable path otherwise.
 *
 * xt_ternary_mlp_f32 is Mlp::forward (src/models/llama/mlp.rs:43-128) for
 * all-ternary projections: it quantises x; one row (M == 1) takes the fused
 * path above, several rows take the reference's unfused path (SiLU as
 * silu_mul_inplace).  Uses a per-stream device workspace of
 * M * (8 * I + padded I + 8) bytes. */
int xt_ternary_mlp_q(const xt_weights* gate, const xt_weights* up, const xt_weights* down,
                     const float* norm_weight, float eps, int use_silu, const int8_t* q,
                     const float* inv_scale, int64_t M, float* y, int mode, void* stream);
int xt_ternary_mlp_f32(const xt_weights* gate, const xt_weights* up, const xt_weights* down,
                       const float* norm_weight, float eps, int use_silu, const float* x,
                       int64_t M, float* y, int mode, void* stream);

/* ---- Decode stack: a whole list of projections, planned once ----
 * The decode step of the reference runs its layers' projections one call
 * after the other (src/models/llama/mod.rs:420-470: per layer
 * fused_forward_qkv, o, fused_forward_mlp / gate+up, down; the next block's
 * weights prefetched while the current one computes, :446-453).  A stack
 * holds such a list and runs it in one of two plans:
 *   XT_STACK_ONE_LAUNCH  ONE persistent launch in which the waves stream the
 *                        weights of later projections while earlier ones
 *                        finish (dependencies are kept inside the launch);
 *   XT_STACK_PER_OP      one library call per op in dependency order (a
 *                        dependency is then a kernel boundary).
 * xt_stack_create picks the faster plan for the list unless mode carries one
 * of the flags: a dependency kept inside a launch costs about 20 us here
 * against a few us for a kernel boundary, so long chains run per op and
 * wide lists (many ops per dependency level) in one launch.  Every output is
 * bit-identical to xt_ternary_linear_f32 / xt_ternary_linear_multi_f32 of
 * the same op in both plans.
 *
 * One op: n (1..4) projections that share one f32 input x [M][in_dim]
 * (same in_dim and format), outputs y[p] [M][out_dim(p)].  dep: index of an
 * EARLIER op whose outputs this op's x reads (x is then one of that op's y
 * buffers), or -1 when x is ready before the run.  Ops without a dep path
 * between them may run concurrently: no op may write a buffer that another
 * op reads or writes unless a dep chain orders them.  M is 1..32 for the
 * whole stack.  The one-launch plan takes Pack4, Pack5 and XorSparse tile
 * weights (in_dim a multiple of 4, a padded row of at most 32768 bytes; the
 * projections of one op in one tile format); the per-op plan takes every
 * format, and is what XT_STACK_AUTO picks for a list the one-launch kernel
 * does not take (the compact XorSparse stream).  The stack keeps the pointers (x, y,
 * weights): they must stay valid while it is used; change the data in place
 * between runs.  No reference counterpart as an API: the reference has no
 * device launches. */
typedef struct xt_stack_op {
    const xt_weights* w[4];
    int n;
    const float* x;
    float* y[4];
    int dep;
} xt_stack_op;
typedef struct xt_stack xt_stack;

/* Plan flags, OR'd into xt_stack_create's mode (XT_STACK_AUTO: none). */
enum { XT_STACK_AUTO = 0, XT_STACK_ONE_LAUNCH = 256, XT_STACK_PER_OP = 512 };

/* Validate the ops, choose the plan and build the device work list
 * (allocates; load time).  mode: XT_QUANT_* | optional plan flag. */
int xt_stack_create(const xt_stack_op* ops, int nops, int64_t M, int mode, xt_stack** out);
/* The plan of a stack: XT_STACK_ONE_LAUNCH or XT_STACK_PER_OP (negative on
 * a NULL stack). */
int xt_stack_plan(const xt_stack* st);
/* Run the whole list on `stream` (asynchronous).  One launch: no allocation,
 * no memset, capturable in a HIP graph.  Per op: the calls of
 * xt_ternary_linear_f32 / _multi_f32, with their workspaces (run once
 * outside capture first, as for those calls).  Runs of one stack must not
 * overlap (they share its counters and scratch): order them on one stream. */
int xt_stack_run(const xt_stack* st, void* stream);
/* Wait for the device, then report whether any dependency wait of the runs
 * since the last check gave up (*gave_up = 1: outputs of those runs are not
 * valid; a wait gives up after seconds, e.g. if the device is shared with a
 * kernel that never yields), and clear the flag.  Per-op stacks have no
 * such waits: *gave_up = 0. */
int xt_stack_check(xt_stack* st, int* gave_up);
int xt_stack_destroy(xt_stack* st);

#ifdef __cplusplus
}
#endif
#endif /* XTERN_H */
