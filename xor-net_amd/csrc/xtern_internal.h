// Internal declarations shared by the xtern host API and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace xt {

// Device tile geometry.  A tile holds 16 output rows x CH input columns of
// one matrix, 1024 bytes: 64 lanes x 16 bytes, one global_load_dwordx4 per
// lane.  Lane l = 16*g + j serves output row j of the tile and, inside every
// 64-wide MFMA k-step s, the 16 columns s*64 + g*16 .. +15.
//   Pack4 tiles (also used for XorSparse): CH = 256, 4 k-steps, dword s of a
//     lane holds the 16 codes of step s with the code of column 4*jj + d at
//     bit 8*d + 2*jj, so (dword >> 2*jj) & 0x03030303 yields the codes of
//     columns 4*jj .. 4*jj+3 in byte order.
//   Pack5 tiles: CH = 320, 5 k-steps, byte b of a lane holds the trits of
//     columns s*64 + g*16 + b for s = 0..4 as the fixed-point base-3 value
//     e = ceil(v * 256 / 243), v = sum_s t_s * 3^(4-s); trit s is recovered by
//     five rounds of y = 3*x, t = y >> 8, x = y & 255.
// Codes are the weight plus one (0 = -1, 1 = 0, 2 = +1); padding holds code
// 1.  The kernels multiply codes, not weights, and subtract the activation
// row sum once at the end: sum_k a*(w+1) - sum_k a = sum_k a*w, exactly.
//   Int8 / Int4 weights (formats 3 / 4, the reference's Int8Linear /
//     Int4Linear): CH = 256 columns, 4 k-steps, in 4 (Int8) or 2 (Int4)
//     consecutive 1 KiB tiles per chunk.  Int8 tile w holds k-step w as the
//     signed weights themselves; Int4 tile w holds k-steps 2w (low nibbles)
//     and 2w+1 (high nibbles) as codes q + 8 in [0, 15].
constexpr int kTileBytes = 1024;
inline int chunk_cols(int fmt) { return fmt == 1 ? 320 : 256; }
// 1 KiB tiles per 16-row chunk.
inline int tiles_per_chunk(int fmt) { return fmt == 3 ? 4 : (fmt == 4 ? 2 : 1); }
inline bool is_int_format(int fmt) { return fmt == 3 || fmt == 4; }

// Up to four projections that share one input, in one launch.
struct Proj {
    const uint8_t* tiles;  // [NG][nch][64][16]
    const float* ws;       // w_scales, [N]
    float* y;              // [M][N]
    int32_t* acc;          // optional [M][N] exact i32 dots
    int N;
    int tile0;             // first blockIdx.x of this projection
    int col0;              // first column of this projection in the split-K workspace
};

struct MMArgs {
    Proj proj[4];
    int nproj;
    const int8_t* q;        // [M][ldq], zero beyond in_dim up to nch*CH
    const float* inv;       // [M]
    const int32_t* rowsum;  // [M] sum of q over the row, or null
    int M;
    int ldq;
    int nch;                // chunks per row
    int cps;                // chunks per split-K slice (blockIdx.z)
    int32_t* part;          // split-K partial sums [M][ldp], all zero between calls
    int ldp;
    unsigned* cnt;          // split-K arrival counters, one per (x, y) tile, zero between calls
    // GEMV only: when x is set the kernel quantises the f32 rows x [M][ldx]
    // (in_dim K, rounding `mode`) itself instead of reading q / inv.
    const float* x;
    int64_t ldx;
    int K;
    int mode;
    int rg;                 // decode GEMV: 16-row groups per workgroup (0 or 1: one)
};
// GEMV with the quantiser fused when M * K is at most this (every workgroup
// re-reads the f32 rows, so only for small inputs).  The staging-free GEMV
// fuses one row of up to this many columns (its LDS stage bounds K further:
// 31 Pack4 or 28 Pack5 chunks).
constexpr int kGemvFusedQuantMax = 8192;
constexpr int kGemv2FusedQuantMax = 16384;

// Streaming decode GEMV (xtern_gstream.hip): one projection, M <= 16 rows
// of i8 activations given.
struct GStreamArgs {
    const uint8_t* tiles;  // [NG][nch][64][16]
    const float* ws;       // [N]
    float* y;              // [M][N]
    int32_t* acc;          // optional [M][N]
    const int8_t* q;       // [M][ldq], zero beyond in_dim up to nch * CH
    const float* inv;      // [M]
    int M, ldq, nch, NG, N;
    // set by the launcher: LDS row stride, row groups [G0, G1) of this
    // launch, the most groups of one wave, the sums' LDS offset
    int lda, G0, G1, rg_max, sums_off;
};
bool gstream_fits(int fmt, int M, int nch);
hipError_t launch_gstream(int fmt, const GStreamArgs& a, int grid, int d, hipStream_t s);

struct MMConfig {
    int mb, nb, waves, pf;  // tokens per WG = 16*mb, rows per WG = 16*nb
    int splitk;             // workgroups along K (blockIdx.z)
    int kind = 0;           // 0 mm_kernel, 1 prefill GEMM, 2 decode GEMV (waves used),
                            // 3 prefill GEMM on 32x32x32 MFMA (Pack4 tiles)
};

// Kernel launchers (xtern_kernels.hip).  Return the hipError_t of the launch.
hipError_t launch_quantize(const float* x, int64_t ldx, int M, int K, int8_t* q, int ldq,
                           float* inv, int32_t* rowsum, int mode, hipStream_t s);
hipError_t launch_rowsum(const int8_t* qin, int64_t ldin, int M, int K, int8_t* qout,
                         int ldout, int32_t* rowsum, hipStream_t s);
hipError_t launch_mm(int fmt, const MMConfig& cfg, const MMArgs& a, int ntiles_total,
                     hipStream_t s);
MMConfig choose_config(int fmt, int M, int ntiles_nb1, int nch, bool have_rowsum);
// Prefill GEMM (M > 16, row sums required): 32 tokens x 128 rows per
// workgroup, at most gemm_ncmax(fmt) chunks per split-K slice.
int gemm_ncmax(int fmt);
hipError_t launch_gemm(int fmt, const MMArgs& a, int ntiles, int splitk, hipStream_t s);
// Prefill GEMM on 32x32x32 MFMA (Pack4 tiles, M > 16, row sums required):
// 32 tokens x 128 rows per workgroup, at most gemm32_ncmax() chunks per slice.
int gemm32_ncmax();
int g32_splitk(int nch);
hipError_t launch_gemm32(const MMArgs& a, int ntiles, int splitk, hipStream_t s);
// Decode GEMV (M <= 16): 16 output rows per workgroup, activations in LDS.
hipError_t launch_gemv(int fmt, const MMArgs& a, int ntiles, int waves, hipStream_t s);
int gemv_ncw(int waves);
// Largest M * K the staging-free GEMV quantises itself for nch chunks and rg
// row groups per workgroup (0: none).
int gemv2_fused_max(int fmt, int nch, int rg);
// 16-row groups per workgroup of the decode GEMV that launch_gemv runs for
// this format and K (its ntiles count workgroups of that many groups).
int gemv_row_groups(int fmt, int nch, int ngroups);
// Whether launch_gemv runs the staging-free GEMV for this format and K
// (i8 rows given).
bool gemv2_takes(int fmt, int nch);
int int_gemv_waves(int fmt, int mb, int nch);
bool gemv_fits(int fmt, int M, int nch, int waves, int ncw);
// MLP middle stage (xtern_kernels.hip): per row of gate/up, activation,
// optional RMSNorm, optional f32 output, optional requantisation.
struct MidArgs {
    const float* gate;  // [M][ldg]
    const float* up;    // [M][ldg]
    int64_t ldg;
    int n;              // row length (intermediate size)
    int C;              // set by the launcher
    int act;            // XT_ACT_*
    const float* norm_w;  // [n] RMSNorm weight, or null
    float eps;
    int mode;             // requantisation rounding (XT_QUANT_*)
    int8_t* q;            // [M][ldq] (zero padded to ldq), or null
    int ldq;
    float* inv;           // [M]
    int32_t* rowsum;      // [M] or null
    float* out;           // [M][ldo] f32 activation (+ norm) result, or null
    int64_t ldo;
};
constexpr int kActIdentity = 100;  // MidArgs::act: no activation (up unused)
int mid_max_cols();
hipError_t launch_mlp_mid(const MidArgs& a, int M, hipStream_t s);

// GEMV over the XorSparse compact stream (xtern_xs.hip).  Sections as built
// by build_xs_stream; q [M][ldq] i8 with ldq >= ceil(K/64) * 64 (zero past
// K), M <= 16, nb = ceil(K/64) <= xs_max_blocks().
struct XsArgs {
    const uint32_t* seg;
    const uint32_t* mask;
    const uint32_t* sign;
    unsigned seg_bytes, mask_bytes, sign_bytes;
    const int8_t* q;
    unsigned q_bytes;
    int ldq;
    const float* inv;
    const float* ws;
    float* y;
    int32_t* acc;  // or null
    int M, N, nb;
};
hipError_t launch_xs_gemv(const XsArgs& a, hipStream_t s);
int xs_max_blocks();
int xs_max_rows();
// Address (on the current device) and size of the static device scratch used
// by the allocation-free entry point; resolved once per device.
hipError_t scratch_region(void** ptr, size_t* bytes);
// Streaming decode stack, M = 1 (xtern_sstack.hip).
constexpr int kSStackMaxOps = 8191;          // op index: 13 bits of a task
constexpr int kSStackMaxRowBytes = 32768;    // i8 row (nch * chunk columns) of one op, at most
constexpr int kSStackMaxM = 32;              // tokens of the streaming stack (two MFMA blocks)
// One task, 64 bytes: everything a wave needs to start it, loaded one task
// ahead.  flags bits 0-15: 1 quantiser task, 2 other ops read the outputs
// (count the groups' completion), 4 Pack5 tiles; bits 16-31: the task's
// consecutive 16-row groups (one projection), nrows: rows of the last one.
// An op's quantised rows: q [M][ldq] i8, then M i32 row sums, then M f32
// inverse scales.
struct alignas(16) SStackTask {
    const void* tiles;        // group: its first tile; quantiser: its token's f32 input row
    const float* ws;          // group: w_scales of its rows; quantiser: its token's sum slot
    float* y;                 // group: outputs of its rows (token 0; token t at + t * K)
    int8_t* q;                // group: the op's rows q; quantiser: its token's i8 row
    int opi, flags, nch, nrows;
    int K, ldq, dep, dep_groups;  // K: quantiser: in_dim; group: out_dim (the output row stride).
                                  // dep: op whose outputs x reads, or -1; its group count
};
static_assert(sizeof(SStackTask) == 64, "a task record is four 16-byte loads");
struct SStackArgs {
    const SStackTask* tasks;  // wave w runs tasks[woff[w] .. woff[w + 1]) in order
    const int* woff;          // [waves + 1]
    unsigned* ctr;            // (4 + 2 * nops) slots of 128 bytes, zero between launches
    int ntasks, nops, mode, spin_limit;
    int row_bytes;            // LDS per wave: one chunk of the form's token rows, padded
    int M;                    // tokens, 1..kSStackMaxM
    int pack5;                // 1: the base-3 token forms (Pack5 tiles are most of the bytes)
};
hipError_t launch_sstack(const SStackArgs& a, int blocks, hipStream_t s);
hipError_t sstack_blocks_per_cu(int M, bool p5, int row_bytes, int* n);
int sstack_lds_rows(int M);         // token rows of a wave's LDS region
int sstack_groups_per_task(int M, bool p5);  // 16-row groups per group task
bool sstack_quant_tasks(int M);     // quantiser tasks (else each group task quantises its row: M = 1)
int sstack_waves_per_block();
// HF prepacked striped bytes [N/f][K] (device) -> tiles (device).
hipError_t launch_hf_tiles(int fmt, const uint8_t* stored, int64_t K, int64_t N, uint8_t* tiles,
                           hipStream_t s);

}  // namespace xt
