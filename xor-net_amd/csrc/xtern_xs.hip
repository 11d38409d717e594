// XorSparse GEMV over the compact stream (weights of format
// XT_XORSPARSE_STREAM): the block masks and set-order sign bits of the
// reference's row blobs (src/bit1_58/sparse.rs:9-17, :61-86, decoded as
// simd.rs:416-548 does), read as they are -- no expansion to 2-bit tiles in
// memory, so the bytes streamed are the format's own.
//
// Layout (built on the host, xtern_layout.cpp build_xs_stream): per 16-row
// group G and 64-column block b, the 16 row masks (u64) and one bit offset
// into a sign stream where the 16 rows' set-order sign bits follow each
// other.
//
// Workgroup = one row group; 16 waves.  A wave takes block quads (4 blocks x
// 16 rows, one (row, block) per lane).  Phase 1 loads every mask and segment
// offset the wave needs (and, for one token, its activation pieces); phase 2
// turns them into each lane's sign window: the row's offset inside the
// segment is an exclusive prefix sum of the 16 rows' popcounts (a 16-lane
// scan), and three dwords from there hold the row's up to 64 sign bits;
// phase 3 expands them to lane order four weights at a time -- a 256-entry
// LDS table indexed by the 4-bit mask nibble and the next 4 set-order sign
// bits gives the four signed weight bytes -- and multiplies with v_dot4
// against the i8 activations (exact i32 sums).  Rows are reduced across the
// wave's 4 block lanes by shuffles and across waves through LDS.
//
// Every global read is a buffer load bounded by its section's size (a load
// past it reads zeros and touches no memory), with the offset in the vector
// offset (the one the bound applies to); every load is issued whatever the
// lane's block, so the compiler's wait counts stay exact.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xtern_device.h"
#include "xtern_internal.h"

namespace xt {

namespace {

constexpr unsigned kXsOOR = 0x80000000u;  // an offset past every section

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xs_rsrc(const void* p, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ unsigned xs_ld32(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return (unsigned)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ v4i xs_ld128(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// MT: token rows per launch (1, 4 or 16; M <= MT); NIT: block quads per
// wave; W: waves per workgroup.
template <int MT, int NIT, int W>
__global__ __launch_bounds__(W * 64) void xs_gemv_kernel(const XsArgs a) {
    constexpr int kXsWaves = W;
    __shared__ unsigned table[256];
    __shared__ int red[kXsWaves][MT][16];
    // MT > 1: per wave, the quad's expanded weights [block][row][16-byte
    // piece] and activation rows [token][piece] (one piece of padding per row)
    __shared__ v4i wsl[MT > 1 ? kXsWaves : 1][4][16][4];
    __shared__ v4i asl[MT > 1 ? kXsWaves : 1][16][17];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int j = lane & 15, bq = lane >> 4;
    const unsigned G = blockIdx.x;
    // table[nib * 16 + s]: the four weight bytes of a mask nibble `nib`
    // whose set lanes take the set-order signs s (bit 0 first; 1 = -1)
    if (t < 256) {
        const unsigned nib = (unsigned)t >> 4, s = (unsigned)t & 15u;
        unsigned v = 0, r = 0;
        for (int p = 0; p < 4; ++p)
            if ((nib >> p) & 1u) {
                v |= (((s >> r) & 1u) ? 0xffu : 0x01u) << (8 * p);
                ++r;
            }
        table[t] = v;
    }
    const int nb = a.nb, M = a.M, N = a.N;
    const __amdgpu_buffer_rsrc_t mr = xs_rsrc(a.mask, a.mask_bytes);
    const __amdgpu_buffer_rsrc_t sr = xs_rsrc(a.seg, a.seg_bytes);
    const __amdgpu_buffer_rsrc_t gr = xs_rsrc(a.sign, a.sign_bytes);
    const __amdgpu_buffer_rsrc_t qr = xs_rsrc(a.q, a.q_bytes);

    // phase 1: masks and segment offsets (and one token's pieces)
    unsigned mlo[NIT], mhi[NIT], seg[NIT];
    bool live[NIT];
    int blk[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        blk[it] = 4 * (wave + it * kXsWaves) + bq;
        live[it] = blk[it] < nb;
        const unsigned gb = G * (unsigned)nb + (unsigned)blk[it];
        const unsigned mo = live[it] ? (gb * 16u + (unsigned)j) * 8u : kXsOOR;
        mlo[it] = xs_ld32(mr, mo);
        mhi[it] = xs_ld32(mr, mo + 4u);
        seg[it] = xs_ld32(sr, live[it] ? gb * 4u : kXsOOR);
    }
    v4i x1[MT == 1 ? NIT : 1][4];
    if constexpr (MT == 1) {
#pragma unroll
        for (int it = 0; it < NIT; ++it)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                x1[it][u] = xs_ld128(qr, live[it] ? (unsigned)blk[it] * 64u + 16u * u : kXsOOR);
    }
    __builtin_amdgcn_sched_barrier(0);

    // phase 2: each lane's sign window (bits [bitpos, bitpos + 96) of the
    // stream: the row's <= 64 signs start within the first word)
    unsigned w0[NIT], w1[NIT], w2[NIT], sh[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const unsigned cnt = __popc(mlo[it]) + __popc(mhi[it]);
        unsigned inc = cnt;  // inclusive prefix over the 16 rows of the block
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const unsigned o = __shfl_up(inc, d, 16);
            if (j >= d) inc += o;
        }
        const unsigned bitpos = seg[it] + inc - cnt;
        const unsigned wo = live[it] ? (bitpos >> 5) * 4u : kXsOOR;
        w0[it] = xs_ld32(gr, wo);
        w1[it] = xs_ld32(gr, wo + 4u);
        w2[it] = xs_ld32(gr, wo + 8u);
        sh[it] = bitpos & 31u;
    }
    __syncthreads();  // the table

    // phase 3: expand and multiply
    int acc[MT == 1 ? 1 : 1];
    acc[0] = 0;
    v4i macc = v4i{0, 0, 0, 0};  // MT > 1: tokens 4g..4g+3 of row (lane & 15)
    const int g = lane >> 4;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const unsigned S0 = __builtin_amdgcn_alignbit(w1[it], w0[it], sh[it]);
        const unsigned S1 = __builtin_amdgcn_alignbit(w2[it], w1[it], sh[it]);
        unsigned wd[16];
        unsigned r = 0;  // set lanes before this nibble
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
            const unsigned nib = ((tt < 8 ? mlo[it] : mhi[it]) >> (4 * (tt & 7))) & 15u;
            const unsigned lo = __builtin_amdgcn_alignbit(S1, S0, r & 31u);
            const unsigned hi = S1 >> (r & 31u);
            const unsigned sb = ((r & 32u) ? hi : lo) & 15u;
            wd[tt] = table[(nib << 4) | sb];
            r += __popc(nib);
        }
        if constexpr (MT == 1) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    acc[0] = __builtin_amdgcn_sdot4((int)wd[4 * u + d], x1[it][u][d], acc[0], false);
        } else {
            // The quad's 4 x 64 columns: the expanded weights (lane order,
            // row j of block bq) and the activation rows (4-row loads:
            // token 4u + lane / 16, piece lane % 16) go through the wave's
            // LDS slices, then one MFMA per block takes 16 tokens x 16 rows
            // x 64 columns.  (A wave's LDS accesses complete in order: no
            // barrier.)
            const int q0 = wave + it * kXsWaves;  // the quad
            const bool qlive = 4 * q0 < nb;
            v4i xa[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int m = 4 * u + (lane >> 4);
                xa[u] = xs_ld128(qr, (qlive && m < M) ? (unsigned)m * (unsigned)a.ldq + (unsigned)q0 * 256u +
                                                            (unsigned)(lane & 15) * 16u
                                                      : kXsOOR);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p)
                wsl[wave][bq][j][p] = v4i{(int)wd[4 * p], (int)wd[4 * p + 1], (int)wd[4 * p + 2], (int)wd[4 * p + 3]};
#pragma unroll
            for (int u = 0; u < 4; ++u) asl[wave][4 * u + (lane >> 4)][lane & 15] = xa[u];
            __asm__ volatile("" ::: "memory");
#pragma unroll
            for (int b = 0; b < 4; ++b)
                macc = mfma(asl[wave][j][4 * b + g], wsl[wave][b][j][g], macc);
            __asm__ volatile("" ::: "memory");
        }
    }
    if constexpr (MT == 1) {
        // rows: the wave's 4 block lanes, then the waves
        int v = acc[0];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (bq == 0) red[wave][0][j] = v;
    } else {
        // lane (g, j): tokens 4g + r of row j
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) red[wave][4 * g + rr][j] = macc[rr];
    }
    __syncthreads();
    if (t < 16 * MT) {
        const int m = t >> 4, jj = t & 15;
        const int o = (int)G * 16 + jj;
        if (m < M && o < N) {
            int sum = 0;
#pragma unroll
            for (int w = 0; w < kXsWaves; ++w) sum += red[w][m][jj];
            // layers.rs:294 -- (dot as f32 * inv_scale) * w_scale
            a.y[(size_t)m * N + o] = __fmul_rn(__fmul_rn((float)sum, a.inv[m]), a.ws[o]);
            if (a.acc) a.acc[(size_t)m * N + o] = sum;
        }
    }
}

template <int MT>
hipError_t launch_mt(const XsArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.N + 15) / 16));
    const int nq = (a.nb + 3) / 4;  // block quads of a row group
    if constexpr (MT == 1) {
        // W waves of NIT quads each: four waves while they cover the row at
        // four quads per lane (independent items interleave in a lane), else 16
        if (nq <= 4 * 4) hipLaunchKernelGGL((xs_gemv_kernel<1, 4, 4>), grid, dim3(256), 0, s, a);
        else if (nq <= 16) hipLaunchKernelGGL((xs_gemv_kernel<1, 1, 16>), grid, dim3(1024), 0, s, a);
        else if (nq <= 32) hipLaunchKernelGGL((xs_gemv_kernel<1, 2, 16>), grid, dim3(1024), 0, s, a);
        else hipLaunchKernelGGL((xs_gemv_kernel<1, 4, 16>), grid, dim3(1024), 0, s, a);
    } else {
        // 8 waves (LDS slices of 8.3 KiB each)
        if (nq <= 8) hipLaunchKernelGGL((xs_gemv_kernel<MT, 1, 8>), grid, dim3(512), 0, s, a);
        else if (nq <= 16) hipLaunchKernelGGL((xs_gemv_kernel<MT, 2, 8>), grid, dim3(512), 0, s, a);
        else if (nq <= 32) hipLaunchKernelGGL((xs_gemv_kernel<MT, 4, 8>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((xs_gemv_kernel<MT, 8, 8>), grid, dim3(512), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace

int xs_max_blocks() { return 4 * 4 * 16; }  // (M > 1: 8 waves x 8 quads x 4)
int xs_max_rows() { return 16; }

hipError_t launch_xs_gemv(const XsArgs& a, hipStream_t s) {
    if (a.M <= 1) return launch_mt<1>(a, s);
    return launch_mt<16>(a, s);
}

}  // namespace xt
