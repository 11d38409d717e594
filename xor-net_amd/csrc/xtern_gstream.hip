// Streaming decode GEMV: few tokens (M <= 16) times a tall ternary matrix,
// as one continuous stream of weight tiles per wave.
//
// Reference behaviour: TernaryLinear::forward_with_quantized
// (src/bit1_58/layers.rs:315-345) -- per output row `dot_row` (:216-231) over
// the pack4 / pack5 / sparse dot (src/bit1_58/simd.rs:358-548), then
// (dot as f32 * inv_scale) * w_scale (:340) -- bit-exact.
//
// Why a second decode GEMV.  The one-shot GEMV (gemv2_kernel) gives every
// workgroup a few row groups, loads all of their tiles at once, reduces across
// waves through LDS and exits.  On a tall matrix that alternates bursts of
// loads with phases that have none in flight, and it reaches about 4.7 TB/s.
// A plain streaming read on MI355X reaches 7.1-7.2 TB/s with about 32 KB in
// flight per CU issued continuously (more in flight is slower: 128-512 KB per
// CU fall back to 5.1-6.0 TB/s), whether the waves sweep the buffer together
// or each wave walks its own 10 KB segments.  So here every wave owns whole
// row groups (16 output rows over all of K: no cross-wave reduction and no
// barrier after the start) and walks them as one sequence of tiles -- row
// group gw, gw + TW, gw + 2 TW, ... (gw the wave's global index, TW the
// waves of the grid) -- D tiles per batch: the batch's loads are issued back
// to back, then its tiles are multiplied.  With four 4-wave workgroups per CU
// and D = 2 that is 32 KB in flight per CU; measured on a 535 MB matrix
// (121 stacked C0 matrices) 6.4 TB/s, against 5.6 TB/s for the same walk
// through a ring of LDS slots filled by direct-to-LDS loads.
//
// The activation rows (M x K i8) are copied to LDS once per workgroup, with
// their exact sums; the A fragment of a k-step is one ds_read_b128 that the
// lanes of one token share.  The MFMAs multiply codes w + 1 (Pack4: shifts
// and masks; Pack5: the base-3 digit rounds; code 3 never reaches the device,
// the repack writes it as 1), and the row sum is subtracted once per row
// group: sum a (w + 1) - sum a = sum a w, exactly.  A row group's i32 sums
// wait in LDS until the wave's stream ends, so the loop issues no stores and
// no scale loads; the f32 epilogue runs once at the end.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "xtern_device.h"
#include "xtern_internal.h"

namespace xt {

namespace {

__device__ __forceinline__ v4i lds16(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) v4i*>((uintptr_t)addr);
}
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int FMT, int D, int W>
__global__ __launch_bounds__(W * 64) void gstream_kernel(const GStreamArgs a) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    extern __shared__ __align__(16) uint8_t lds[];  // rows [M][lda], row sums, then the waves' sums
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, j = lane & 15;
    const int M = a.M, nch = a.nch, N = a.N;
    const int lda = a.lda;
    const int ng4 = (M + 3) >> 2;  // token lane groups that carry rows < M
    int32_t* const rsum = reinterpret_cast<int32_t*>(lds + a.sums_off) - 16;

    // activation rows -> LDS (16 bytes per thread per trip) with their sums
    if (threadIdx.x < 16) rsum[threadIdx.x] = 0;
    __syncthreads();
    {
        const int per_row = (nch * CH) / 16;
        const int total = M * per_row;
        for (int i = threadIdx.x; i < total; i += W * 64) {
            const int m = i / per_row, p = i - m * per_row;
            const v4i v = *reinterpret_cast<const v4i*>(a.q + (size_t)m * a.ldq + p * 16);
            *reinterpret_cast<v4i*>(lds + m * lda + p * 16) = v;
            int sm = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) sm = __builtin_amdgcn_sdot4(v[d], 0x01010101, sm, false);
            atomicAdd(&rsum[m], sm);
        }
    }
    const int TW = gridDim.x * W;
    const int gw = blockIdx.x * W + wave;
    const int nrg = a.G0 + gw < a.G1 ? (a.G1 - 1 - a.G0 - gw) / TW + 1 : 0;  // this wave's groups
    const int T = nrg * nch;                                                // its tiles
    // this wave's sums: M = 1 one i32 per (group, row); else 16 bytes per
    // (group, token lane group, row)
    int32_t* const sums = reinterpret_cast<int32_t*>(lds + a.sums_off) +
                          (size_t)wave * a.rg_max * (M == 1 ? 16 : ng4 * 64);
    __syncthreads();
    if (T == 0) return;

    const uint8_t* const tl0 = a.tiles + lane * 16;
    const uint32_t abase = lds_u32(lds) + (uint32_t)(min(j, M - 1) * lda + g * 16);
    int Gl = a.G0 + gw, cl = 0;  // the next tile to load
    int c = 0, rr = 0;           // the next tile to multiply, and its group
    v4i acc[STEPS];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) acc[st] = v4i{0, 0, 0, 0};
    for (int t0 = 0; t0 < T; t0 += D) {
        v4i wb[D];
#pragma unroll
        for (int s = 0; s < D; ++s) {
            // (past the stream: tile 0 again, an L2 hit that is never used)
            const size_t off = t0 + s < T ? ((size_t)Gl * nch + cl) * kTileBytes : 0;
            wb[s] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(tl0 + off));
            if (++cl == nch) {
                cl = 0;
                Gl += TW;
            }
        }
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const uint32_t ab = abase + (uint32_t)(c * CH);
            if constexpr (FMT == XT_PACK5) {
                int E[4], O[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    E[d] = wb[s][d] & 0x00ff00ff;
                    O[d] = ((unsigned)wb[s][d] >> 8) & 0x00ff00ff;
                }
#pragma unroll
                for (int st = 0; st < STEPS; ++st) {
                    v4i b;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int pE = E[d] * 3, pO = O[d] * 3;
                        b[d] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                        E[d] = pE & 0x00ff00ff;
                        O[d] = pO & 0x00ff00ff;
                    }
                    acc[st] = mfma(lds16(ab + st * 64), b, acc[st]);
                }
            } else {
#pragma unroll
                for (int st = 0; st < STEPS; ++st) acc[st] = mfma(lds16(ab + st * 64), decode4(wb[s][st]), acc[st]);
            }
            if (++c == nch) {  // (uniform) a row group is complete
                v4i sum = acc[0];
#pragma unroll
                for (int st = 1; st < STEPS; ++st) sum += acc[st];
                if (rr < nrg) {
                    if (M == 1) {
                        if (g == 0) sums[rr * 16 + j] = sum[0];
                    } else if (g < ng4) {
                        reinterpret_cast<v4i*>(sums)[(rr * ng4 + g) * 16 + j] = sum;
                    }
                }
#pragma unroll
                for (int st = 0; st < STEPS; ++st) acc[st] = v4i{0, 0, 0, 0};
                c = 0;
                ++rr;
            }
        }
    }
    // epilogue, layers.rs:340: (dot as f32 * inv_scale) * w_scale
    float invr[4];
    int rs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        invr[r] = a.inv[min(4 * g + r, M - 1)];
        rs[r] = rsum[min(4 * g + r, M - 1)];
    }
    for (int k = 0; k < nrg; ++k) {
        const int o = (a.G0 + gw + k * TW) * 16 + j;
        if (g >= ng4 || o >= N) continue;
        v4i sum;
        if (M == 1) sum = v4i{sums[k * 16 + j], 0, 0, 0};
        else sum = reinterpret_cast<const v4i*>(sums)[(k * ng4 + g) * 16 + j];
        const float wsc = a.ws[o];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 4 * g + r;
            if (i < M) {
                const int dot = sum[r] - rs[r];
                a.y[(size_t)i * N + o] = __fmul_rn(__fmul_rn((float)dot, invr[r]), wsc);
                if (a.acc) a.acc[(size_t)i * N + o] = dot;
            }
        }
    }
}

}  // namespace

// LDS of one launch: the activation rows, their sums, and every wave's group
// sums (rg_max groups each).
static size_t gs_lds(int M, int nch, int fmt, int w, int rg_max, size_t* sums_off) {
    const size_t rows = (size_t)M * (size_t)(nch * chunk_cols(fmt) + 16);
    *sums_off = ((rows + 15) & ~(size_t)15) + 64;
    return *sums_off + (size_t)w * rg_max * (M == 1 ? 64 : ((M + 3) / 4) * 256);
}
constexpr size_t kGsLdsMax = 40 * 1024;  // four workgroups per CU
constexpr int kGsWaves = 4;

bool gstream_fits(int fmt, int M, int nch) {
    size_t off;
    return M >= 1 && M <= 16 && gs_lds(M, nch, fmt, kGsWaves, 1, &off) <= kGsLdsMax;
}

// Row groups [0, NG) in as few launches as the sums' LDS allows.  d: tiles
// per batch (2 or 4), grid: workgroups of kGsWaves waves.
hipError_t launch_gstream(int fmt, const GStreamArgs& a0, int grid, int d, hipStream_t s) {
    GStreamArgs a = a0;
    a.lda = a.nch * chunk_cols(fmt) + 16;
    if (!gstream_fits(fmt, a.M, a.nch) || grid < 1 || (d != 2 && d != 4)) return hipErrorInvalidValue;
    size_t off = 0;
    const size_t base = gs_lds(a.M, a.nch, fmt, kGsWaves, 0, &off);
    const size_t per_rg = gs_lds(a.M, a.nch, fmt, kGsWaves, 1, &off) - base;
    const int rg_fit = (int)((kGsLdsMax - base) / per_rg);
    const int tw = grid * kGsWaves;
    const int per_launch = std::max(1, std::min(rg_fit, (a.NG + tw - 1) / tw)) * tw;
    for (int g0 = 0; g0 < a.NG; g0 += per_launch) {
        a.G0 = g0;
        a.G1 = std::min(a.NG, g0 + per_launch);
        a.rg_max = (a.G1 - a.G0 + tw - 1) / tw;
        const size_t lds = gs_lds(a.M, a.nch, fmt, kGsWaves, a.rg_max, &off);
        a.sums_off = (int)off;
        const dim3 gr(grid), bl(kGsWaves * 64);
        if (fmt == XT_PACK5) {
            if (d == 2) hipLaunchKernelGGL((gstream_kernel<XT_PACK5, 2, kGsWaves>), gr, bl, lds, s, a);
            else hipLaunchKernelGGL((gstream_kernel<XT_PACK5, 4, kGsWaves>), gr, bl, lds, s, a);
        } else {
            if (d == 2) hipLaunchKernelGGL((gstream_kernel<XT_PACK4, 2, kGsWaves>), gr, bl, lds, s, a);
            else hipLaunchKernelGGL((gstream_kernel<XT_PACK4, 4, kGsWaves>), gr, bl, lds, s, a);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace xt
