// xtern HIP kernels for gfx950 (MI355X): activation quantiser and the
// ternary x i8 product on MFMA.
//
// Reference behaviour these kernels reproduce (paths relative to xor-net):
//   quantize_f32_to_i8          src/bit1_58/quantization.rs:95-195
//   ternary_dot_product_pack4   src/bit1_58/simd.rs:256-382
//   ternary_dot_product_pack5   src/bit1_58/simd.rs:384-414
//   TernaryLinear::forward      src/bit1_58/layers.rs:262-345 (epilogue :294)
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <type_traits>

#include "../../include/xtern.h"
#include "xtern_internal.h"
#include "xtern_device.h"



namespace xt {

// One workgroup per row.  Pass 1: absmax (fmaxf ignores NaN; NaN inputs are
// off-contract).  Pass 2: quantise, write i8 (zero-filling [K, ldq)), and the
// exact i32 row sum the product kernels subtract.
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ x, int64_t ldx,
                                                       int K, int8_t* __restrict__ q, int ldq,
                                                       float* __restrict__ inv,
                                                       int32_t* __restrict__ rowsum, int mode) {
    __shared__ float sm_f[4];
    __shared__ int sm_i[4];
    const int m = blockIdx.x;
    const float* xr = x + (size_t)m * ldx;
    int8_t* qr = q + (size_t)m * ldq;
    const bool vec = ((K & 3) == 0) && ((((uintptr_t)xr) & 15) == 0);

    float mx = 0.0f;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (int i = threadIdx.x; i < (K >> 2); i += 256) {
            const float4 v = x4[i];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(xr[k]));
    }
    mx = block_reduce(mx, MaxOp(), sm_f);
    const float scale = (mx > 0.0f) ? __fdiv_rn(127.0f, mx) : 1.0f;
    const float invs = (mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;

    int sum = 0;
    if (vec && (ldq & 3) == 0 && ((((uintptr_t)qr) & 3) == 0)) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (int i = threadIdx.x; i < (ldq >> 2); i += 256) {
            int b[4] = {0, 0, 0, 0};
            if (4 * i < K) {
                const float4 v = x4[i];
                const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) b[t] = quant_one(e[t], scale, mode, 4 * i + t < kmain);
            }
            sum += b[0] + b[1] + b[2] + b[3];
            const uint32_t packed = (uint32_t)(b[0] & 255) | ((uint32_t)(b[1] & 255) << 8) |
                                    ((uint32_t)(b[2] & 255) << 16) | ((uint32_t)(b[3] & 255) << 24);
            reinterpret_cast<uint32_t*>(qr)[i] = packed;
        }
    } else {
        for (int k = threadIdx.x; k < ldq; k += 256) {
            const int v = (k < K) ? quant_one(xr[k], scale, mode, k < kmain) : 0;
            qr[k] = (int8_t)v;
            sum += v;
        }
    }
    sum = block_reduce(sum, AddOp(), sm_i);
    if (threadIdx.x == 0) {
        inv[m] = invs;
        if (rowsum) rowsum[m] = sum;
    }
}

// Single-pass variant for K <= 4 * NT * NV with 16-byte aligned rows: each
// thread keeps its NV float4 of the row in registers between the absmax
// reduction and the quantisation, so the row is read from memory once.
// NT = 1024 for long rows (more loads in flight per row).
template <int NV, int NT>
__global__ __launch_bounds__(NT) void quantize_reg_kernel(const float* __restrict__ x, int64_t ldx,
                                                          int K, int8_t* __restrict__ q, int ldq,
                                                          float* __restrict__ inv,
                                                          int32_t* __restrict__ rowsum, int mode) {
    __shared__ float sm_f[NT / 64];
    __shared__ int sm_i[NT / 64];
    const int m = blockIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
    uint32_t* q4 = reinterpret_cast<uint32_t*>(q + (size_t)m * ldq);
    const int K4 = K >> 2;  // >= 1 (the launcher sends K < 4 elsewhere)
    // (every argument is consumed here, so all of them arrive in one round of
    // scalar loads ahead of the row load)
    asm volatile("" ::"s"(x), "s"(ldx), "s"(K), "s"(q), "s"(ldq), "s"(inv), "s"(rowsum), "s"(mode));
    float4 v[NV];
    float mx = 0.0f;
    // unconditional loads at clamped pieces, zeroed afterwards
#pragma unroll
    for (int u = 0; u < NV; ++u) v[u] = x4[min((int)threadIdx.x + u * NT, K4 - 1)];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i = threadIdx.x + u * NT;
        if (i >= K4) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    }
    mx = block_reduce<NT / 64>(mx, MaxOp(), sm_f);
    const float scale = (mx > 0.0f) ? __fdiv_rn(127.0f, mx) : 1.0f;
    const float invs = (mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;
    int sum = 0;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i = threadIdx.x + u * NT;
        if (i >= K4) continue;
        const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        int b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) b[t] = quant_one(e[t], scale, mode, 4 * i + t < kmain);
        sum += b[0] + b[1] + b[2] + b[3];
        q4[i] = (uint32_t)(b[0] & 255) | ((uint32_t)(b[1] & 255) << 8) |
                ((uint32_t)(b[2] & 255) << 16) | ((uint32_t)(b[3] & 255) << 24);
    }
    for (int i = K4 + threadIdx.x; i < (ldq >> 2); i += NT) q4[i] = 0u;  // padding
    if (rowsum) sum = block_reduce<NT / 64>(sum, AddOp(), sm_i);  // uniform: skipped when unused
    if (threadIdx.x == 0) {
        inv[m] = invs;
        if (rowsum) rowsum[m] = sum;
    }
}

// Row sums of caller-provided i8 activations, optionally copying them into a
// zero-padded buffer with a 16-byte aligned stride.
__global__ __launch_bounds__(256) void rowsum_kernel(const int8_t* __restrict__ qin, int64_t ldin,
                                                     int K, int8_t* __restrict__ qout, int ldout,
                                                     int32_t* __restrict__ rowsum) {
    __shared__ int sm_i[4];
    const int m = blockIdx.x;
    const int8_t* r = qin + (size_t)m * ldin;
    int sum = 0;
    const int lim = qout ? ldout : K;
    for (int k = threadIdx.x; k < lim; k += 256) {
        const int v = (k < K) ? (int)r[k] : 0;
        sum += v;
        if (qout) qout[(size_t)m * ldout + k] = (int8_t)v;
    }
    sum = block_reduce(sum, AddOp(), sm_i);
    if (threadIdx.x == 0) rowsum[m] = sum;
}

hipError_t launch_quantize(const float* x, int64_t ldx, int M, int K, int8_t* q, int ldq,
                           float* inv, int32_t* rowsum, int mode, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const bool aligned = (K % 4 == 0) && (ldx % 4 == 0) && (ldq % 4 == 0) &&
                         ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 4 == 0);
    if (aligned && K >= 4 && K <= 16384) {
#define XT_QREG(NV_, NT_)                                                                        \
    if (K <= 4 * NT_ * NV_) {                                                                    \
        hipLaunchKernelGGL((quantize_reg_kernel<NV_, NT_>), dim3(M), dim3(NT_), 0, s, x, ldx, K, q, \
                           ldq, inv, rowsum, mode);                                              \
        return hipGetLastError();                                                                \
    }
        XT_QREG(1, 256)
        XT_QREG(2, 256)
        XT_QREG(1, 1024)
        XT_QREG(2, 1024)
        XT_QREG(4, 1024)
#undef XT_QREG
    }
    hipLaunchKernelGGL(quantize_kernel, dim3(M), dim3(256), 0, s, x, ldx, K, q, ldq, inv, rowsum,
                       mode);
    return hipGetLastError();
}

// Static scratch of the allocation-free entry point: device memory that the
// library never allocates at run time.  Each GPU holds its own copy; host
// code reaches it only through the address hipGetSymbolAddress returns for
// the current device (the array's name is a host-side stand-in).  Every call
// on one GPU shares it: calls that overlap on one GPU race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

hipError_t scratch_region(void** ptr, size_t* bytes) {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    *bytes = kScratchBytes;
    return hipSuccess;
}

hipError_t launch_rowsum(const int8_t* qin, int64_t ldin, int M, int K, int8_t* qout, int ldout,
                         int32_t* rowsum, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(rowsum_kernel, dim3(M), dim3(256), 0, s, qin, ldin, K, qout, ldout, rowsum);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Ternary x i8 product on MFMA
// ---------------------------------------------------------------------------

// The projection workgroup column bx belongs to, read through the kernel
// argument segment (scalar loads; the selected projection is one load at a
// computed offset -- selecting among by-value fields instead makes the
// compiler copy the arguments to scratch memory).
struct ProjView {
    const uint8_t* tiles;
    const float* ws;
    float* y;
    int32_t* acc;
    int N, tile0, col0;
};
typedef const __attribute__((address_space(4))) MMArgs* KArgPtr;
struct ProjBounds {
    int np, t0, t1, t2, t3;
};
// Read at kernel entry, in the same round of scalar loads as the grid size.
// proj[0].tile0 (always 0) is read in this round too: it shares the first
// argument line with proj[0]'s pointers, so that line is fetched beside the
// bounds and the selected projection's load (proj[0] in a single-projection
// launch) hits the scalar cache instead of waiting on a second cold line.
__device__ __forceinline__ ProjBounds proj_bounds() {
    KArgPtr ka = (KArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    return ProjBounds{ka->nproj, ka->proj[0].tile0, ka->proj[1].tile0, ka->proj[2].tile0,
                      ka->proj[3].tile0};
}
__device__ __forceinline__ ProjView select_proj(const ProjBounds& pb, int bx) {
    KArgPtr ka = (KArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    bx -= pb.t0;  // (tile0 of the first projection is 0)
    const int sel = ((pb.np > 1) & (bx >= pb.t1)) + ((pb.np > 2) & (bx >= pb.t2)) +
                    ((pb.np > 3) & (bx >= pb.t3));
    ProjView v;
    v.tiles = ka->proj[sel].tiles;
    v.ws = ka->proj[sel].ws;
    v.y = ka->proj[sel].y;
    v.acc = ka->proj[sel].acc;
    v.N = ka->proj[sel].N;
    v.tile0 = ka->proj[sel].tile0;
    v.col0 = ka->proj[sel].col0;
    return v;
}

// Workgroup (blockIdx.x, blockIdx.y, blockIdx.z) computes a (16*MB tokens) x
// (16*NB output rows) tile over chunk slice z of the reduction dimension.  Its
// WAVES waves take interleaved chunks of the slice and are summed through
// LDS.  Each wave loads PF chunks (weights and activations) before consuming
// any, so one HBM round trip covers PF chunks.  With gridDim.z > 1 the slices
// write their partial sums to planes of a workspace; the last workgroup to
// arrive at a tile (device-scope counter, release/acquire fences) adds the
// planes, runs the epilogue and clears the counter for the next call.
// OWN_ROWSUM (MB == 1): the activation row sums come from one extra MFMA per
// k-step against an all-ones B operand instead of the caller.
#ifndef XT_MM_SLICE
#define XT_MM_SLICE 1
#endif
template <int FMT, int MB, int NB, int WAVES, int PF, bool OWN_ROWSUM>
__global__ __launch_bounds__(WAVES * 64) void mm_kernel(const MMArgs a) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    constexpr int NBLK = MB * NB;
    constexpr int NACC = NBLK + (OWN_ROWSUM ? 1 : 0);
    static_assert(!OWN_ROWSUM || MB == 1, "in-kernel row sums need MB == 1");
    __shared__ v4i red[WAVES][NACC][64];
    __shared__ int last_flag;
    // SLICE (one 16-token block, 2-bit tiles): each activation load covers
    // 4 token rows x 256 bytes, one distinct 16-byte piece per lane, instead
    // of 16 rows x 64 bytes (an instruction spanning 16 rows at the row
    // stride kept the address path stalled on translation); the pieces go
    // through a wave-private LDS slice (rows padded by one piece) and come
    // back as MFMA fragments.  No barrier: a wave's LDS accesses complete in
    // order.
    constexpr bool SLICE = XT_MM_SLICE && FMT != XT_PACK5 && MB == 1 &&
                           WAVES * NACC * 1024 + WAVES * PF * 16 * 17 * 16 <= 150 * 1024;
    __shared__ v4i aslice[WAVES][SLICE ? PF : 1][SLICE ? 16 * 17 : 1];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int j = lane & 15;

    // Which projection this workgroup belongs to (constant-index selects keep
    // the kernel-argument struct out of scratch memory).
    const int bx = blockIdx.x;
    const ProjView pv = select_proj(proj_bounds(), bx);
    const uint8_t* tiles = pv.tiles;
    const float* ws = pv.ws;
    float* y = pv.y;
    int32_t* accout = pv.acc;
    const int N = pv.N;
    const int tile0 = pv.tile0;
    const int col0 = pv.col0;
    const int ntile = bx - tile0;
    const int NG = (N + 15) >> 4;
    const int M = a.M;
    const int mbase = blockIdx.y * (16 * MB);
    const int nch = a.nch;
    const int ldq = a.ldq;
    const int cbeg = blockIdx.z * a.cps;
    const int cend = min(nch, cbeg + a.cps);
    const int8_t* const qbase = a.q;
    // (consumed here, so the activation pointer and strides are loaded with
    // the projection's fields rather than in a third round inside the loop)
    asm volatile("" ::"s"(qbase), "s"(ldq), "s"(nch), "s"(M), "s"(cend), "s"(tiles));

    v4i acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = v4i{0, 0, 0, 0};
    v4i accs = v4i{0, 0, 0, 0};
    const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
    const v4i zero = v4i{0, 0, 0, 0};

    for (int c0 = cbeg + wave; c0 < cend; c0 += WAVES * PF) {
        v4i wv[PF][NB];
        v4i av[PF][MB][STEPS];
#pragma unroll
        for (int pp = 0; pp < PF; ++pp) {
            const int c = c0 + pp * WAVES;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int G = ntile * NB + nb;
                wv[pp][nb] = (c < cend && G < NG)
                                 ? ld_stream(tiles + ((size_t)(G * nch + c) * 64 + lane) * 16)
                                 : zero;
            }
            if constexpr (SLICE) {
                // (clamped rows and chunk: zeroed when read back)
                const int cc = min(c, cend - 1);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = min(mbase + 4 * u + (lane >> 4), M - 1);
                    av[pp][0][u] = ld_cached(qbase + (size_t)row * ldq + cc * CH + (lane & 15) * 16);
                }
            } else {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int row = mbase + mb * 16 + j;
#pragma unroll
                for (int s = 0; s < STEPS; ++s)
                    av[pp][mb][s] = (c < cend && row < M)
                                        ? ld_cached(qbase + (size_t)row * ldq + c * CH + s * 64 + g * 16)
                                        : zero;
            }
            }
        }
        if constexpr (SLICE) {
            // rows 4u + lane / 16, piece lane % 16 -> the fragments of
            // lane (g, j): row j, pieces 4 s + g
#pragma unroll
            for (int pp = 0; pp < PF; ++pp)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    aslice[wave][pp][(4 * u + (lane >> 4)) * 17 + (lane & 15)] = av[pp][0][u];
            __asm__ volatile("" ::: "memory");
#pragma unroll
            for (int pp = 0; pp < PF; ++pp) {
                const bool live = c0 + pp * WAVES < cend && mbase + j < M;
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    const v4i v = aslice[wave][pp][j * 17 + 4 * s + g];
                    av[pp][0][s] = live ? v : zero;
                }
            }
        }
#pragma unroll
        for (int pp = 0; pp < PF; ++pp) {
            if (c0 + pp * WAVES >= cend) break;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if constexpr (FMT == XT_PACK5) {
                    int E[4], O[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        E[d] = wv[pp][nb][d] & 0x00ff00ff;
                        O[d] = ((unsigned)wv[pp][nb][d] >> 8) & 0x00ff00ff;
                    }
#pragma unroll
                    for (int s = 0; s < STEPS; ++s) {
                        v4i b;
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const int pE = E[d] * 3, pO = O[d] * 3;
                            b[d] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                            E[d] = pE & 0x00ff00ff;
                            O[d] = pO & 0x00ff00ff;
                        }
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma(av[pp][mb][s], b, acc[mb][nb]);
                        if constexpr (OWN_ROWSUM)
                            if (nb == 0) accs = mfma(av[pp][0][s], ones, accs);
                    }
                } else {
#pragma unroll
                    for (int s = 0; s < STEPS; ++s) {
                        const v4i b = decode4(wv[pp][nb][s]);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma(av[pp][mb][s], b, acc[mb][nb]);
                        if constexpr (OWN_ROWSUM)
                            if (nb == 0) accs = mfma(av[pp][0][s], ones, accs);
                    }
                }
            }
        }
    }

    // Reduction over the waves through LDS: every wave parks all its
    // accumulators, then wave w finishes blocks w, w + WAVES, ...
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) red[wave][mb * NB + nb][lane] = acc[mb][nb];
    if constexpr (OWN_ROWSUM) red[wave][NACC - 1][lane] = accs;
    __syncthreads();

    // OWN_ROWSUM: row sums of this slice's activations, laid out like the
    // accumulators (lane (g, j) register r belongs to token 4g + r).
    v4i rs = zero;
    if constexpr (OWN_ROWSUM) {
#pragma unroll
        for (int w = 0; w < WAVES; ++w) rs += red[w][NACC - 1][lane];
    }
    const bool split = gridDim.z > 1;

    if (split) {
        // Publish this slice's partial sums (code domain; an OWN_ROWSUM slice
        // has already subtracted its own share of the row sums) to plane z of
        // the workspace, then count arrivals at this tile.
        int32_t* plane = a.part + (size_t)blockIdx.z * a.M * a.ldp;
        for (int blk = wave; blk < NBLK; blk += WAVES) {
            const int mb = blk / NB, nb = blk % NB;
            v4i sum = zero;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) sum += red[w][blk][lane];
            const int o = (ntile * NB + nb) * 16 + j;
            if (o >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = mbase + mb * 16 + 4 * g + r;
                if (i >= M) continue;
                int ownr = 0;
                if constexpr (OWN_ROWSUM) ownr = rs[r];
                plane[(size_t)i * a.ldp + col0 + o] = sum[r] - ownr;
            }
        }
        __threadfence();  // release: the planes are visible device-wide
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* c = a.cnt + (size_t)blockIdx.y * gridDim.x + blockIdx.x;
            const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (old == gridDim.z - 1);
            if (last_flag) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_flag) return;
        __threadfence();  // acquire: see every other slice's plane
    }

    for (int blk = wave; blk < NBLK; blk += WAVES) {
        const int mb = blk / NB, nb = blk % NB;
        v4i sum = zero;
        if (!split) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) sum += red[w][blk][lane];
        }
        const int o = (ntile * NB + nb) * 16 + j;
        if (o >= N) continue;
        const float wscale = ws[o];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = mbase + mb * 16 + 4 * g + r;
            if (i >= M) continue;
            int d;
            if (split) {
                const size_t off = (size_t)i * a.ldp + col0 + o;
                const size_t plane_sz = (size_t)a.M * a.ldp;
                int tot = 0;
                for (unsigned z = 0; z < gridDim.z; ++z)
                    tot += __builtin_nontemporal_load(a.part + z * plane_sz + off);
                d = OWN_ROWSUM ? tot : tot - a.rowsum[i];
            } else {
                d = sum[r] - (OWN_ROWSUM ? rs[r] : a.rowsum[i]);
            }
            // layers.rs:294 — (dot as f32 * inv_scale) * w_scale, two roundings.
            y[(size_t)i * N + o] = __fmul_rn(__fmul_rn((float)d, a.inv[i]), wscale);
            if (accout) accout[(size_t)i * N + o] = d;
        }
    }
}

template <int FMT, int MB, int NB, int W, int PF, bool OWN>
static hipError_t launch_t(const MMArgs& a, int ntiles, int splitk, hipStream_t s) {
    dim3 grid(ntiles, (a.M + 16 * MB - 1) / (16 * MB), splitk);
    hipLaunchKernelGGL((mm_kernel<FMT, MB, NB, W, PF, OWN>), grid, dim3(W * 64), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode GEMV (M <= 16): activations staged in LDS, all weights in flight
// ---------------------------------------------------------------------------
//
// Workgroup x owns the 16 output rows of row group x (or of the projection
// x falls in) over the full reduction dimension.  The M <= 16 activation
// rows go to LDS once ([chunk][step][g][token][16 B], only real tokens), so
// each wave keeps nothing but weights in registers: wave w loads chunks
// w, w + WAVES, ... (at most NCW each) before its first MFMA, one HBM round
// trip for the whole row group.  The exact row sums are taken while staging
// (v_dot4 against 1s, LDS atomics); the epilogue's scales are loaded at entry;
// waves are summed through LDS.
template <int FMT, int WAVES, int NCW>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const MMArgs a) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    // 1 KiB tiles per chunk, and the weight code offset the activation row
    // sum removes: ternary codes are w + 1, Int4 codes q + 8, Int8 none.
    constexpr int TPC = (FMT == XT_INT8) ? 4 : (FMT == XT_INT4 ? 2 : 1);
    constexpr int OFF = (FMT == XT_INT8) ? 0 : (FMT == XT_INT4 ? 8 : 1);
    constexpr int SEGS = CH / 16;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ v4i red[WAVES][64];
    __shared__ int rsum[16];
    __shared__ unsigned rmax[16];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int j = lane & 15;

    const int bx = blockIdx.x;
    const ProjView pv = select_proj(proj_bounds(), bx);
    const uint8_t* tiles = pv.tiles;
    const float* ws = pv.ws;
    float* y = pv.y;
    int32_t* accout = pv.acc;
    const int N = pv.N;
    const int tile0 = pv.tile0;
    const int G = bx - tile0;
    const int M = a.M;
    const int nch = a.nch;
    if (threadIdx.x < 16) rsum[threadIdx.x] = 0;

    // weights first: they come from HBM and take longest
    v4i wv[NCW][TPC];
#pragma unroll
    for (int t = 0; t < NCW; ++t) {
        const int c = wave + t * WAVES;
#pragma unroll
        for (int u = 0; u < TPC; ++u)
            wv[t][u] = c < nch ? ld_stream(tiles + (((size_t)(G * nch + c) * TPC + u) * 64 + lane) * 16)
                               : v4i{0, 0, 0, 0};
    }
    // epilogue operands, so no memory round trip is left after the MFMAs
    const int o = G * 16 + j;
    const float wscale = (wave == 0 && o < N) ? ws[o] : 0.0f;
    float invr[4];
    const bool fused = a.x != nullptr;
#pragma unroll
    for (int r = 0; r < 4; ++r) invr[r] = (!fused && wave == 0 && 4 * g + r < M) ? a.inv[4 * g + r] : 0.0f;
    if (threadIdx.x < 16) rmax[threadIdx.x] = 0u;
    __syncthreads();  // rsum / rmax cleared

    const int pieces = M * nch * SEGS;
    if (fused) {
        // Quantiser fused (quantization.rs:95-195, as quantize_kernel): every
        // piece (16 columns of one row) is read as f32, the row absmax is
        // gathered through LDS, then the piece is quantised into the stage.
        // The caller guarantees at most one piece per thread.
        const int p = threadIdx.x;
        const int m = p % M;
        const int seg = (p / M) % SEGS;
        const int c = p / (M * SEGS);
        const int col = c * CH + seg * 16;
        float f[16];
        float mx = 0.0f;
        if (p < pieces) {
            const float* xr = a.x + (size_t)m * a.ldx + col;
            if (col + 16 <= a.K && ((((uintptr_t)xr) & 15) == 0)) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float4 v = reinterpret_cast<const float4*>(xr)[t];
                    f[4 * t] = v.x;
                    f[4 * t + 1] = v.y;
                    f[4 * t + 2] = v.z;
                    f[4 * t + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t) f[t] = col + t < a.K ? xr[t] : 0.0f;
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) mx = fmaxf(mx, fabsf(f[t]));  // NaN ignored
            atomicMax(&rmax[m], __float_as_uint(mx));  // non-negative floats order as ints
        }
        __syncthreads();
        if (p < pieces) {
            const float rmx = __uint_as_float(rmax[m]);
            const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
            const int kmain = (a.K / 16) * 16;
            v4i v;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                unsigned w4 = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int k = col + 4 * d + t;
                    const int b = k < a.K ? quant_one(f[4 * d + t], scale, a.mode, k < kmain) : 0;
                    w4 |= (unsigned)(b & 255) << (8 * t);
                }
                v[d] = (int)w4;
            }
            int part = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) part = __builtin_amdgcn_sdot4(v[d], 0x01010101, part, false);
            atomicAdd(&rsum[m], part);
            const int st = seg >> 2, gg = seg & 3;
            *reinterpret_cast<v4i*>(lds + ((((c * STEPS + st) * 4 + gg) * M + m) << 4)) = v;
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float rmx = __uint_as_float(rmax[4 * g + r]);
                invr[r] = (4 * g + r < M) ? ((rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f) : 0.0f;
            }
        }
    } else {
        // activations -> LDS, with exact per-token byte sums (v_dot4 by 1s)
        for (int p = threadIdx.x; p < pieces; p += WAVES * 64) {
            const int m = p % M;
            const int seg = (p / M) % SEGS;
            const int c = p / (M * SEGS);
            const v4i v = ld_cached(a.q + (size_t)m * a.ldq + (size_t)c * CH + seg * 16);
            int part = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) part = __builtin_amdgcn_sdot4(v[d], 0x01010101, part, false);
            atomicAdd(&rsum[m], part);
            const int st = seg >> 2, gg = seg & 3;
            *reinterpret_cast<v4i*>(lds + ((((c * STEPS + st) * 4 + gg) * M + m) << 4)) = v;
        }
        __syncthreads();
    }

    // one accumulator per k-step: short dependent MFMA chains
    v4i acc[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) acc[s] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NCW; ++t) {
        const int c = wave + t * WAVES;
        if (c < nch) {
            if constexpr (FMT == XT_PACK5) {
                int E[4], O[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    E[d] = wv[t][0][d] & 0x00ff00ff;
                    O[d] = ((unsigned)wv[t][0][d] >> 8) & 0x00ff00ff;
                }
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    v4i b;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int pE = E[d] * 3, pO = O[d] * 3;
                        b[d] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                        E[d] = pE & 0x00ff00ff;
                        O[d] = pO & 0x00ff00ff;
                    }
                    v4i av = v4i{0, 0, 0, 0};
                    if (j < M)
                        av = *reinterpret_cast<const v4i*>(lds + ((((c * STEPS + s) * 4 + g) * M + j) << 4));
                    acc[s] = mfma(av, b, acc[s]);
                }
            } else {
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    v4i av = v4i{0, 0, 0, 0};
                    if (j < M)
                        av = *reinterpret_cast<const v4i*>(lds + ((((c * STEPS + s) * 4 + g) * M + j) << 4));
                    v4i b;
                    if constexpr (FMT == XT_INT8) {
                        b = wv[t][s];
                    } else if constexpr (FMT == XT_INT4) {
#pragma unroll
                        for (int d = 0; d < 4; ++d)  // tiles hold the codes q + 8
                            b[d] = (int)(((unsigned)wv[t][s >> 1][d] >> (4 * (s & 1))) & 0x0f0f0f0fu);
                    } else {
                        b = decode4(wv[t][0][s]);
                    }
                    acc[s] = mfma(av, b, acc[s]);
                }
            }
        }
    }
#pragma unroll
    for (int s = 1; s < STEPS; ++s) acc[0] += acc[s];

    red[wave][lane] = acc[0];
    __syncthreads();
    if (wave != 0) return;
    v4i sum = v4i{0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < WAVES; ++w) sum += red[w][lane];
    if (o >= N) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = 4 * g + r;
        if (i >= M) continue;
        const int d = sum[r] - OFF * rsum[i];
        // layers.rs:294 — (dot as f32 * inv_scale) * w_scale, two roundings.
        y[(size_t)i * N + o] = __fmul_rn(__fmul_rn((float)d, invr[r]), wscale);
        if (accout) accout[(size_t)i * N + o] = d;
    }
}

// LDS budget for staged activations and the chunk bound per wave.
constexpr int kGemvLds = 96 * 1024;

// chunks per wave each compiled GEMV width can hold
int gemv_ncw(int waves) { return waves == 16 ? 4 : waves == 8 ? 8 : 16; }

bool gemv_fits(int fmt, int M, int nch, int waves, int ncw) {
    const int ch = fmt == XT_PACK5 ? 320 : 256;
    return M >= 1 && M <= 16 && (size_t)M * nch * ch <= (size_t)kGemvLds &&
           (nch + waves - 1) / waves <= ncw;
}

// ---------------------------------------------------------------------------
// Decode GEMV for ternary formats without staging (M <= 16, q given)
// ---------------------------------------------------------------------------
//
// Workgroup x owns the 16 output rows of row group x (of the projection x
// falls in) over all of K; wave w takes chunks w, w + WAVES, ...  Every lane
// loads its weight slot and its four (Pack5: five) 16-byte activation pieces
// straight from memory -- no LDS stage, no barrier before the MFMAs -- and all
// loads are unconditional (clamped indices, zero-selected afterwards), so
// they issue back to back.  Codes are decoded to signed weights with one
// v_perm_b32 (code 0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0), so no activation row
// sum is needed.  Waves are summed through LDS once at the end.

// FUSED: the kernel quantises the f32 rows a.x itself (quantization.rs:95-195,
// as quantize_kernel): each lane reads its pieces as f32, the per-token
// absmax goes through the waves' shuffles and LDS (one barrier), then each
// lane quantises its own pieces.  No separate quantiser launch.
// AM > 0 (M <= AM, q given): the wave's activation bytes (rows < M of its
// chunks, 256 / 320 bytes each) are loaded once, one distinct 16-byte piece
// per lane, passed through a wave-private LDS slice and read back as MFMA
// fragments, instead of every lane loading its four / five pieces from
// memory (16 token lanes per fragment, most of them duplicates for small M).
template <int FMT, int WAVES, int NCW, bool FUSED, int RG, int AM = 0>
__global__ __launch_bounds__(WAVES * 64) void gemv2_kernel(const MMArgs a) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    // 1 KiB tiles per chunk: Int8 one per k-step, Int4 one per two k-steps
    constexpr int TPC = (FMT == XT_INT8) ? 4 : (FMT == XT_INT4 ? 2 : 1);
    constexpr int APR = NCW * CH / 16;                   // pieces per row and wave
    constexpr int APS = APR + 1;                         // row stride in the slice: one
                                                         // piece of padding, so the rows
                                                         // of a fragment read hit distinct banks
    constexpr int APW = AM > 0 ? AM * APR : 1;           // pieces per wave
    constexpr int ALL = (APW + 63) / 64;                 // of them per lane
    __shared__ v4i red[WAVES][RG][64];
    __shared__ v4i aslice[WAVES][AM == 16 ? 16 * 17 : (AM > 0 ? AM * APS : 1)];
    __shared__ unsigned tmax[WAVES][16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int j = lane & 15;
    const int bx = blockIdx.x;
    const int M = a.M;
    const int nch = a.nch;
    const int ldq = a.ldq;
    const int8_t* q = a.q;
    const float* inv = a.inv;
    const ProjBounds pb = proj_bounds();
    __builtin_amdgcn_sched_barrier(0);  // one round of argument loads
    const ProjView pv = select_proj(pb, bx);
    const int N = pv.N;
    const int NG = (N + 15) >> 4;
    const int G0 = (bx - pv.tile0) * RG;  // first row group of the workgroup

    // epilogue operands (wave w < RG finishes row group G0 + w: tokens
    // 4g + r, output row o)
    const int o = (G0 + min(wave, RG - 1)) * 16 + j;
    const float wscale = pv.ws[min(o, N - 1)];
    float invr[4];
    if constexpr (!FUSED) {
#pragma unroll
        for (int r = 0; r < 4; ++r) invr[r] = inv[min(4 * g + r, M - 1)];
    }

    const uint8_t* wsrc[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r)
        wsrc[r] = pv.tiles + ((size_t)min(G0 + r, NG - 1) * nch * TPC * 64 + lane) * 16;
    v4i wv[NCW][RG][TPC];
    v4i av[NCW][STEPS];
    if constexpr (AM == 16) {
        // 9-16 rows of 2-bit tiles: each activation load covers 4 token rows
        // x 256 bytes of one chunk (one instruction spanning 16 rows at the
        // row stride stalls the address path on translation); chunk by
        // chunk the 16 rows go through the wave's LDS slice (rows padded by
        // one piece) and come back as MFMA fragments.
        static_assert(!FUSED && FMT != XT_PACK5, "AM 16: quantised rows, 256-column chunks");
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int u = 0; u < 4; ++u)  // (rows >= M clamped, zeroed at the MFMA)
                av[t][u] = ld_cached(q + (size_t)min(4 * u + (lane >> 4), M - 1) * ldq + (size_t)c * CH +
                                     (lane & 15) * 16);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int r = 0; r < RG; ++r)
#pragma unroll
                for (int u = 0; u < TPC; ++u)
                    wv[t][r][u] = ld_stream(wsrc[r] + ((size_t)c * TPC + u) * kTileBytes);
        }
        __builtin_amdgcn_sched_barrier(0);
        // (a wave's LDS accesses complete in order: each chunk's reads see
        // its stores, and precede the next chunk's stores)
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
#pragma unroll
            for (int u = 0; u < 4; ++u) aslice[wave][(4 * u + (lane >> 4)) * 17 + (lane & 15)] = av[t][u];
            __asm__ volatile("" ::: "memory");
#pragma unroll
            for (int st = 0; st < 4; ++st) av[t][st] = aslice[wave][j * 17 + 4 * st + g];
            __asm__ volatile("" ::: "memory");
        }
    } else if constexpr (AM > 0) {
        static_assert(!FUSED, "AM takes quantised rows");
        const int npc = M * APR;  // pieces of rows < M
        v4i ap[ALL];
#pragma unroll
        for (int u = 0; u < ALL; ++u) {
            const int p = min(lane + 64 * u, npc - 1);
            const int m = p / APR, pr = p - m * APR;
            const int c = min(wave + (pr / (CH / 16)) * WAVES, nch - 1);
            ap[u] = ld_cached(q + (size_t)m * ldq + (size_t)c * CH + (pr % (CH / 16)) * 16);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int r = 0; r < RG; ++r)
#pragma unroll
                for (int u = 0; u < TPC; ++u)
                    wv[t][r][u] = ld_stream(wsrc[r] + ((size_t)c * TPC + u) * kTileBytes);
        }
        __builtin_amdgcn_sched_barrier(0);
        // (a wave's LDS accesses complete in order: the reads below see
        // these stores without a barrier)
#pragma unroll
        for (int u = 0; u < ALL; ++u)
            if (lane + 64 * u < npc) aslice[wave][lane + 64 * u + (lane + 64 * u) / APR] = ap[u];
        __asm__ volatile("" ::: "memory");
        const int jr = min(j, M - 1) * APS;
#pragma unroll
        for (int t = 0; t < NCW; ++t)
#pragma unroll
            for (int s = 0; s < STEPS; ++s) av[t][s] = aslice[wave][jr + t * (CH / 16) + 4 * s + g];
    } else if constexpr (!FUSED) {
        const int8_t* arow = q + (size_t)min(j, M - 1) * ldq + 16 * g;
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int r = 0; r < RG; ++r)
#pragma unroll
                for (int u = 0; u < TPC; ++u)
                    wv[t][r][u] = ld_stream(wsrc[r] + ((size_t)c * TPC + u) * kTileBytes);
#pragma unroll
            for (int s = 0; s < STEPS; ++s) av[t][s] = ld_cached(arow + (size_t)c * CH + s * 64);
        }
    } else {
        // Cooperative quantisation: thread t takes float4 pieces t, t + NT,
        // ... of the M x K rows (K % 4 == 0, so a piece never straddles two
        // rows), gathers each token's absmax through LDS, quantises its
        // pieces into the A-operand stage [chunk][step][g][token 0..15][16 B],
        // and after a barrier every lane reads its fragments.  Stage bytes of
        // columns >= K are never written; their weights are padding code 1,
        // which decodes to 0.
        extern __shared__ __align__(16) uint8_t stage[];
        const int K = a.K;
        constexpr int NT = WAVES * 64;
        const int n4 = (M * K) >> 2;
        // One row: lane l of wave w loads float4 piece l of each chunk the
        // wave multiplies (chunks w + t WAVES), and for Pack5's 80-piece
        // chunks also piece 64 + l (l < 16), so every lane finds its A
        // fragment in the packed bytes of four lanes of its own wave
        // (ds_bpermute, no LDS stage); the row maximum comes from per-wave
        // maxima (no atomics, so no clearing barrier).  One barrier in all.
        constexpr int PPC = CH / 4;  // float4 pieces per chunk: 64 or 80
        bool one_pass = false;
        if constexpr (FMT == XT_PACK4 || FMT == XT_PACK5) one_pass = M == 1;
        if (one_pass) {
            float4 x0[NCW], x1[NCW];
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
                const int f = (wave + t * WAVES) * PPC + lane;
                x0[t] = x1[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (f < n4) x0[t] = *reinterpret_cast<const float4*>(a.x + 4 * f);
                if constexpr (PPC > 64)
                    if (lane < PPC - 64 && f + 64 < n4) x1[t] = *reinterpret_cast<const float4*>(a.x + 4 * (f + 64));
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
                const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
                for (int r = 0; r < RG; ++r)
#pragma unroll
                    for (int u = 0; u < TPC; ++u)
                        wv[t][r][u] = ld_stream(wsrc[r] + ((size_t)c * TPC + u) * kTileBytes);
            }
            __builtin_amdgcn_sched_barrier(0);
            // (non-negative floats order as their bit patterns; NaN is ignored)
            auto amax = [](float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
            float mx = 0.0f;
#pragma unroll
            for (int t = 0; t < NCW; ++t) mx = fmaxf(mx, fmaxf(amax(x0[t]), amax(x1[t])));
            const int wm = wave_reduce_bits(__float_as_int(mx), [](int p, int q) {
                return __float_as_int(fmaxf(__int_as_float(p), __int_as_float(q)));
            });
            if (lane == 0) tmax[wave][0] = (unsigned)wm;
            __syncthreads();
            unsigned mb = 0u;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) mb = max(mb, tmax[w][0]);
            const float rmx = __uint_as_float(mb);
            const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
            const float iv = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) invr[r] = iv;
            const int kmain = (K / 16) * 16;
            unsigned w4[NCW], w5[NCW];
            auto pack = [&](auto mode_c) {
                auto q4 = [&](float4 v, int f) {
                    const int col = 4 * f;
                    const float e4[4] = {v.x, v.y, v.z, v.w};
                    unsigned r = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        r |= (unsigned)(quant_one(e4[e], scale, decltype(mode_c)::value, col + e < kmain) & 255)
                             << (8 * e);
                    return f < n4 ? r : 0u;  // columns past K: zero activations
                };
#pragma unroll
                for (int t = 0; t < NCW; ++t) {
                    const int f = (wave + t * WAVES) * PPC + lane;
                    w4[t] = q4(x0[t], f);
                    w5[t] = PPC > 64 ? q4(x1[t], f + 64) : 0u;
                }
            };
            if (a.mode == XT_QUANT_AVX512) pack(std::integral_constant<int, XT_QUANT_AVX512>{});
            else pack(std::integral_constant<int, XT_QUANT_SCALAR>{});
            // lane (g, j) of step s takes chunk pieces 16 s + 4 g + d: lanes
            // 0..63 of the first packed value, then lanes 0..15 of the second
#pragma unroll
            for (int t = 0; t < NCW; ++t)
#pragma unroll
                for (int st = 0; st < STEPS; ++st)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int idx = 16 * st + 4 * g + d;
                        av[t][st][d] = st < 4 ? __builtin_amdgcn_ds_bpermute(idx << 2, (int)w4[t])
                                              : __builtin_amdgcn_ds_bpermute((idx - 64) << 2, (int)w5[t]);
                    }
        } else {
        if (threadIdx.x < 16) tmax[0][threadIdx.x] = 0u;
        // The f32 pieces are loaded before the weights: loads return in
        // order, so the quantiser then waits for its own loads only and runs
        // while the weights are in flight.
        float4 xv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int f = threadIdx.x + u * NT;
            if (f < n4) {
                const int m = (4 * f) / K, col = 4 * f - m * K;
                xv[u] = *reinterpret_cast<const float4*>(a.x + (size_t)m * a.ldx + col);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int r = 0; r < RG; ++r)
#pragma unroll
                for (int u = 0; u < TPC; ++u)
                    wv[t][r][u] = ld_stream(wsrc[r] + ((size_t)c * TPC + u) * kTileBytes);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // tmax cleared
        // (non-negative floats order as their bit patterns; NaN is ignored)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int f = threadIdx.x + u * NT;
            const int f0 = wave * 64 + u * NT;  // first piece of this wave
            if (f0 >= n4) continue;
            const float mx = f < n4 ? fmaxf(fmaxf(fabsf(xv[u].x), fabsf(xv[u].y)),
                                            fmaxf(fabsf(xv[u].z), fabsf(xv[u].w)))
                                    : 0.0f;
            const int m0 = (4 * f0) / K, m1 = (4 * min(f0 + 63, n4 - 1)) / K;
            if (m0 == m1) {  // the wave's pieces lie in one row: one atomic per wave
                const int wm = wave_reduce_bits(__float_as_int(mx), [](int x, int y) {
                    return __float_as_int(fmaxf(__int_as_float(x), __int_as_float(y)));
                });
                if (lane == 0) atomicMax(&tmax[0][m0], (unsigned)wm);
            } else if (f < n4) {
                atomicMax(&tmax[0][(4 * f) / K], __float_as_uint(mx));
            }
        }
        __syncthreads();
        const int kmain = (K / 16) * 16;
        // (the rounding mode is chosen once, so that only one quantiser's
        // code runs through the unrolled loop)
        auto quant_pieces = [&](auto mode_c) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int f = threadIdx.x + u * NT;
                if (f < n4) {
                    const int m = (4 * f) / K, col = 4 * f - m * K;
                    const float rmx = __uint_as_float(tmax[0][m]);
                    const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
                    const float e4[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
                    unsigned w4 = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w4 |= (unsigned)(quant_one(e4[e], scale, decltype(mode_c)::value, col + e < kmain) & 255)
                              << (8 * e);
                    const int c = col / CH, r = col - c * CH, st = r >> 6, gg = (r >> 4) & 3;
                    *reinterpret_cast<unsigned*>(stage + ((((c * STEPS + st) * 4 + gg) * 16 + m) << 4) + (col & 15)) = w4;
                }
            }
        };
        if (a.mode == XT_QUANT_AVX512) quant_pieces(std::integral_constant<int, XT_QUANT_AVX512>{});
        else quant_pieces(std::integral_constant<int, XT_QUANT_SCALAR>{});
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const int c = min(wave + t * WAVES, nch - 1);
#pragma unroll
            for (int s = 0; s < STEPS; ++s)
                av[t][s] = *reinterpret_cast<const v4i*>(stage + ((((c * STEPS + s) * 4 + g) * 16 + j) << 4));
        }
        // inverse scales of tokens 4g + r (wave 0 finishes)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float x2 = __uint_as_float(tmax[0][min(4 * g + r, 15)]);
            invr[r] = (x2 > 0.0f) ? __fdiv_rn(x2, 127.0f) : 1.0f;
        }
        }
    }
    v4i acc[RG][STEPS];
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int s = 0; s < STEPS; ++s) acc[r][s] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NCW; ++t) {
        const bool live = wave + t * WAVES < nch;
#pragma unroll
        for (int r = 0; r < RG; ++r) {
            if constexpr (FMT == XT_PACK5) {
                int E[4], O[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    E[d] = wv[t][r][0][d] & 0x00ff00ff;
                    O[d] = ((unsigned)wv[t][r][0][d] >> 8) & 0x00ff00ff;
                }
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    v4i b;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int pE = E[d] * 3, pO = O[d] * 3;
                        b[d] = signed_codes((int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u));
                        E[d] = pE & 0x00ff00ff;
                        O[d] = pO & 0x00ff00ff;
                    }
                    const v4i x = (live && j < M) ? av[t][s] : v4i{0, 0, 0, 0};
                    acc[r][s] = mfma(x, b, acc[r][s]);
                }
            } else {
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    v4i b;
                    if constexpr (FMT == XT_INT8) {
                        b = wv[t][r][s];
                    } else if constexpr (FMT == XT_INT4) {
                        // code c = q + 8 -> (c ^ 8) in the high nibble is the
                        // signed byte 16 q; the sum is divided by 16 at the end
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const unsigned w = (unsigned)wv[t][r][s >> 1][d] ^ 0x88888888u;
                            b[d] = (int)(((s & 1) ? w : (w << 4)) & 0xf0f0f0f0u);
                        }
                    } else {
                        b = decode4(wv[t][r][0][s]);
#pragma unroll
                        for (int d = 0; d < 4; ++d) b[d] = signed_codes(b[d]);
                    }
                    const v4i x = (live && j < M) ? av[t][s] : v4i{0, 0, 0, 0};
                    acc[r][s] = mfma(x, b, acc[r][s]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
#pragma unroll
        for (int s = 1; s < STEPS; ++s) acc[r][0] += acc[r][s];
        red[wave][r][lane] = acc[r][0];
    }
    __syncthreads();
    if (wave >= RG || o >= N) return;
    v4i sum = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[w][wave][lane];
    if constexpr (FMT == XT_INT4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] >>= 4;  // exact: every term is a multiple of 16
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = 4 * g + r;
        if (i >= M) continue;
        // layers.rs:294 — (dot as f32 * inv_scale) * w_scale, two roundings.
        pv.y[(size_t)i * N + o] = __fmul_rn(__fmul_rn((float)sum[r], invr[r]), wscale);
        if (pv.acc) pv.acc[(size_t)i * N + o] = sum[r];
    }
}

// Row groups per workgroup of the staging-free GEMV: the most (4, 2, 1)
// that leave at least 200 workgroups and at most 80 KiB of weights per
// workgroup.  Measured (MI355X, rotating weights, µs at M = 1 / 16 for 1, 2,
// 4 groups): C0 2560 -> 6912 3.7 / 3.5 / 4.1 at M = 1; 4096 -> 14336 7.5 /
// 5.9 / 5.3 and 11.8 / 7.9 / 6.4; 2560 -> 32768 at M = 16 14.3 / 11.1 / 7.8;
// Int4 head 128256 rows 33.3 / 29.7 / 27.9; Int8 head 48.9 / 49.9 / 52.1 at
// M = 1 and 72.6 / 61.9 / 61.1 at M = 16.  Pack5 never takes two (3200 ->
// 8640: 5.3 / 6.1 / 6.1; 3200 -> 32000: 11.0 / 12.1 / 9.3).
static int gemv2_rg_for(int fmt, int nch, int ngroups) {
    const int tpc = fmt == XT_INT8 ? 4 : (fmt == XT_INT4 ? 2 : 1);
    for (int rg : {4, 2})
        if (ngroups / rg >= 200 && rg * nch * tpc * kTileBytes <= 80 * 1024 &&
            !(fmt == XT_PACK5 && rg == 2))
            return rg;
    return 1;
}

// Waves of the staging-free GEMV for nch chunks, and the most f32 elements
// (M * K) its fused quantiser takes: 8 float4 per thread.
static int gemv2_waves(int nch) {
    for (int w : {4, 8, 10, 16})
        if (nch <= w) return w;
    // (as the launcher's list: 14 waves where they cover K at 2, 3 or 4
    // chunks per wave)
    return (nch <= 28 || (nch > 32 && nch <= 42) || (nch > 48 && nch <= 56)) ? 14 : 16;
}
// LDS of the fused GEMV: the A stage (1 KiB per k-step) plus the static
// cross-wave sums and maxima; it must fit the 160 KiB of a CU.
static size_t gemv2_fused_lds(int nch, int steps, int rg) {
    const int w = gemv2_waves(nch);
    return (size_t)nch * steps * 1024 + (size_t)w * rg * 64 * 16 + (size_t)w * 16 * 4;
}
constexpr size_t kLdsBytes = 160 * 1024;
int gemv2_fused_max(int fmt, int nch, int rg) {
    if (nch > 64 || gemv2_fused_lds(nch, fmt == XT_PACK5 ? 5 : 4, rg) > kLdsBytes) return 0;
    return gemv2_waves(nch) * 64 * 32;
}

// Quantised rows given: the activation pieces through a wave-private LDS
// slice when the wave multiplies two or more chunks and the slice of M rows
// fits (measured: 14336 -> 4096 at M = 1 / 4 6.42 -> 5.24-5.39 / 6.93 ->
// 6.04 us; Pack5 3200 -> 8640 at M = 1 / 8 4.80 -> 4.48-4.54 / 5.99 ->
// 5.23; with one chunk per wave it did not help: 4096 -> 14336 at M = 1
// 5.33 -> 5.55).
template <int FMT, int W, int NCW, int RG, int AM>
static constexpr bool gemv2_am_fits() {
    return (size_t)W * AM * (NCW * (FMT == XT_PACK5 ? 320 : 256) + 16) + (size_t)W * RG * 1024 <= 120 * 1024;
}
template <int FMT, int W, int NCW, int RG>
static hipError_t launch_gemv2_am(const MMArgs& a, int ntiles, hipStream_t s) {
    const dim3 g(ntiles), b(W * 64);
    if constexpr (NCW >= 2) {
        if (a.M == 1) {
            hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG, 1>), g, b, 0, s, a);
            return hipGetLastError();
        }
        if constexpr (gemv2_am_fits<FMT, W, NCW, RG, 4>()) {
            if (a.M <= 4) {
                hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG, 4>), g, b, 0, s, a);
                return hipGetLastError();
            }
        }
        if constexpr (gemv2_am_fits<FMT, W, NCW, RG, 8>()) {
            if (a.M <= 8) {
                hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG, 8>), g, b, 0, s, a);
                return hipGetLastError();
            }
        }
    }
    // 5-16 rows of 2-bit tiles the slices above do not take: 4-row loads,
    // staged chunk by chunk (measured: TA address stalls 68 % -> see the
    // profile of this kernel)
    if constexpr (FMT == XT_PACK4 && (size_t)W * (16 * 17 * 16 + RG * 1024) <= 150 * 1024) {
        if (a.M > 4 && a.M <= 16) {
            hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG, 16>), g, b, 0, s, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG>), g, b, 0, s, a);
    return hipGetLastError();
}

// Int8 rows given: 5-16 rows take the 4-row activation loads staged through
// the LDS slice, as the ternary tiles do (measured on the 128256-row head at
// M = 16: Int8 63.2 -> 60.2 us; Int4 36.4 -> 38.1, so Int4 keeps the direct
// loads).
template <int FMT, int W, int NCW, int RG>
static hipError_t launch_gemv2_int(const MMArgs& a, int ntiles, hipStream_t s) {
    const dim3 g(ntiles), b(W * 64);
    if constexpr (FMT == XT_INT8 && (size_t)W * (16 * 17 * 16 + RG * 1024) <= 150 * 1024) {
        if (a.M > 4 && a.M <= 16) {
            hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG, 16>), g, b, 0, s, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv2_kernel<FMT, W, NCW, false, RG>), g, b, 0, s, a);
    return hipGetLastError();
}

// The staging-free GEMV applies to ternary tiles (given or fused-quantised rows).
template <int RG>
static hipError_t launch_gemv2_rg(int fmt, const MMArgs& a, int ntiles, hipStream_t s) {
    const int nch = a.nch;
    // fused rows: at most 8 float4 per thread, A stage of 1 KiB per k-step
    const int steps = fmt == XT_PACK5 ? 5 : 4;
    const size_t stage = (size_t)nch * steps * 1024;
    if (a.x && gemv2_fused_lds(nch, steps, RG) > kLdsBytes) return hipErrorInvalidValue;
#define XT_GV2(W_, NCW_)                                                                         \
    if (nch <= W_ * NCW_) {                                                                      \
        if (a.x) {                                                                               \
            if ((size_t)a.M * a.K > (size_t)W_ * 64 * 32) {                                   \
                return hipErrorInvalidValue; /* fused rows: 8 float4 per thread */               \
            } else if (fmt == XT_PACK5) {                                                        \
                hipLaunchKernelGGL((gemv2_kernel<XT_PACK5, W_, NCW_, true, RG>), dim3(ntiles), dim3(W_ * 64), a.M == 1 ? 0 : stage, s, a); \
            } else {                                                                             \
                /* one row in one pass: no LDS stage */                                          \
                const size_t st_ = a.M == 1 ? 0 : stage;                                    \
                hipLaunchKernelGGL((gemv2_kernel<XT_PACK4, W_, NCW_, true, RG>), dim3(ntiles), dim3(W_ * 64), st_, s, a); \
            }                                                                                    \
        } else if (fmt == XT_PACK5) {                                                            \
            return launch_gemv2_am<XT_PACK5, W_, NCW_, RG>(a, ntiles, s);                      \
        } else if (fmt == XT_INT8) {                                                             \
            if constexpr (NCW_ <= 2)                                                             \
                return launch_gemv2_int<XT_INT8, W_, NCW_, RG>(a, ntiles, s);                        \
            else                                                                                 \
                return hipErrorInvalidValue;                                                     \
        } else if (fmt == XT_INT4) {                                                             \
            if constexpr (NCW_ <= 2)                                                             \
                return launch_gemv2_int<XT_INT4, W_, NCW_, RG>(a, ntiles, s);                        \
            else                                                                                 \
                return hipErrorInvalidValue;                                                     \
        } else {                                                                                 \
            return launch_gemv2_am<XT_PACK4, W_, NCW_, RG>(a, ntiles, s);                      \
        }                                                                                        \
        return hipGetLastError();                                                                \
    }
    // Pack5 at 5..10 chunks: five waves of two chunks (measured, 3200 ->
    // 8640: 4.8 vs 5.3 us at M = 1, 6.0 vs 6.2 at M = 8; Pack4 is fastest
    // with one chunk per wave)
    if (fmt == XT_PACK5 && !a.x && nch > 4 && nch <= 10) {
        return launch_gemv2_am<XT_PACK5, 5, 2, RG>(a, ntiles, s);
        return hipGetLastError();
    }
    // Above 16 chunks, 14 waves where they cover K with the same chunks per
    // wave (27 or 28 chunks, 42, 56): fewer idle waves (measured at M = 1 /
    // 8: 6912 -> 2560 4.3 -> 4.1 / 5.3 -> 5.0 us; 14336 -> 4096 6.7 -> 6.3 /
    // 8.3 -> 7.7; Pack5 8640 -> 3200 5.1 -> 5.0 / 5.6 -> 5.5)
    XT_GV2(4, 1) XT_GV2(8, 1) XT_GV2(10, 1) XT_GV2(16, 1) XT_GV2(14, 2) XT_GV2(16, 2)
    XT_GV2(14, 3) XT_GV2(16, 3) XT_GV2(14, 4) XT_GV2(16, 4)
#undef XT_GV2
    return hipErrorInvalidValue;
}

static hipError_t launch_gemv2(int fmt, const MMArgs& a, int ntiles, hipStream_t s) {
    if (a.rg == 4) return launch_gemv2_rg<4>(fmt, a, ntiles, s);
    return a.rg == 2 ? launch_gemv2_rg<2>(fmt, a, ntiles, s) : launch_gemv2_rg<1>(fmt, a, ntiles, s);
}

static bool use_gemv2(int fmt, int nch) {
    if (fmt == XT_INT8 || fmt == XT_INT4) return nch <= 32;  // weight registers: 4 / 2 tiles a chunk
    return (fmt == XT_PACK4 || fmt == XT_PACK5 || fmt == XT_XORSPARSE) && nch <= 64;
}
bool gemv2_takes(int fmt, int nch) { return use_gemv2(fmt, nch); }
int gemv_row_groups(int fmt, int nch, int ngroups) {
    return use_gemv2(fmt, nch) ? gemv2_rg_for(fmt, nch, ngroups) : 1;
}

hipError_t launch_gemv(int fmt, const MMArgs& a, int ntiles, int waves, hipStream_t s) {
    // (Int8 / Int4 rows quantised in the kernel stay on the staged GEMV)
    if (use_gemv2(fmt, a.nch) && !(a.x && is_int_format(fmt)))
        return launch_gemv2(fmt == XT_XORSPARSE ? XT_PACK4 : fmt, a, ntiles, s);
    const int ch = fmt == XT_PACK5 ? 320 : 256;
    const size_t lds = (size_t)a.M * a.nch * ch;
#define XT_GEMV(W_, NCW_)                                                                        \
    if (waves == W_) {                                                                           \
        if (fmt == XT_PACK5)                                                                     \
            hipLaunchKernelGGL((gemv_kernel<XT_PACK5, W_, NCW_>), dim3(ntiles), dim3(W_ * 64), lds, s, a); \
        else if (fmt == XT_INT8)                                                                 \
            hipLaunchKernelGGL((gemv_kernel<XT_INT8, W_, NCW_>), dim3(ntiles), dim3(W_ * 64), lds, s, a); \
        else if (fmt == XT_INT4)                                                                 \
            hipLaunchKernelGGL((gemv_kernel<XT_INT4, W_, NCW_>), dim3(ntiles), dim3(W_ * 64), lds, s, a); \
        else                                                                                     \
            hipLaunchKernelGGL((gemv_kernel<XT_PACK4, W_, NCW_>), dim3(ntiles), dim3(W_ * 64), lds, s, a); \
        return hipGetLastError();                                                                \
    }
    XT_GEMV(4, 16)
    XT_GEMV(8, 8)
    XT_GEMV(2, 16)
    XT_GEMV(16, 4)
#undef XT_GEMV
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Prefill GEMM (M > 16): one load round per workgroup
// ---------------------------------------------------------------------------
//
// Workgroup (x, y, z): 32 tokens (y) x 128 output rows (x) over chunk slice z
// of at most NCMAX chunks.  Its 8 waves are 4 row groups of 32 rows x 2
// chunk groups (even / odd chunks of the slice).  At entry every thread
// issues all of its loads: the activation slice (32 x slice bytes, coalesced
// 16-byte pieces) goes to LDS in MFMA A-operand order
// [chunk][step][token block][lane][16 B], and each wave pulls its own weights
// (32 rows x its chunks) into registers.  After one barrier the waves run
// 2 x 2 accumulator blocks of 16x16x64 i8 MFMAs, prefetching the next
// k-step's A operands from LDS before issuing the current step's MFMAs (two
// waves per SIMD hide the rest).  The two chunk groups are added through LDS.
// gridDim.z == 1 writes y; otherwise the slice's code-domain partial sums go
// to plane z of `part` and gemm_reduce_kernel finishes.
template <int FMT, int NCMAX, int KG>
__global__ __launch_bounds__(256 * KG) void gemm_kernel(const MMArgs a) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    constexpr int SEGS = CH / 16;       // 16-byte pieces per token per chunk
    constexpr int MB = 2;               // token blocks of 16
    constexpr int NBW = 2;              // output-row blocks of 16 per wave
    constexpr int NCW = (NCMAX + KG - 1) / KG;  // chunks per wave
    constexpr int NT = 256 * KG;                 // threads
    extern __shared__ __align__(16) uint8_t lds_a[];
    __shared__ v4i red[KG - 1][4][MB * NBW][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int ngrp = wave & 3;          // row group of 32 rows
    const int kgrp = wave >> 2;         // chunks kgrp, kgrp + KG, ...
    const int g = lane >> 4;
    const int j = lane & 15;

    // Logical tile: token blocks (y) fastest, so the token blocks that read the
    // same weight rows sit on one XCD and share its L2.
    const int gx = gridDim.x, gy = gridDim.y;
    const int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int t = xcd_remap(lin, gx * gy * gridDim.z);
    const int by = t % gy;
    const int bx = (t / gy) % gx;
    const int bz = t / (gx * gy);
    const ProjView pv = select_proj(proj_bounds(), bx);
    const uint8_t* tiles = pv.tiles;
    const float* ws = pv.ws;
    float* y = pv.y;
    int32_t* accout = pv.acc;
    const int N = pv.N;
    const int tile0 = pv.tile0;
    const int col0 = pv.col0;
    const int NG = (N + 15) >> 4;
    const int M = a.M;
    const int mbase = by * 32;
    const int nch = a.nch;
    const int cbeg = bz * a.cps;
    const int nc = min(nch - cbeg, a.cps);  // chunks in this slice (<= NCMAX)
    const int gbase = (bx - tile0) * 8 + ngrp * NBW;  // first row group of this wave

    // Weights of this wave: NBW row groups x its chunks, 16 bytes per lane each.
    v4i wv[NCW][NBW];
#pragma unroll
    for (int u = 0; u < NCW; ++u)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const int cc = kgrp + KG * u;
            const int G = gbase + nb;
            wv[u][nb] = (cc < nc && G < NG)
                            ? *reinterpret_cast<const v4i*>(tiles + ((size_t)(G * nch + cbeg + cc) * 64 + lane) * 16)
                            : v4i{0, 0, 0, 0};
        }

    // Epilogue operands now, so no memory round trip is left after the MFMAs.
    const bool split = gridDim.z > 1;
    float wsc[NBW];
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
        const int o = (gbase + nb) * 16 + j;
        wsc[nb] = (!split && kgrp == 0 && o < N) ? ws[o] : 0.0f;
    }
    float invr[MB][4];
    int rsr[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = mbase + mb * 16 + 4 * g + r;
            const bool ok = !split && kgrp == 0 && i < M;
            invr[mb][r] = ok ? a.inv[i] : 0.0f;
            rsr[mb][r] = ok ? a.rowsum[i] : 0;
        }

    // Activation slice -> LDS, A-operand order.  Pieces are taken in LDS
    // order (lane fastest), so the LDS stores are sequential; the global side
    // reads 64-byte runs of 16 token rows.
    // All of a thread's loads are issued before its first LDS store, so the
    // slice costs one memory round trip, not one per piece.
    const int pieces = 32 * nc * SEGS;
    constexpr int PPT = (32 * NCMAX * SEGS + NT - 1) / NT;  // pieces per thread
    v4i stage[PPT];
#pragma unroll
    for (int r = 0; r < PPT; ++r) {
        const int p = threadIdx.x + r * NT;
        const int ln = p & 63;
        const int blk = p >> 6;                 // (cc * STEPS + st) * MB + mb
        const int mb = blk % MB;
        const int cs = blk / MB;                // cc * STEPS + st
        const int row = mbase + mb * 16 + (ln & 15);
        stage[r] = v4i{0, 0, 0, 0};
        if (p < pieces && row < M)
            stage[r] = ld_cached(a.q + (size_t)row * a.ldq + (size_t)cbeg * CH + cs * 64 + (ln >> 4) * 16);
    }
#pragma unroll
    for (int r = 0; r < PPT; ++r) {
        const int p = threadIdx.x + r * NT;
        if (p < pieces) *reinterpret_cast<v4i*>(lds_a + ((size_t)p << 4)) = stage[r];
    }
    __syncthreads();

    v4i acc[MB][NBW];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) acc[mb][nb] = v4i{0, 0, 0, 0};

    // A operands of k-step (u, s) of this wave; `nxt` is read one step ahead.
    auto a_addr = [&](int u, int st, int mb) {
        return lds_a + (((((kgrp + KG * u) * STEPS + st) * MB + mb) * 64 + lane) << 4);
    };
    v4i cur[MB], nxt[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        cur[mb] = (kgrp < nc) ? *reinterpret_cast<const v4i*>(a_addr(0, 0, mb)) : v4i{0, 0, 0, 0};

#pragma unroll
    for (int u = 0; u < NCW; ++u) {
        if (kgrp + KG * u < nc) {
            int E[NBW][4], O[NBW][4];
            if constexpr (FMT == XT_PACK5) {
#pragma unroll
                for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        E[nb][d] = wv[u][nb][d] & 0x00ff00ff;
                        O[nb][d] = ((unsigned)wv[u][nb][d] >> 8) & 0x00ff00ff;
                    }
            }
#pragma unroll
            for (int st = 0; st < STEPS; ++st) {
                // prefetch the next k-step's operands
                const int nu = (st + 1 < STEPS) ? u : u + 1;
                const int ns = (st + 1 < STEPS) ? st + 1 : 0;
                const bool have_next = (nu < NCW) && (kgrp + KG * nu < nc);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    nxt[mb] = have_next ? *reinterpret_cast<const v4i*>(a_addr(nu, ns, mb))
                                        : v4i{0, 0, 0, 0};
                v4i b[NBW];
#pragma unroll
                for (int nb = 0; nb < NBW; ++nb) {
                    if constexpr (FMT == XT_PACK5) {
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const int pE = E[nb][d] * 3, pO = O[nb][d] * 3;
                            b[nb][d] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                            E[nb][d] = pE & 0x00ff00ff;
                            O[nb][d] = pO & 0x00ff00ff;
                        }
                    } else {
                        b[nb] = decode4(wv[u][nb][st]);
                    }
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NBW; ++nb) acc[mb][nb] = mfma(cur[mb], b[nb], acc[mb][nb]);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) cur[mb] = nxt[mb];
            }
        }
    }

    // Add the odd-chunk waves into the even-chunk waves, stage the 32 x 128
    // tile in LDS (every wave is past its LDS operand reads at the first
    // barrier), then all 512 threads write whole rows with 16-byte stores.
    if (kgrp > 0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NBW; ++nb) red[kgrp - 1][ngrp][mb * NBW + nb][lane] = acc[mb][nb];
    }
    __syncthreads();
    float* ytile = reinterpret_cast<float*>(lds_a);            // [32][128]
    int* dtile = reinterpret_cast<int*>(lds_a + 32 * 128 * 4);  // [32][128]
    if (kgrp == 0) {
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const int col = ngrp * 32 + nb * 16 + j;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = mb * 16 + 4 * g + r;
                    int v = acc[mb][nb][r];
#pragma unroll
                    for (int kk = 0; kk < KG - 1; ++kk) v += red[kk][ngrp][mb * NBW + nb][lane][r];
                    if (split) {
                        dtile[row * 128 + col] = v;
                    } else {
                        const int d = v - rsr[mb][r];
                        // layers.rs:294 — (dot as f32 * inv_scale) * w_scale.
                        ytile[row * 128 + col] = __fmul_rn(__fmul_rn((float)d, invr[mb][r]), wsc[nb]);
                        dtile[row * 128 + col] = d;
                    }
                }
        }
    }
    __syncthreads();
    const int obase = (bx - tile0) * 128;
    int32_t* plane = a.part + (size_t)bz * a.M * a.ldp;
    const bool vec = (N & 3) == 0;
    for (int idx = threadIdx.x; idx < 32 * 32; idx += NT) {
        const int row = idx >> 5, c4 = (idx & 31) * 4;
        const int i = mbase + row, o = obase + c4;
        if (i >= M || o >= N) continue;
        if (split) {
            // planes have a padded stride (a multiple of 16 columns)
            *reinterpret_cast<int4*>(plane + (size_t)i * a.ldp + col0 + o) =
                *reinterpret_cast<const int4*>(dtile + row * 128 + c4);
            continue;
        }
        if (vec && o + 3 < N) {
            *reinterpret_cast<float4*>(y + (size_t)i * N + o) =
                *reinterpret_cast<const float4*>(ytile + row * 128 + c4);
            if (accout)
                *reinterpret_cast<int4*>(accout + (size_t)i * N + o) =
                    *reinterpret_cast<const int4*>(dtile + row * 128 + c4);
        } else {
            for (int e2 = 0; e2 < 4 && o + e2 < N; ++e2) {
                y[(size_t)i * N + o + e2] = ytile[row * 128 + c4 + e2];
                if (accout) accout[(size_t)i * N + o + e2] = dtile[row * 128 + c4 + e2];
            }
        }
    }
}

// Sum the split-K planes of every projection and apply the epilogue.
// One thread per (token, workspace column).
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const MMArgs a, int nsplit) {
    const int i = blockIdx.y;
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= a.ldp || i >= a.M) return;
    int p = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q)
        if (q < a.nproj && col >= a.proj[q].col0) p = q;
    const Proj& pr = a.proj[p];
    const int o = col - pr.col0;
    if (o >= pr.N) return;
    const size_t plane_sz = (size_t)a.M * a.ldp;
    int tot = 0;
    for (int z = 0; z < nsplit; ++z) tot += a.part[z * plane_sz + (size_t)i * a.ldp + col];
    const int d = tot - (a.rowsum ? a.rowsum[i] : 0);  // signed-decode kernels pass none
    pr.y[(size_t)i * pr.N + o] = __fmul_rn(__fmul_rn((float)d, a.inv[i]), pr.ws[o]);
    if (pr.acc) pr.acc[(size_t)i * pr.N + o] = d;
}

int gemm_ncmax(int fmt) { return fmt == XT_PACK5 ? 8 : 10; }

hipError_t launch_gemm(int fmt, const MMArgs& a, int ntiles, int splitk, hipStream_t s) {
    const dim3 grid(ntiles, (a.M + 31) / 32, splitk);
    const int ch = fmt == XT_PACK5 ? 320 : 256;
    size_t lds = (size_t)a.cps * ch * 32;
    if (lds < 32 * 128 * 8) lds = 32 * 128 * 8;  // the staged output tile
#ifndef XT_GEMM_KG
#define XT_GEMM_KG 4
#endif
    constexpr int KG = XT_GEMM_KG;
    if (fmt == XT_PACK5)
        hipLaunchKernelGGL((gemm_kernel<XT_PACK5, 8, KG>), grid, dim3(256 * KG), lds, s, a);
    else
        hipLaunchKernelGGL((gemm_kernel<XT_PACK4, 10, KG>), grid, dim3(256 * KG), lds, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splitk == 1) return e;
    const dim3 rgrid((a.ldp + 255) / 256, a.M);
    hipLaunchKernelGGL(gemm_reduce_kernel, rgrid, dim3(256), 0, s, a, splitk);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prefill GEMM on v_mfma_i32_32x32x32_i8 (Pack4 / XorSparse tiles, M > 16)
// ---------------------------------------------------------------------------
//
// The 32x32x32 i8 MFMA runs at twice the rate of 16x16x64 on gfx950 (about
// 4.1 vs 2.6 POP/s measured on MI355X), so this kernel computes 32-token x
// 32-row blocks.  Workgroup (x, y, z): 32 tokens (y) x 128 output rows (x)
// over chunk slice z.  Its eight MFMA waves are 4 row blocks (n) x 2 column
// halves (L) of every 256-column chunk.
//
// Operands.  B (weights) lane 32h + r holds output row r of the wave's 32
// rows: tile G = 2n + r/16 of the block, tile lane 16(2L + h) + r%16, whose
// dword s holds columns 64s + 32L + 16h .. +15.  One 16-byte tile slot per
// lane and chunk therefore gives four k-steps (s = 0..3) of the wave's half
// L.  A (activations) lane 32h + r' holds the same 16 columns of token r'.
// The MFMA pairs byte b of A with byte b of B in lanes of equal h, so only
// the pairing has to match, not any particular column order.
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// 16 bytes per lane from global memory straight into LDS; the wave's 64
// lanes fill 1 KiB at `wave_lds` in lane order.
__device__ __forceinline__ void load_lds16(const void* g, uint8_t* wave_lds) {
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)wave_lds, 16, 0, 0);
#endif
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
// `vm` must fold to a constant (it is called from fully unrolled loops).
#define XT_VMCNT_IMM(V) (((V) & 15) | (((V) >> 4) << 14) | (7 << 4) | (15 << 8))
__device__ __forceinline__ void wait_vmcnt(int vm) {
    switch (vm) {
#define XT_W4(B) case B: __builtin_amdgcn_s_waitcnt(XT_VMCNT_IMM(B)); break;    \
                 case B + 1: __builtin_amdgcn_s_waitcnt(XT_VMCNT_IMM(B + 1)); break; \
                 case B + 2: __builtin_amdgcn_s_waitcnt(XT_VMCNT_IMM(B + 2)); break; \
                 case B + 3: __builtin_amdgcn_s_waitcnt(XT_VMCNT_IMM(B + 3)); break;
        XT_W4(0) XT_W4(4) XT_W4(8) XT_W4(12) XT_W4(16) XT_W4(20) XT_W4(24) XT_W4(28)
        XT_W4(32) XT_W4(36) XT_W4(40) XT_W4(44) XT_W4(48) XT_W4(52) XT_W4(56) XT_W4(60)
#undef XT_W4
        default: __builtin_amdgcn_s_waitcnt(XT_VMCNT_IMM(0)); break;
    }
}

// 32-bit LDS address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// ds_read_b128 whose completion the caller waits for with lgkm_wait4.
__device__ __forceinline__ v4i ds_read16(uint32_t addr) {
    v4i v;
    __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
// Wait for all LDS reads; the operands tie the wait to the values read.
__device__ __forceinline__ void lgkm_wait4(v4i& a, v4i& b, v4i& c, v4i& d) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}


// ---------------------------------------------------------------------------
// Prefill GEMM, warp-specialised: loader waves stream chunks into LDS while
// eight MFMA waves consume them
// ---------------------------------------------------------------------------
//
// Measured on MI355X, one workgroup per CU pulls only ~33-50 bytes per clock
// from L2, so the 160 KiB a 32-token x 128-row tile needs over K = 2560 take
// ~2 us -- as long as its MFMA work -- and a wave that issues its own loads
// stalls at issue until the memory pipeline drains.  Here four loader waves
// issue every load as a direct-to-LDS copy (no registers), chunk by chunk,
// and signal each landed chunk with a workgroup barrier; the eight MFMA waves
// (operands as above, both read from LDS) compute chunk c while later chunks
// are still in flight.  Slot c of LDS holds chunk c: 8 KiB of activations
// (token row t at 256 t, 16-byte piece p in slot p ^ (t & 15), so that 16
// tokens reading one piece hit 16 distinct bank groups) then the 8 weight
// tiles of the block (1 KiB each, as in memory).  The loaders keep
// kG32sAhead chunks in flight before they start signalling.  The two halves
// L are added through LDS, the 32 x 128 code-domain tile is staged in LDS
// and written as whole 16-byte row pieces.  With gridDim.z > 1 the slice's
// code-domain sums go to plane z of `part` and gemm_reduce_kernel finishes.
constexpr int kG32sSlot = 8192;
// First LDS slot of the epilogue's exchange (2 slots) and output tile (2).
__host__ __device__ constexpr int g32s_xch_slot(int ncmax) { return ncmax >= 3 ? 0 : ncmax; }
#ifndef XT_G32S_AHEAD
#define XT_G32S_AHEAD 4
#endif
constexpr int kG32sAhead = XT_G32S_AHEAD;

template <int NCMAX>
__global__ __launch_bounds__(768) void gemm32s_kernel(const MMArgs a) {
    constexpr int CH = 256;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    const ProjBounds pb = proj_bounds();
    const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    const int M = a.M;
    const int nch = a.nch;
    const int cps = a.cps;
    // (the bounds are consumed here, so their loads join the grid-size round
    // instead of being sunk to their first use after it)
    asm volatile("" ::"s"(pb.np), "s"(pb.t0), "s"(pb.t1), "s"(pb.t2), "s"(pb.t3), "s"(gx), "s"(gy), "s"(gz));
    __builtin_amdgcn_sched_barrier(0);  // one round of argument loads
    const int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int t = xcd_remap(lin, gx * gy * gz);
    const int by = t % gy;
    const int bx = (t / gy) % gx;
    const int bz = t / (gx * gy);
    const ProjView pv = select_proj(pb, bx);
    const int N = pv.N;
    const int NG = (N + 15) >> 4;
    const int mbase = by * 32;
    const int cbeg = bz * cps;
    const int nc = min(nch - cbeg, cps);  // chunks of this slice, 1..NCMAX

    // The gy token blocks that share the weights start at different quarters
    // of the slice (different HBM lines in flight; integer sums do not depend
    // on the order).  Chunk c of the loop is slice chunk chunk_at(c); chunks
    // past the slice re-read its last chunk and count as code 0.
    const int rot = ((by & 3) * nc) >> 2;
    auto chunk_at = [&](int c) {
        const int cr = c + rot;
        return c < nc ? (cr >= nc ? cr - nc : cr) : nc - 1;
    };

    if (wave >= 8) {
        // Loader wave lw copies activation rows 8 lw .. 8 lw + 7 of every
        // chunk (two 1 KiB direct-to-LDS copies), so each chunk's vmcnt is a
        // compile-time number, and signals landed chunks with barriers.
        const int lw = wave - 8;
        const int8_t* as[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int tk = 4 * (2 * lw + jj) + (lane >> 4);
            const int trow = min(mbase + tk, M - 1);
            as[jj] = a.q + (size_t)trow * a.ldq + (size_t)cbeg * CH + ((lane & 15) ^ (tk & 15)) * 16;
        }
        constexpr int D = kG32sAhead < NCMAX ? kG32sAhead : NCMAX;
#pragma unroll
        for (int c = 0; c < NCMAX; ++c) {
            const int cc = chunk_at(c);
            uint8_t* slot = lds + c * kG32sSlot;
            load_lds16(as[0] + cc * CH, slot + (2 * lw) * 1024);
            load_lds16(as[1] + cc * CH, slot + (2 * lw + 1) * 1024);
            if (c >= D - 1) {  // chunk c - D + 1 has landed
                wait_vmcnt(2 * (D - 1));
                __builtin_amdgcn_s_barrier();
            }
        }
#pragma unroll
        for (int c = NCMAX - D + 1; c < NCMAX; ++c) {
            wait_vmcnt(2 * (NCMAX - 1 - c));
            __builtin_amdgcn_s_barrier();
        }
        __builtin_amdgcn_s_barrier();  // the MFMA waves' exchange
        __builtin_amdgcn_s_barrier();  // and output staging barriers
        return;
    }

    const int n = wave & 3;
    const int L = wave >> 2;
    const int h = lane >> 5;
    const int r = lane & 31;
    const bool split = gz > 1;

    // Output phase operands, loaded now: thread t writes tokens t/32 and
    // t/32 + 16 of the tile, columns 4 (t % 32) .. +3.
    const int srow = threadIdx.x >> 5;
    const int sc4 = (threadIdx.x & 31) * 4;
    const int ob = (bx - pv.tile0) * 128;
    float sinv[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) sinv[u] = a.inv[min(mbase + srow + 16 * u, M - 1)];
    float sws[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) sws[e] = pv.ws[min(ob + sc4 + e, N - 1)];

    // This wave's weights: its 16-byte tile slot of every chunk, loaded into
    // registers kG32sAhead chunks ahead of use.
    const int G = min((bx - pv.tile0) * 8 + 2 * n + (r >> 4), NG - 1);
    const uint8_t* wsrc = pv.tiles + ((size_t)(G * nch + cbeg) * 64 + 16 * (2 * L + h) + (r & 15)) * 16;
    constexpr int DW = kG32sAhead < NCMAX ? kG32sAhead : NCMAX;
    v4i wv[NCMAX];
#pragma unroll
    for (int c = 0; c < DW; ++c)
        wv[c] = *reinterpret_cast<const v4i*>(wsrc + (size_t)chunk_at(c) * kTileBytes);

    // Software-pipelined by one chunk: after the barrier that says chunk
    // c + 1 has landed, the wave reads its A fragments while chunk c's four
    // MFMAs (one accumulator per k-step, so none waits for another) run.
    const uint32_t abase = lds_addr(lds) + r * CH;
    auto read_a = [&](int c, v4i* av) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int p = 4 * s + 2 * L + h;
            av[s] = ds_read16(abase + c * kG32sSlot + ((p ^ (r & 15)) << 4));
        }
        lgkm_wait4(av[0], av[1], av[2], av[3]);
    };
    v16i acc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[s][k] = 0;
    v4i acur[4];
    __syncthreads();  // chunk 0 has landed
    read_a(0, acur);
#pragma unroll
    for (int c = 0; c < NCMAX; ++c) {
        if (c + DW < NCMAX)
            wv[c + DW] = *reinterpret_cast<const v4i*>(wsrc + (size_t)chunk_at(c + DW) * kTileBytes);
        // chunks past the slice: code 1 everywhere, i.e. weight 0
        const v4i bv = (c < nc) ? wv[c] : v4i{0x55555555, 0x55555555, 0x55555555, 0x55555555};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v4i b = decode4(bv[s]);
#pragma unroll
            for (int d = 0; d < 4; ++d) b[d] = signed_codes(b[d]);
            acc[s] = mfma32(acur[s], b, acc[s]);
        }
        if (c + 1 < NCMAX) {
            __syncthreads();  // chunk c + 1 has landed
            read_a(c + 1, acur);
        }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[0][k] += acc[1][k] + acc[2][k] + acc[3][k];

    // Add the halves L through LDS, in slots 0-1 when every wave is past
    // their reads (their chunks completed before the last chunk's barrier),
    // else after the chunk slots.  Entry [L][n][k][lane] carries registers
    // 8(1 - L) + k for the other wave of the pair.
    int32_t* xch = reinterpret_cast<int32_t*>(lds + g32s_xch_slot(NCMAX) * kG32sSlot);
    int keep[8];
    if (L == 0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            xch[((0 * 4 + n) * 8 + k) * 64 + lane] = acc[0][8 + k];
            keep[k] = acc[0][k];
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            xch[((1 * 4 + n) * 8 + k) * 64 + lane] = acc[0][k];
            keep[k] = acc[0][8 + k];
        }
    }
    __syncthreads();
    // Code-domain sums of the 32 x 128 tile -> LDS (slot 1), then whole rows.
    int32_t* dtile = reinterpret_cast<int32_t*>(xch + 4096);  // [32][128], two slots on
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int il = 8 * (2 * L + (k >> 2)) + 4 * h + (k & 3);
        dtile[il * 128 + 32 * n + r] = keep[k] + xch[(((1 - L) * 4 + n) * 8 + k) * 64 + lane];
    }
    __syncthreads();
    const bool vec = (N & 3) == 0;
    int32_t* plane = a.part + (size_t)bz * a.M * a.ldp;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int il = srow + 16 * u;
        const int i = mbase + il;
        const int o = ob + sc4;
        if (i >= M || o >= N) continue;
        const v4i d4 = *reinterpret_cast<const v4i*>(dtile + il * 128 + sc4);
        if (split) {
            // planes have a padded stride (a multiple of 16 columns)
            *reinterpret_cast<v4i*>(plane + (size_t)i * a.ldp + pv.col0 + o) = d4;
            continue;
        }
        float yv[4];
        v4i dv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dv[e] = d4[e];
            // layers.rs:294 — (dot as f32 * inv_scale) * w_scale.
            yv[e] = __fmul_rn(__fmul_rn((float)dv[e], sinv[u]), sws[e]);
        }
        if (vec) {
            *reinterpret_cast<float4*>(pv.y + (size_t)i * N + o) = make_float4(yv[0], yv[1], yv[2], yv[3]);
            if (pv.acc) *reinterpret_cast<v4i*>(pv.acc + (size_t)i * N + o) = dv;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (o + e < N) {
                    pv.y[(size_t)i * N + o + e] = yv[e];
                    if (pv.acc) pv.acc[(size_t)i * N + o + e] = dv[e];
                }
            }
        }
    }
}

int gemm32s_ncmax() { return 18; }

hipError_t launch_gemm32s(const MMArgs& a, int ntiles, int splitk, hipStream_t s) {
    const dim3 grid(ntiles, (a.M + 31) / 32, splitk);
    const int ncm = a.cps;
    if (ncm < 1 || ncm > gemm32s_ncmax()) return hipErrorInvalidValue;
    const int xs = g32s_xch_slot(ncm) + 4;
    const size_t lds = (size_t)(ncm < xs ? xs : ncm) * kG32sSlot;
    switch (ncm) {
#define XT_G32S(V) \
    case V: hipLaunchKernelGGL((gemm32s_kernel<V>), grid, dim3(768), lds, s, a); break;
        XT_G32S(1) XT_G32S(2) XT_G32S(3) XT_G32S(4) XT_G32S(5) XT_G32S(6) XT_G32S(7)
        XT_G32S(8) XT_G32S(9) XT_G32S(10) XT_G32S(11) XT_G32S(12) XT_G32S(13) XT_G32S(14)
        XT_G32S(15) XT_G32S(16) XT_G32S(17) XT_G32S(18)
#undef XT_G32S
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splitk == 1) return e;
    const dim3 rgrid((a.ldp + 255) / 256, a.M);
    hipLaunchKernelGGL(gemm_reduce_kernel, rgrid, dim3(256), 0, s, a, splitk);
    return hipGetLastError();
}

// Fewest K slices whose chunks fit the LDS stage of the prefill GEMM.
int gemm32_ncmax() { return gemm32s_ncmax(); }
int g32_splitk(int nch) { return nch <= 0 ? 1 : (nch + gemm32_ncmax() - 1) / gemm32_ncmax(); }
hipError_t launch_gemm32(const MMArgs& a, int ntiles, int splitk, hipStream_t s) {
    return launch_gemm32s(a, ntiles, splitk, s);
}

// Compiled tile shapes, selectable by MMConfig.
#define XT_MM_SHAPES(X)  \
    X(1, 1, 4, 4)        \
    X(1, 1, 2, 8)        \
    X(1, 1, 2, 4)        \
    X(1, 1, 8, 2)        \
    X(1, 1, 4, 2)        \
    X(1, 2, 4, 4)        \
    X(1, 4, 4, 2)        \
    X(2, 4, 4, 2)        \
    X(2, 8, 4, 2)        \
    X(4, 4, 4, 1)        \
    X(4, 2, 4, 1)        \
    X(1, 5, 4, 2)        \
    X(1, 5, 8, 2)        \
    X(1, 4, 8, 2)        \
    X(2, 5, 8, 2)        \
    X(1, 5, 16, 1)       \
    X(1, 5, 8, 1)        \
    X(1, 5, 16, 2)       \
    X(1, 10, 8, 2)       \
    X(2, 8, 8, 2)        \
    X(1, 8, 8, 2)        \
    X(4, 4, 8, 1)

namespace {
bool shape_known(const MMConfig& c, bool own) {
#define XT_KNOWN(MB_, NB_, W_, PF_) \
    if (c.mb == MB_ && c.nb == NB_ && c.waves == W_ && c.pf == PF_) return !own || MB_ == 1;
    XT_MM_SHAPES(XT_KNOWN)
#undef XT_KNOWN
    return false;
}

// XTERN_CONFIG="mb,nb,waves,pf,splitk" forces one tile shape (for tuning).
bool env_config(MMConfig* c) {
    const char* e = getenv("XTERN_CONFIG");
    MMConfig f;
    if (e && sscanf(e, "g32,%d", &f.splitk) == 1 && f.splitk >= 1) {
        f = MMConfig{2, 8, 8, 1, f.splitk};
        f.kind = 3;
        *c = f;
        return true;
    }
    if (e && sscanf(e, "gemv,%d", &f.waves) == 1) {
        f = MMConfig{1, 1, f.waves, 1, 1};
        f.kind = 2;
        *c = f;
        return true;
    }
    if (e && sscanf(e, "%d,%d,%d,%d,%d", &f.mb, &f.nb, &f.waves, &f.pf, &f.splitk) == 5 &&
        f.splitk >= 1) {
        *c = f;
        return true;
    }
    return false;
}
}  // namespace

// Default tile shapes (chosen by measurement on MI355X):
//   M <= 16  the decode GEMV (activations in LDS, 16 waves) when the staged
//            activations fit, else 16 rows per workgroup, 8 waves x 2 chunks;
//   M > 16   the prefill GEMM (32 tokens x 128 rows) when K fits one LDS
//            slice, else 16 tokens x 64 rows with 4 waves splitting K.
// Split-K across workgroups (gridDim.z > 1) is only taken when forced: its
// device-scope release/acquire costs more than it saves at these sizes.
// Waves per workgroup of the Int8 / Int4 GEMV for row blocks of mb tokens.
int int_gemv_waves(int fmt, int mb, int nch) {
    MMConfig c;
    if (env_config(&c) && c.kind == 2 && gemv_fits(fmt, mb, nch, c.waves, gemv_ncw(c.waves)))
        return c.waves;
    // Measured on the 128256 x 2560 LM head: Int4 streams fastest with 8
    // waves (46.5 vs 58 us at M = 1), Int8 with 16.
    return (fmt == XT_INT4 && gemv_fits(fmt, mb, nch, 8, gemv_ncw(8))) ? 8 : 16;
}

MMConfig choose_config(int fmt, int M, int ntiles_nb1, int nch, bool have_rowsum) {
    MMConfig c;
    if (env_config(&c)) {
        if (c.kind == 2 && M <= 16 && gemv_fits(fmt, M, nch, c.waves, gemv_ncw(c.waves))) {
            c.nb = gemv_row_groups(fmt, nch, ntiles_nb1);
            return c;
        }
        if (c.kind == 3 && M > 16 && fmt == XT_PACK4 &&
            (nch + c.splitk - 1) / c.splitk <= gemm32_ncmax())
            return c;
        if (c.kind == 0 && shape_known(c, !have_rowsum)) {
            if (c.splitk > nch) c.splitk = nch;
            return c;
        }
    }
    if (M <= 16) {
        // Measured (MI355X, rotating weights, M = 1..16): the staging-free
        // GEMV wins or ties everywhere, also for many rows (K 2560 -> 8192,
        // M = 4: 3.9 vs 4.7 us on the 32-row, 4-wave K-split kernel;
        // 4096 -> 14336, M = 16: 7.9 vs 8.7).
        if (nch <= 64 || gemv_fits(fmt, M, nch, 16, gemv_ncw(16))) {
            c = MMConfig{1, gemv_row_groups(fmt, nch, ntiles_nb1), 16, 1, 1};
            c.kind = 2;
            return c;
        }
        return MMConfig{1, 1, 8, 2, 1};
    }
    // Prefill, Pack4 tiles: the warp-specialised 32x32x32 MFMA GEMM when K
    // fits its LDS stage (C1 up: 10.9 -> 7.8 us).  Longer K stays on the
    // K-split kernel below: splitting it over workgroups plus a reduction
    // launch measured slower (C1 down: 12.6 vs 8.5 us).
    // A grid of fewer than ~80 of its 32 x 128 tiles leaves most CUs idle
    // while each tile takes the same ~7 us; 16 tokens x 32 rows with K over 4
    // waves spreads such shapes over 4-8x the workgroups (M = 32: K 2560 ->
    // N 2560 / 3840 7.2 -> 5.0 / 5.2 us; M = 24, N = 6912: 7.4 -> 6.2 us;
    // 108 tiles, N = 13824 at M = 32: 7.8 vs 8.3 us, the GEMM stays).
    const long g32_tiles = (long)((ntiles_nb1 * 16 + 127) / 128) * ((M + 31) / 32);
    if (fmt == XT_PACK4 && ntiles_nb1 > 0 && g32_tiles < 80) return MMConfig{1, 2, 4, 4, 1};
    if (fmt == XT_PACK4 && nch <= gemm32_ncmax()) {
        c = MMConfig{2, 8, 8, 1, 1};
        c.kind = 3;
        return c;
    }
    // Prefill: the LDS GEMM when its activation slice covers K in one
    // workgroup; otherwise 16 tokens x 64 rows per workgroup with K split
    // over 4 waves (measured faster than split-K planes plus a reduction).
    if (have_rowsum && nch <= gemm_ncmax(fmt)) {
        c = MMConfig{2, 8, 4, 1, 1};
        c.kind = 1;
        (void)ntiles_nb1;
        return c;
    }
    // Long K (activation slice too big for the GEMM's LDS): 16 tokens per
    // workgroup, K over 8 waves, and the row-block width that fills the
    // chip in the fewest rounds of workgroups -- e.g. C1 down (M 128, 160
    // row groups): 80 rows -> 256 workgroups in one round, 8.6 us, against
    // 64 rows -> 320 workgroups in two rounds, 12.5 us.
    const int tb = (M + 15) / 16;
    int best_nb = 4;
    long best_cost = -1;
    for (int nb : {4, 5, 8}) {
        const long wgs = (long)((ntiles_nb1 + nb - 1) / nb) * tb;
        const long cost = ((wgs + 255) / 256) * nb;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best_nb = nb;
        }
    }
    return MMConfig{1, best_nb, 8, 2, 1};
}

hipError_t launch_mm(int fmt, const MMConfig& cfg, const MMArgs& a, int ntiles_total,
                     hipStream_t s) {
    const bool own = (a.rowsum == nullptr);
    const int sk = cfg.splitk;
#define XT_LAUNCH(MB_, NB_, W_, PF_)                                                          \
    if (cfg.mb == MB_ && cfg.nb == NB_ && cfg.waves == W_ && cfg.pf == PF_) {                \
        if constexpr (MB_ == 1) {                                                              \
            if (own)                                                                           \
                return fmt == XT_PACK5                                                         \
                           ? launch_t<XT_PACK5, MB_, NB_, W_, PF_, true>(a, ntiles_total, sk, s) \
                           : launch_t<XT_PACK4, MB_, NB_, W_, PF_, true>(a, ntiles_total, sk, s); \
        }                                                                                      \
        if (own) return hipErrorInvalidValue;                                                  \
        return fmt == XT_PACK5 ? launch_t<XT_PACK5, MB_, NB_, W_, PF_, false>(a, ntiles_total, sk, s) \
                               : launch_t<XT_PACK4, MB_, NB_, W_, PF_, false>(a, ntiles_total, sk, s); \
    }
    XT_MM_SHAPES(XT_LAUNCH)
#undef XT_LAUNCH
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// HF prepacked weights -> device tiles (src/loader/mod.rs:301-394)
// ---------------------------------------------------------------------------

// The checkpoint stores U8 bytes [R][K], R = N/f, whose digit j (Pack4: bits
// 2j..2j+1, Pack5: base-3 digit j) of byte [p][i] is the weight of output row
// j*R + p at input column i.  One thread builds the 16 bytes of one lane of
// one tile (geometry in xtern_internal.h), reading the digits it needs
// straight from the striped bytes, so the loader's host-side unpack /
// transpose / repack is not needed.  Pack4 code 11 reads as weight 0, as
// unpack_1_58bit_4pack does (quantization.rs:36-41); Pack5 digits are the
// repeated %3, /3 of unpack_1_58bit_5pack (:72-91).
template <int FMT>
__global__ void __launch_bounds__(256)
hf_tiles_kernel(const uint8_t* __restrict__ stored, int64_t K, int64_t N, int64_t R, int64_t nch,
                int64_t nlanes, uint8_t* __restrict__ tiles) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= nlanes) return;
    const int lane = (int)(t & 63);
    const int64_t tile = t >> 6;
    const int64_t G = tile / nch, c = tile % nch;
    const int g = lane >> 4, jr = lane & 15;
    const int64_t o = G * 16 + jr;
    const bool row_ok = o < N;
    const int64_t js = row_ok ? o / R : 0, p = row_ok ? o % R : 0;
    const uint8_t* src = stored + p * K;
    uint32_t out[4];
    if constexpr (FMT == XT_PACK5) {
        const unsigned div = js == 0 ? 1u : js == 1 ? 3u : js == 2 ? 9u : js == 3 ? 27u : 81u;
        uint8_t bytes[16];
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            unsigned v = 0;
#pragma unroll
            for (int st = 0; st < 5; ++st) {
                const int64_t k = c * 320 + st * 64 + g * 16 + b;
                const unsigned code = (row_ok && k < K) ? (src[k] / div) % 3u : 1u;
                v = v * 3u + code;
            }
            bytes[b] = (uint8_t)((v * 256u + 242u) / 243u);
        }
#pragma unroll
        for (int w = 0; w < 4; ++w)
            out[w] = (uint32_t)bytes[4 * w] | ((uint32_t)bytes[4 * w + 1] << 8) |
                     ((uint32_t)bytes[4 * w + 2] << 16) | ((uint32_t)bytes[4 * w + 3] << 24);
    } else {
        const int sh = (int)(2 * js);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            uint32_t d = 0;
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int64_t k = c * 256 + st * 64 + g * 16 + b;
                unsigned code = 1u;
                if (row_ok && k < K) {
                    const unsigned f = (src[k] >> sh) & 3u;
                    code = f == 0u ? 0u : (f == 2u ? 2u : 1u);
                }
                d |= code << (8 * (b & 3) + 2 * (b >> 2));
            }
            out[st] = d;
        }
    }
    *reinterpret_cast<uint4*>(tiles + t * 16) = make_uint4(out[0], out[1], out[2], out[3]);
}

hipError_t launch_hf_tiles(int fmt, const uint8_t* stored, int64_t K, int64_t N, uint8_t* tiles,
                           hipStream_t s) {
    const int64_t f = fmt == XT_PACK5 ? 5 : 4;
    const int64_t nch = (K + chunk_cols(fmt) - 1) / chunk_cols(fmt);
    const int64_t nlanes = (N + 15) / 16 * nch * 64;
    const int64_t blocks = (nlanes + 255) / 256;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (fmt == XT_PACK5)
        hipLaunchKernelGGL(hf_tiles_kernel<XT_PACK5>, dim3((unsigned)blocks), dim3(256), 0, s,
                           stored, K, N, N / f, nch, nlanes, tiles);
    else
        hipLaunchKernelGGL(hf_tiles_kernel<XT_PACK4>, dim3((unsigned)blocks), dim3(256), 0, s,
                           stored, K, N, N / f, nch, nlanes, tiles);
    return hipGetLastError();
}

}  // namespace xt


namespace xt {

// ---------------------------------------------------------------------------
// MLP middle: activation, optional RMSNorm, requantisation
// ---------------------------------------------------------------------------

// expf of the C library the reference links (glibc 2.28+, from ARM's
// optimized-routines): x * 32/ln2 rounded to an integer k, 2^(k/32) from a
// 32-entry table with k/32's integer part added to the exponent bits, and a
// cubic in the remainder, all in double, rounded once to float.  The two
// products with InvLn2N are fused multiply-adds, as the FMA build of the
// library compiles them.  Equal to the host expf on every one of the 2^32
// float inputs (checked exhaustively on the build host).
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

__device__ __forceinline__ float libc_expf(float x) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t top = (ux >> 20) & 0x7ffu;
    if (top >= 0x42bu) {  // |x| >= 88, inf, NaN
        if (ux == 0xff800000u) return 0.0f;
        if (top >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double inv = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double xd = (double)x;
    double kd = __fma_rn(inv, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = __dsub_rn(kd, shift);
    const double r = __fma_rn(inv, xd, -kd);
    const uint64_t t = kExp2Tab[ki & 31] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __fma_rn(C0, r, C1);
    const double r2 = __dmul_rn(r, r);
    double y = __fma_rn(C2, r, 1.0);
    y = __fma_rn(z, r2, y);
    return (float)__dmul_rn(y, s);
}

// quantization.rs:213 / :280: g * (1 / (1 + exp(-g))) * u.
__device__ __forceinline__ float silu_scalar(float g, float u) {
    const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, libc_expf(-g)));
    return __fmul_rn(__fmul_rn(g, sig), u);
}
// tensor.rs:186-188: (x / (1 + exp(-x))) * u.
__device__ __forceinline__ float silu_div(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, libc_expf(-g))), u);
}
// quantization.rs:215-216, :268-270; tensor.rs:223-224: max(g, 0)^2 * u.
__device__ __forceinline__ float relu2_mul(float g, float u) {
    const float r = (g > 0.0f) ? g : 0.0f;
    return __fmul_rn(__fmul_rn(r, r), u);
}
// One lane of silu_inplace_avx512's vector body (quantization.rs:243-272).
__device__ __forceinline__ float silu_poly(float g, float u) {
    const float inv_ln2 = 1.44269504088896341f, ln2 = 0.693147180559945309f;
    const float hi = 88.3762626647949f, lo = -88.3762626647949f;
    float x = __fsub_rn(0.0f, g);
    x = (x < hi) ? x : hi;  // MINPS: second operand unless x < hi (NaN -> hi)
    x = (x > lo) ? x : lo;  // MAXPS
    const float fx = __fmul_rn(x, inv_ln2);
    const float n_f = __builtin_rintf(fx);
    const float t = __fsub_rn(x, __fmul_rn(n_f, ln2));
    float e = __fmaf_rn(1.0f / 24.0f, t, 1.0f / 6.0f);
    e = __fmaf_rn(e, t, 0.5f);
    e = __fmaf_rn(e, t, 1.0f);
    e = __fmaf_rn(e, t, 1.0f);
    const uint32_t bits = ((uint32_t)(int)n_f + 127u) << 23;
    const float exp_x = __fmul_rn(e, __uint_as_float(bits));
    const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, exp_x));
    return __fmul_rn(__fmul_rn(g, sig), u);
}

__device__ __forceinline__ float apply_act(int act, float g, float u, bool main_lane) {
    switch (act) {
        case XT_ACT_SILU_INPLACE_AVX512:
            return main_lane ? silu_poly(g, u) : silu_scalar(g, u);
        case XT_ACT_SILU_INPLACE_SCALAR:
            return silu_scalar(g, u);
        case XT_ACT_SILU_MUL:
            return silu_div(g, u);
        case kActIdentity:
            return g;
        default:
            return relu2_mul(g, u);
    }
}

constexpr int kMidThreads = 1024;
constexpr int kMidWaves = kMidThreads / 64;
constexpr int kMidCmax = 16;                         // row length <= 16 * 1024
constexpr int kMidRecMax = 1024;                     // piece records in LDS
constexpr uint32_t kGrid = 1u << 24;                 // grid points per binade

// Wave-wide data movement with DPP (gfx9 encodings): row_shr:n = 0x110 + n
// shifts within rows of 16 lanes, row_bcast:15 / row_bcast:31 = 0x142 / 0x143
// broadcast lane 15 / 31 into the following rows, wave_shr:1 = 0x138 and
// wave_shl:1 = 0x130 shift across the whole wave.  Lanes without a source
// (or outside ROW_MASK) receive 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    const uint32_t lo = dpp32<CTRL, ROW_MASK>((uint32_t)v);
    const uint32_t hi = dpp32<CTRL, ROW_MASK>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Inclusive wave scans (Hillis-Steele in rows of 16, then row broadcasts).
__device__ __forceinline__ uint64_t wave_scan_add(uint64_t v) {
    v += dpp64<0x111, 0xf>(v);
    v += dpp64<0x112, 0xf>(v);
    v += dpp64<0x114, 0xf>(v);
    v += dpp64<0x118, 0xf>(v);
    v += dpp64<0x142, 0xa>(v);
    v += dpp64<0x143, 0xc>(v);
    return v;
}
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v) {
    v += dpp32<0x111, 0xf>(v);
    v += dpp32<0x112, 0xf>(v);
    v += dpp32<0x114, 0xf>(v);
    v += dpp32<0x118, 0xf>(v);
    v += dpp32<0x142, 0xa>(v);
    v += dpp32<0x143, 0xc>(v);
    return v;
}
// Wave maximum of non-negative floats (0 is the identity), in every lane.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = fmaxf(v, __uint_as_float(dpp32<0x111, 0xf>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<0x112, 0xf>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<0x114, 0xf>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<0x118, 0xf>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<0x142, 0xa>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<0x143, 0xc>(__float_as_uint(v))));
    return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}
__device__ __forceinline__ int wave_sum_int(int v) {
    const uint32_t s = wave_scan_add((uint32_t)v);
    return (int)__builtin_amdgcn_readlane(s, 63);
}
template <typename T>
__device__ __forceinline__ T lane_read(T v, int k) {
    if constexpr (sizeof(T) == 8) {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, k);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), k);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    } else {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, v), k));
    }
}

// Integer increment of adding t (finite, >= 0) to a running sum on the grid
// u = 2^(b-23): q = floor(t / u) (capped at 2^24), r = 0 below half, 1 at an
// exact half, 2 above.
__device__ __forceinline__ void grid_split(float t, int b, uint32_t* q, int* r) {
    const uint32_t bits = __float_as_uint(t);
    const uint32_t ef = (bits >> 23) & 0xffu;
    const uint32_t m = ef ? ((bits & 0x7fffffu) | 0x800000u) : (bits & 0x7fffffu);
    const int et = ef ? (int)ef - 150 : -149;
    const int shift = (b - 23) - et;
    // shift <= 0: t is a multiple of u (q = m << -shift, capped at 2^24)
    const int ls = min(-shift, 24);
    const uint32_t qup = min(m << max(ls, 0), kGrid);
    // shift > 0: m < 2^24, so shifts of 25 or more leave q = 0, remainder m
    const int sc = min(max(shift, 1), 25);
    const uint32_t qdn = m >> sc;
    const uint32_t rem = m & ((1u << sc) - 1u), half = 1u << (sc - 1);
    const int rdn = rem < half ? 0 : (rem == half ? 1 : 2);
    *q = shift <= 0 ? (m ? qup : 0u) : qdn;
    *r = shift <= 0 ? 0 : rdn;
}

struct SeqSumLds {
    float wtot[kMidWaves];
    uint64_t wgp[kMidWaves];
    int wcnt[kMidWaves];
    float res;
};

__device__ __forceinline__ float wave_scan_addf(float v) {
    v = __fadd_rn(v, __uint_as_float(dpp32<0x111, 0xf>(__float_as_uint(v))));
    v = __fadd_rn(v, __uint_as_float(dpp32<0x112, 0xf>(__float_as_uint(v))));
    v = __fadd_rn(v, __uint_as_float(dpp32<0x114, 0xf>(__float_as_uint(v))));
    v = __fadd_rn(v, __uint_as_float(dpp32<0x118, 0xf>(__float_as_uint(v))));
    v = __fadd_rn(v, __uint_as_float(dpp32<0x142, 0xa>(__float_as_uint(v))));
    v = __fadd_rn(v, __uint_as_float(dpp32<0x143, 0xc>(__float_as_uint(v))));
    return v;
}
// Binade of a float >= 0 (subnormals and 0 in -126, infinity 128).
__device__ __forceinline__ int binade_f(float a) {
    const int e = (int)(__float_as_uint(a) >> 23);
    return e == 0 ? -126 : e - 127;
}

// Significand of s >= 0 on the grid of its binade (implicit bit included;
// for binade -126 the subnormal or smallest-normal encoding), and the float
// of significand T < 2^24 in binade b.
__device__ __forceinline__ int sig_binade(float s, uint32_t* S) {
    const uint32_t sbits = __float_as_uint(s);
    const int se = (int)(sbits >> 23);
    *S = (sbits & 0x7fffffu) | (se ? 0x800000u : 0u);
    return se == 0 ? -126 : se - 127;
}
__device__ __forceinline__ float from_grid(uint64_t T, int b) {
    return __uint_as_float(T >= 0x800000u ? ((uint32_t)(b + 127) << 23) | ((uint32_t)T & 0x7fffffu)
                                          : (uint32_t)T);  // b = -126, subnormal
}

// s + lt[j] + ... + lt[end - 1], each partial sum rounded to f32, by one
// whole wave (s is the same in every lane): 256 elements at a time (4
// consecutive ones per lane) are split on the grid of the running sum's
// binade and prefix-summed; the leading ones that are no tie and keep the sum
// inside the binade are added at once (exact integer addition on the grid),
// the next one with a real f32 add.
__device__ float seq_advance(float s, const float* lt, int j, int end) {
    const int lane = threadIdx.x & 63;
    s = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s)));
    while (j < end) {
        uint32_t S;
        const int bs = sig_binade(s, &S);
        if (bs > 127) return s;  // infinity plus finite non-negative terms
        // lane l: elements j + 4 l .. j + 4 l + 3; local inclusive prefixes
        uint32_t pre[4];
        int kbad = 4;  // first element of the lane that is a tie or past `end`
        uint32_t acc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = j + 4 * lane + k;
            uint32_t q = 0;
            int r = 1;  // past the end: treated as a stop
            if (e < end) grid_split(lt[e], bs, &q, &r);
            if (r == 1 && kbad == 4) kbad = k;
            acc += min(q + (r == 2 ? 1u : 0u), kGrid);
            pre[k] = acc;  // <= 4 * 2^24 per lane
        }
        const uint32_t lincl = wave_scan_add(acc);  // <= 256 * 2^24 < 2^32
        const uint32_t lexcl = lincl - acc;
        // first element (in order) that is a stop or leaves the binade
        int kfirst = kbad;
#pragma unroll
        for (int k = 3; k >= 0; --k)
            if ((uint64_t)S + lexcl + pre[k] >= kGrid) kfirst = min(kfirst, k);
        const uint64_t bad = __ballot(kfirst < 4);
        int m;  // elements added on the grid
        uint32_t pm = 0;
        if (bad) {
            const int L = (int)__builtin_ctzll(bad);
            const int kL = lane_read(kfirst, L);
            m = 4 * L + kL;
            if (m > 0) {
                // prefix through element m - 1
                uint32_t mine = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k == kL - 1) mine = lexcl + pre[k];
                pm = kL > 0 ? lane_read(mine, L) : lane_read(lincl, L - 1);
            }
        } else {
            m = 256;
            pm = lane_read(lincl, 63);
        }
        if (m > 0) {
            s = from_grid((uint64_t)S + pm, bs);
            j += m;
        }
        if (m < 256 && j < end) {
            s = __fadd_rn(s, lt[j]);
            ++j;
        }
        s = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s)));
    }
    return s;
}

// Sequential float sum t[0] + t[1] + ... + t[n-1] (each partial sum rounded
// to f32, in index order) -- the order of rms_norm's sum of squares --
// computed by the whole workgroup.  Within one binade [2^b, 2^(b+1)) of the
// running sum, every f32 add is an integer add on the grid u = 2^(b-23):
// fl(s + t) = s + u * round(t / u), except when t / u is an exact half (a
// tie, whose rounding depends on the parity of s) or when the sum leaves the
// binade.  So:
//  1. a float prefix sum predicts the binade of the running sum before each
//     element;
//  2. elements that are ties, or after which the predicted binade changes,
//     end a "piece"; every other element contributes its integer increment,
//     and the increments are prefix-summed;
//  3. one wave walks the pieces in order with the running sum's bits on the
//     scalar unit: if they lie in the piece's precomputed range (the sum is
//     in the predicted binade and stays below its top after the piece), the
//     piece is one integer add on the bits; otherwise seq_advance adds the
//     piece; the piece's end element is always a real f32 add.
// The result never depends on the prediction being right, only the speed
// does.  `lt` holds t[0..n) (finite, >= 0) in LDS; thread j handles the
// contiguous elements [j*E, j*E + E), E = ceil(n / 1024) <= CM.
template <int CM>
__device__ __forceinline__ float exact_seq_sum(int n, const float* lt, SeqSumLds& sl, int* rec_idx,
                                               uint64_t* rec_gp, int* rec_b) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int E = (n + kMidThreads - 1) / kMidThreads;
    const int i0 = tid * E;
    const int cnt = max(0, min(E, n - i0));  // this thread's elements: [i0, i0 + cnt)
    float t[CM];
#pragma unroll
    for (int e = 0; e < CM; ++e) t[e] = e < cnt ? lt[i0 + e] : 0.0f;
    // 1. prefix sums: thread-local, then across lanes and waves
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < CM; ++e)
        if (e < cnt) acc = __fadd_rn(acc, t[e]);
    const float incl = wave_scan_addf(acc);
    const float excl = __uint_as_float(dpp32<0x138, 0xf>(__float_as_uint(incl)));  // wave_shr:1
    const float excl_next = __uint_as_float(dpp32<0x130, 0xf>(__float_as_uint(excl)));  // wave_shl:1
    if (lane == 63) sl.wtot[w] = incl;
    __syncthreads();
    float woff = 0.0f;
    for (int j = 0; j < w; ++j) woff = __fadd_rn(woff, sl.wtot[j]);
    const float woff_next = __fadd_rn(woff, sl.wtot[w]);
    // Prefix before this thread's first element, and before the next
    // thread's first element, computed exactly as that thread computes it.
    const float off = __fadd_rn(woff, excl);
    const float off_next = lane < 63 ? __fadd_rn(woff, excl_next) : __fadd_rn(woff_next, 0.0f);

    // 2. The binade before element i is that of off + (local prefix before
    // i) -- the next thread's `off` after the last element.  Piece ends and
    // integer increments, kept in registers.
    uint32_t inc[CM];
    int bb[CM];
    uint32_t endbits = 0;
    uint64_t dsum = 0;
    {
        float lp = 0.0f;
        int b = binade_f(off);
#pragma unroll
        for (int e = 0; e < CM; ++e) {
            inc[e] = 0;
            bb[e] = b;
            if (e < cnt) {
                lp = __fadd_rn(lp, t[e]);
                const int bn = (e + 1 < E) ? binade_f(__fadd_rn(off, lp)) : binade_f(off_next);
                uint32_t q;
                int r;
                grid_split(t[e], b, &q, &r);
                const bool end = r == 1 || bn != b || i0 + e == n - 1;
                inc[e] = end ? 0u : min(q + (r == 2 ? 1u : 0u), kGrid);
                endbits |= (end ? 1u : 0u) << e;
                dsum += inc[e];
                b = bn;
            }
        }
    }
    const uint32_t ends = __builtin_popcount(endbits);
    const uint64_t gincl = wave_scan_add(dsum);
    const uint32_t cincl = wave_scan_add(ends);
    if (lane == 63) {
        sl.wgp[w] = gincl;
        sl.wcnt[w] = (int)cincl;
    }
    __syncthreads();
    uint64_t gp = gincl - dsum;
    int rank = (int)(cincl - ends);
    int total_ends = 0;
    for (int j = 0; j < kMidWaves; ++j) {
        if (j < w) {
            gp += sl.wgp[j];
            rank += sl.wcnt[j];
        }
        total_ends += sl.wcnt[j];
    }
    const bool overflow = total_ends > kMidRecMax;
    if (!overflow && endbits) {
#pragma unroll
        for (int e = 0; e < CM; ++e) {
            if (e < cnt) {
                if ((endbits >> e) & 1u) {
                    rec_idx[rank] = i0 + e;
                    rec_gp[rank] = gp;  // own increment is 0
                    rec_b[rank] = bb[e];
                    ++rank;
                }
                gp += inc[e];
            }
        }
    }
    __syncthreads();

    // 3. walk the pieces (wave 0).  Records are loaded 64 at a time, one per
    // lane, with everything that does not depend on the running sum: the
    // range [lo, lim) of running-sum bits for which the piece's P increments
    // are one integer add on the bits (in binade b the bits are
    // ((b + 127) << 23) + significand - 2^23, or the significand itself for
    // b = -126, so "sum in binade b and sum + P below 2^(b+1)" is
    // lo <= bits < hi - P).  The sequential part reads them with readlane.
    if (w == 0) {
        // (uniform values read from LDS are made scalar, so that the walk
        // runs on the scalar unit instead of under exec masks)
        total_ends = __builtin_amdgcn_readfirstlane(total_ends);
        float s = 0.0f;
        if (overflow) {
            s = seq_advance(0.0f, lt, 0, n);
        } else {
            uint32_t sbits = 0;
            for (int k0 = 0; k0 < total_ends; k0 += 64) {
                const int k = k0 + lane;
                int idx = 0, start = 0;
                uint32_t lo = 0, lim = 0xffffffffu, P32 = 0;
                float tend = 0.0f;
                if (k < total_ends) {
                    idx = rec_idx[k];
                    const int rb = rec_b[k];
                    start = k > 0 ? rec_idx[k - 1] + 1 : 0;
                    const uint64_t P = rec_gp[k] - (k > 0 ? rec_gp[k - 1] : 0ull);
                    tend = lt[idx];
                    if (start < idx) {
                        const uint32_t hi = (uint32_t)(rb + 128) << 23;
                        lo = rb == -126 ? 0u : (uint32_t)(rb + 127) << 23;
                        if (rb > 127 || P >= (uint64_t)(hi - lo)) {
                            lo = 1u;  // empty range
                            lim = 0u;
                        } else {
                            lim = hi - (uint32_t)P;
                            P32 = (uint32_t)P;
                        }
                    }
                }
                const int kn = min(64, total_ends - k0);
                // The dependency chain per piece is two compares, a select
                // and one f32 add; the fallback is a branch not taken.
                for (int kk = 0; kk < kn; ++kk) {
                    const uint32_t klo = lane_read(lo, kk), klim = lane_read(lim, kk);
                    const uint32_t kp = lane_read(P32, kk);
                    const float kt = lane_read(tend, kk);
                    const bool inr = sbits >= klo && sbits < klim;
                    sbits = inr ? sbits + kp : sbits;
                    if (__builtin_expect(!inr, 0)) {
                        sbits = __float_as_uint(seq_advance(__uint_as_float(sbits), lt,
                                                            lane_read(start, kk), lane_read(idx, kk)));
                    }
                    sbits = __float_as_uint(__fadd_rn(__uint_as_float(sbits), kt));
                }
            }
            s = __uint_as_float(sbits);
        }
        if (lane == 0) sl.res = s;
    }
    __syncthreads();
    return sl.res;
}

// One workgroup (16 waves) per row.  Element i = (wave*C + c)*64 + lane is
// held in registers from the load to the quantisation.
template <int ACT, int CM>
__global__ __launch_bounds__(kMidThreads) void mlp_mid_kernel(MidArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ SeqSumLds sl;
    __shared__ float sm_f[kMidWaves];
    __shared__ int sm_i[kMidWaves];
    const int m = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = a.n, C = a.C;
    const int nmain = (n / 16) * 16;
    const float* gr = a.gate + (size_t)m * a.ldg;
    const float* ur = a.up + (size_t)m * a.ldg;
    float v[CM], nwv[CM];
#pragma unroll
    for (int c = 0; c < CM; ++c) {
        const int i = (w * C + c) * 64 + lane;
        v[c] = (c < C && i < n) ? apply_act(ACT, gr[i], ACT == kActIdentity ? 0.0f : ur[i], i < nmain)
                                : 0.0f;
        nwv[c] = (a.norm_w && c < C && i < n) ? a.norm_w[i] : 0.0f;  // fetched early
    }
    if (a.norm_w) {
        float* lt = reinterpret_cast<float*>(lds);
        int* rec_idx = reinterpret_cast<int*>(lds + (size_t)C * kMidThreads * 4);
        int* rec_b = rec_idx + kMidRecMax;
        uint64_t* rec_gp = reinterpret_cast<uint64_t*>(rec_b + kMidRecMax);
        bool bad_nan = false, bad_inf = false;
#pragma unroll
        for (int c = 0; c < CM; ++c) {
            const int i = (w * C + c) * 64 + lane;
            const float t = __fmul_rn(v[c], v[c]);
            if (c < C && i < n) {
                lt[i] = t;
                bad_nan |= (t != t);
                bad_inf |= (bool)__builtin_isinf(t);
            }
        }
        const int wf = (__ballot(bad_nan) ? 1 : 0) | (__ballot(bad_inf) ? 2 : 0);
        if (lane == 0) sm_i[w] = wf;
        __syncthreads();
        int flags = 0;
#pragma unroll
        for (int j = 0; j < kMidWaves; ++j) flags |= sm_i[j];
        float sum;
        if (flags & 1) sum = __builtin_nanf("");
        else if (flags & 2) sum = __builtin_inff();
        else sum = exact_seq_sum<CM>(n, lt, sl, rec_idx, rec_gp, rec_b);
        // fast_attention_simd.rs:485-486.  sqrtf is correctly rounded on the
        // host; the hardware f32 square root is not, so take the correctly
        // rounded double root and round it once (exact: 53 >= 2*24 + 2).
        const float ms = __fadd_rn(__fdiv_rn(sum, (float)n), a.eps);
        const float rms = (float)__dsqrt_rn((double)ms);
        const float invr = __fdiv_rn(1.0f, rms);
#pragma unroll
        for (int c = 0; c < CM; ++c) {
            const int i = (w * C + c) * 64 + lane;
            if (c < C && i < n) v[c] = __fmul_rn(__fmul_rn(v[c], invr), nwv[c]);
        }
    }
    if (a.out) {
        float* orow = a.out + (size_t)m * a.ldo;
#pragma unroll
        for (int c = 0; c < CM; ++c) {
            const int i = (w * C + c) * 64 + lane;
            if (c < C && i < n) orow[i] = v[c];
        }
    }
    if (!a.q) return;
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < CM; ++c) mx = fmaxf(mx, fabsf(v[c]));
    mx = wave_max_nonneg(mx);
    if (lane == 0) sm_f[w] = mx;
    __syncthreads();
    mx = 0.0f;
#pragma unroll
    for (int j = 0; j < kMidWaves; ++j) mx = fmaxf(mx, sm_f[j]);
    const float scale = (mx > 0.0f) ? __fdiv_rn(127.0f, mx) : 1.0f;
    const float invs = (mx > 0.0f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
    int8_t* qr = a.q + (size_t)m * a.ldq;
    int sum = 0;
    // (the rounding mode is chosen once, so that only one quantiser's code
    // runs through the unrolled loop)
    auto quant_row = [&](auto mode_c) {
#pragma unroll
        for (int c = 0; c < CM; ++c) {
            const int i = (w * C + c) * 64 + lane;
            if (c < C && i < n) {
                const int b = quant_one(v[c], scale, decltype(mode_c)::value, i < nmain);
                qr[i] = (int8_t)b;
                sum += b;
            }
        }
    };
    if (a.mode == XT_QUANT_AVX512) quant_row(std::integral_constant<int, XT_QUANT_AVX512>{});
    else quant_row(std::integral_constant<int, XT_QUANT_SCALAR>{});
    for (int i = n + tid; i < a.ldq; i += kMidThreads) qr[i] = 0;
    if (!a.rowsum) {  // the product decodes signed weights or sums the row itself
        if (tid == 0) a.inv[m] = invs;
        return;
    }
    sum = wave_sum_int(sum);
    __syncthreads();  // sm_i reuse after the flag reads
    if (lane == 0) sm_i[w] = sum;
    __syncthreads();
    if (tid == 0) {
        int tot = 0;
        for (int j = 0; j < kMidWaves; ++j) tot += sm_i[j];
        a.inv[m] = invs;
        if (a.rowsum) a.rowsum[m] = tot;
    }
}

int mid_max_cols() { return kMidCmax * kMidThreads; }

hipError_t launch_mlp_mid(const MidArgs& a0, int M, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    MidArgs a = a0;
    a.C = (a.n + kMidThreads - 1) / kMidThreads;
    if (a.n <= 0 || a.C > kMidCmax) return hipErrorInvalidValue;
    const size_t lds = a.norm_w ? (size_t)a.C * kMidThreads * 4 + (size_t)kMidRecMax * 16 : 0;
    // Elements per thread, rounded up to a compiled bound: every per-element
    // loop is unrolled to the bound and runs once, so the smallest bound
    // means the least straight-line code to fetch (measured: n = 6912 with
    // bound 8 instead of 16, 2.8 us less per row).
    const int cm = a.C <= 2 ? 2 : a.C <= 4 ? 4 : a.C <= 8 ? 8 : 16;
#define XT_MID(ACT_, CM_) \
    hipLaunchKernelGGL((mlp_mid_kernel<ACT_, CM_>), dim3(M), dim3(kMidThreads), lds, s, a)
#define XT_MID_CM(ACT_)                 \
    switch (cm) {                       \
        case 2: XT_MID(ACT_, 2); break; \
        case 4: XT_MID(ACT_, 4); break; \
        case 8: XT_MID(ACT_, 8); break; \
        default: XT_MID(ACT_, 16); break; \
    }
    switch (a.act) {
        case XT_ACT_RELU2_MUL: XT_MID_CM(XT_ACT_RELU2_MUL) break;
        case XT_ACT_SILU_INPLACE_AVX512: XT_MID_CM(XT_ACT_SILU_INPLACE_AVX512) break;
        case XT_ACT_SILU_INPLACE_SCALAR: XT_MID_CM(XT_ACT_SILU_INPLACE_SCALAR) break;
        case XT_ACT_SILU_MUL: XT_MID_CM(XT_ACT_SILU_MUL) break;
        case kActIdentity: XT_MID_CM(kActIdentity) break;
        default:
            return hipErrorInvalidValue;
    }
#undef XT_MID_CM
#undef XT_MID
    return hipGetLastError();
}

}  // namespace xt


