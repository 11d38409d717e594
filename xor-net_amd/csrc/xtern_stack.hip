// Persistent decode-stack kernel: one launch runs a whole list of ternary
// projections (a decode step's q/k/v, o, gate/up, down of every layer).
//
// Reference behaviour: the per-layer sequence of TernaryLinear::forward /
// fused_forward_qkv / fused_forward_mlp calls of the BitNet decode step
// (src/models/llama/mod.rs:420-470, which prefetches the next block's
// weights while the current one computes, :446-453), each bit-exact with
// TernaryLinear::forward (src/bit1_58/layers.rs:262-313): per-token absmax
// quantisation (quantization.rs:95-195), exact i32 dots, (f32)dot * inv *
// w_scale.
//
// Work list.  The host flattens the ops into items, op by op: M > 1 ops
// first have M quantiser items (one input row each), then every op has one
// GEMV item per block of up to kSRG 16-row groups of one of its projections
// (all of K).  Workgroups take items in list order from a ticket counter:
// the first item of workgroup b is item b, every later one comes from one
// device-scope atomic add (issued while the current item's weights stream).
// An item that depends on earlier items waits for their completion counter,
// so the earliest unfinished item always has its inputs and is held by a
// running workgroup: the launch finishes whatever the number of resident
// workgroups.  Waits are bounded (a flag tells the host if one gave up).
//
// Coherence across the eight XCDs (each has its own L2): everything one item
// writes for another item of the same launch (op outputs, quantised rows,
// scales) is written with device-scope stores and read with device-scope
// loads, and each completion count is bumped only after the item's stores
// have completed (s_waitcnt + barrier).  No cache-wide fences.
//
// The last workgroup to finish resets the counters, so the next launch
// (stream order) starts from zero without a memset.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xtern_device.h"
#include "xtern_internal.h"

namespace xt {

namespace {

constexpr int kSW = 8;            // waves per workgroup
constexpr int kSNT = kSW * 64;    // threads per workgroup
constexpr int kSRG = kStackRowGroups;  // 16-row groups per GEMV item

// Counter slots, 128 bytes apart: ticket, exit count, error flag, spare, then
// the GEMV completions of every op, then the quantiser completions.
__device__ __forceinline__ unsigned* ctr_at(unsigned* c, int slot) { return c + slot * 32; }
constexpr int kCtrTicket = 0, kCtrExit = 1, kCtrError = 2, kCtrDone0 = 4;

// Device-scope (all XCDs) loads and stores.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr int kCohAux = 16;  // cache policy: device scope
__device__ __forceinline__ v4i ld_coh16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCohAux);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coh_u(unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One lane waits until *c >= target.  Bounded: after `limit` polls it sets
// the error slot and returns; once the slot is set (by any workgroup) every
// wait of the launch returns at once, so a launch that gave up still ends
// promptly (with invalid outputs, reported to the host).
__device__ __forceinline__ void wait_count(unsigned* c, unsigned target, unsigned* err, int limit) {
    for (int n = 0; ld_coh_u(c) < target; ++n) {
        if (n >= limit) {
            st_coh(err, 1u);
            break;
        }
        if ((n & 63) == 63 && ld_coh_u(err)) break;
        __builtin_amdgcn_s_sleep(2);
    }
}

// Every thread's stores have completed, then one count bump.
__device__ __forceinline__ void publish(unsigned* c) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Shared {
    v4i red[kSW][kSRG][64];
    float wmax[kSW];
    unsigned next;
    unsigned last;
};

// Quantiser item: row m of op's input into q / inv (quantization.rs:95-195).
__device__ void quant_item(const StackArgs& a, const StackOpDev* __restrict__ op, int opi, int m,
                           Shared& sh, unsigned* tk) {
    const int K = op->K, n4 = K >> 2, ldq = op->ldq;
    const int dep = op->dep;
    if (threadIdx.x == 0) {
        *tk = __hip_atomic_fetch_add(ctr_at(a.ctr, kCtrTicket), 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        if (dep >= 0)
            wait_count(ctr_at(a.ctr, kCtrDone0 + dep), (unsigned)a.ops[dep].ngemv,
                       ctr_at(a.ctr, kCtrError), a.spin_limit);
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t xr = rsrc(op->x, (unsigned)(a.M * K * 4));
    float4 v[8];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int f = threadIdx.x + u * kSNT;
        const v4i r = ld_coh16(xr, (unsigned)(((size_t)m * K + 4 * min(f, n4 - 1)) * 4));
        v[u] = f < n4 ? make_float4(__int_as_float(r[0]), __int_as_float(r[1]), __int_as_float(r[2]),
                                    __int_as_float(r[3]))
                      : make_float4(0.f, 0.f, 0.f, 0.f);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    }
    const int wm = wave_reduce_bits(__float_as_int(mx), [](int p, int q) {
        return __float_as_int(fmaxf(__int_as_float(p), __int_as_float(q)));
    });
    if ((threadIdx.x & 63) == 0) sh.wmax[threadIdx.x >> 6] = __int_as_float(wm);
    __syncthreads();
    float rmx = sh.wmax[0];
#pragma unroll
    for (int w = 1; w < kSW; ++w) rmx = fmaxf(rmx, sh.wmax[w]);
    const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
    const float invs = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;
    unsigned* qrow = reinterpret_cast<unsigned*>(op->q + (size_t)m * ldq);
    auto body = [&](auto mode_c) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int f = threadIdx.x + u * kSNT;
            if (f < ldq / 4) {
                const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                unsigned w = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    w |= (unsigned)(quant_one(e[t], scale, decltype(mode_c)::value, 4 * f + t < kmain) & 255)
                         << (8 * t);
                st_coh(qrow + f, f < n4 ? w : 0u);
            }
        }
    };
    if (a.mode == XT_QUANT_AVX512) body(std::integral_constant<int, XT_QUANT_AVX512>{});
    else body(std::integral_constant<int, XT_QUANT_SCALAR>{});
    // (ldq <= 16384 = 8 pieces per thread: the loop above covers the padding)
    if (threadIdx.x == 0) st_coh(op->inv + m, invs);
    publish(ctr_at(a.ctr, kCtrDone0 + a.nops + opi));
}

// GEMV item: row groups G0 .. G0 + kSRG - 1 of projection p over all of K,
// for every token.  Wave w multiplies chunks w, w + kSW, ... (NCW of them at
// most); FUSED (M = 1): the item quantises the f32 input row itself, one
// pass, as the decode GEMV does; otherwise it reads the rows quantised by
// the op's quantiser items.
template <int NCW, bool FUSED>
__device__ void gemv_item(const StackArgs& a, const StackOpDev* __restrict__ op, int opi, int blk,
                          Shared& sh, unsigned* tk) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int np = op->nproj;
    const int p = (np > 1 && blk >= op->gend[0]) + (np > 2 && blk >= op->gend[1]) +
                  (np > 3 && blk >= op->gend[2]);
    const int b0 = p ? op->gend[p - 1] : 0;
    const int G0 = (blk - b0) * kSRG;
    const int N = op->N[p], NG = (N + 15) >> 4;
    const int nch = op->nch, K = op->K, M = a.M;
    const uint8_t* tiles = op->tiles[p];

    v4i wv[NCW][kSRG];
#pragma unroll
    for (int t = 0; t < NCW; ++t) {
        const int c = min(wave + t * kSW, nch - 1);
#pragma unroll
        for (int r = 0; r < kSRG; ++r)
            wv[t][r] = ld_stream(tiles + (((size_t)min(G0 + r, NG - 1) * nch + c) * 64 + lane) * 16);
    }
    const int o = (G0 + min(wave, kSRG - 1)) * 16 + j;
    const float wscale = op->ws[p][min(o, N - 1)];
    if (threadIdx.x == 0) {
        *tk = __hip_atomic_fetch_add(ctr_at(a.ctr, kCtrTicket), 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        if (FUSED) {
            if (op->dep >= 0)
                wait_count(ctr_at(a.ctr, kCtrDone0 + op->dep), (unsigned)a.ops[op->dep].ngemv,
                           ctr_at(a.ctr, kCtrError), a.spin_limit);
        } else {
            wait_count(ctr_at(a.ctr, kCtrDone0 + a.nops + opi), (unsigned)M, ctr_at(a.ctr, kCtrError),
                       a.spin_limit);
        }
    }
    __syncthreads();

    const int ntb = FUSED ? 1 : (M + 15) >> 4;
    for (int tb = 0; tb < ntb; ++tb) {
        const int mt = FUSED ? 1 : min(16, M - 16 * tb);  // tokens of this block
        v4i av[NCW][4];
        float invr[4];
        if constexpr (FUSED) {
            const int n4 = K >> 2;
            const __amdgpu_buffer_rsrc_t xr = rsrc(op->x, (unsigned)(K * 4));
            float4 x0[NCW];
            float mx = 0.0f;
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
                const int f = (wave + t * kSW) * 64 + lane;
                const v4i r = ld_coh16(xr, (unsigned)(4 * min(f, n4 - 1) * 4));
                x0[t] = f < n4 ? make_float4(__int_as_float(r[0]), __int_as_float(r[1]),
                                             __int_as_float(r[2]), __int_as_float(r[3]))
                               : make_float4(0.f, 0.f, 0.f, 0.f);
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x0[t].x), fabsf(x0[t].y)),
                                     fmaxf(fabsf(x0[t].z), fabsf(x0[t].w))));
            }
            // (pieces of chunks beyond nch lie past K and read as zero)
            const int wm = wave_reduce_bits(__float_as_int(mx), [](int p_, int q_) {
                return __float_as_int(fmaxf(__int_as_float(p_), __int_as_float(q_)));
            });
            if (lane == 0) sh.wmax[wave] = __int_as_float(wm);
            __syncthreads();
            float rmx = sh.wmax[0];
#pragma unroll
            for (int w = 1; w < kSW; ++w) rmx = fmaxf(rmx, sh.wmax[w]);
            const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
            const float iv = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) invr[r] = iv;
            const int kmain = (K / 16) * 16;
            unsigned w4[NCW];
            auto pack = [&](auto mode_c) {
#pragma unroll
                for (int t = 0; t < NCW; ++t) {
                    const int f = (wave + t * kSW) * 64 + lane;
                    const float e4[4] = {x0[t].x, x0[t].y, x0[t].z, x0[t].w};
                    unsigned r = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        r |= (unsigned)(quant_one(e4[e], scale, decltype(mode_c)::value, 4 * f + e < kmain) & 255)
                             << (8 * e);
                    w4[t] = f < n4 ? r : 0u;
                }
            };
            if (a.mode == XT_QUANT_AVX512) pack(std::integral_constant<int, XT_QUANT_AVX512>{});
            else pack(std::integral_constant<int, XT_QUANT_SCALAR>{});
            // lane (g, j) of k-step s takes the chunk's packed pieces 16 s + 4 g + d
#pragma unroll
            for (int t = 0; t < NCW; ++t)
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        av[t][s][d] = __builtin_amdgcn_ds_bpermute((16 * s + 4 * g + d) << 2, (int)w4[t]);
        } else {
            const int ldq = op->ldq;
            const __amdgpu_buffer_rsrc_t qr = rsrc(op->q, (unsigned)(M * ldq));
            const __amdgpu_buffer_rsrc_t ir = rsrc(op->inv, (unsigned)(M * 4));
            const int row = 16 * tb + min(j, mt - 1);
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
                const int c = min(wave + t * kSW, nch - 1);
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    av[t][s] = ld_coh16(qr, (unsigned)((size_t)row * ldq + c * 256 + s * 64 + 16 * g));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                invr[r] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    ir, (unsigned)(16 * tb + min(4 * g + r, mt - 1)) * 4, 0, kCohAux));
        }
        // (the weights stay packed across token blocks: without this the
        // compiler hoists every decoded weight out of the loop)
#pragma unroll
        for (int t = 0; t < NCW; ++t)
#pragma unroll
            for (int r = 0; r < kSRG; ++r) asm volatile("" : "+v"(wv[t][r]));
        v4i acc[kSRG];
#pragma unroll
        for (int r = 0; r < kSRG; ++r) acc[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            const bool live = wave + t * kSW < nch;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const v4i x = (live && j < mt) ? av[t][s] : v4i{0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < kSRG; ++r) {
                    v4i b = decode4(wv[t][r][s]);
#pragma unroll
                    for (int d = 0; d < 4; ++d) b[d] = signed_codes(b[d]);
                    acc[r] = mfma(x, b, acc[r]);
                }
            }
        }
        if (tb > 0) __syncthreads();  // the previous block's sums are read
#pragma unroll
        for (int r = 0; r < kSRG; ++r) sh.red[wave][r][lane] = acc[r];
        __syncthreads();
        if (wave < kSRG && G0 + wave < NG && o < N) {
            v4i sum = sh.red[0][wave][lane];
#pragma unroll
            for (int w = 1; w < kSW; ++w) sum += sh.red[w][wave][lane];
            float* y = op->y[p];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 4 * g + r;
                if (i < mt)  // layers.rs:294 -- (dot as f32 * inv_scale) * w_scale
                    st_coh(y + (size_t)(16 * tb + i) * N + o,
                           __fmul_rn(__fmul_rn((float)sum[r], invr[r]), wscale));
            }
        }
    }
    publish(ctr_at(a.ctr, kCtrDone0 + opi));
}

__global__ __launch_bounds__(kSNT) void stack_kernel(const StackArgs a) {
    __shared__ Shared sh;
    unsigned t = blockIdx.x;
    while (t < (unsigned)a.nitems) {
        const uint32_t it = a.items[t];
        const int opi = (int)(it >> 20), local = (int)(it & 0xfffff);
        const StackOpDev* op = a.ops + opi;
        unsigned tk = 0;
        if (local < op->nq) {
            quant_item(a, op, opi, local, sh, &tk);
        } else {
            const int blk = local - op->nq;
            const int ncw = (op->nch + kSW - 1) / kSW;
            if (a.M == 1) {
                if (ncw <= 2) gemv_item<2, true>(a, op, opi, blk, sh, &tk);
                else gemv_item<4, true>(a, op, opi, blk, sh, &tk);
            } else {
                if (ncw <= 2) gemv_item<2, false>(a, op, opi, blk, sh, &tk);
                else gemv_item<4, false>(a, op, opi, blk, sh, &tk);
            }
        }
        if (threadIdx.x == 0) sh.next = tk + gridDim.x;
        __syncthreads();
        t = sh.next;
    }
    // the last workgroup out resets the counters for the next launch (its
    // own completion bumps have been performed before its exit is counted)
    if (threadIdx.x == 0) {
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned old = __hip_atomic_fetch_add(ctr_at(a.ctr, kCtrExit), 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        sh.last = old == gridDim.x - 1;
    }
    __syncthreads();
    if (sh.last) {
        for (int i = threadIdx.x; i < a.nops; i += kSNT) {
            st_coh(ctr_at(a.ctr, kCtrDone0 + i), 0u);
            st_coh(ctr_at(a.ctr, kCtrDone0 + a.nops + i), 0u);
        }
        if (threadIdx.x == 0) {
            st_coh(ctr_at(a.ctr, kCtrTicket), 0u);
            st_coh(ctr_at(a.ctr, kCtrExit), 0u);
        }
    }
}

}  // namespace

int stack_threads() { return kSNT; }
int stack_max_chunks() { return 4 * kSW; }

hipError_t launch_stack(const StackArgs& a, int blocks, hipStream_t s) {
    hipLaunchKernelGGL(stack_kernel, dim3(blocks), dim3(kSNT), 0, s, a);
    return hipGetLastError();
}

hipError_t stack_blocks_per_cu(int* n) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, reinterpret_cast<const void*>(stack_kernel),
                                                        kSNT, 0);
}

}  // namespace xt
