// Persistent decode-stack kernel for 17 to 32 tokens (up to 16 take the
// streaming stack, xtern_sstack.hip): one launch runs a whole list of ternary
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
// Work list.  The host flattens the ops into items: every op has quantiser
// items (kSW input rows each) and one GEMV item per block of 8 (K up to 16
// chunks) or 4 16-row groups of one of its projections (all of K).  It then
// deals the list out to the workgroups (greedy, by bytes), each workgroup
// getting its items in list order, and every item after the items it waits
// for.  With every workgroup of the launch resident at once (the grid is
// sized to the occupancy), the earliest unfinished item is always being
// worked on and has its inputs, so the launch always finishes.  Waits are
// bounded anyway: one that gives up sets a flag for the host, and all later
// waits of the launch return at once.
//
// Each workgroup copies every op descriptor and its own item list into LDS at
// entry, so an item starts without a global load (which would also wait for
// the previous item's stores: memory operations complete in issue order).  Weights are read with
// buffer loads whose per-wave part of the address is a scalar offset, and
// whose out-of-range parts (rows past N, chunks past K) read as zero without
// touching memory.
//
// Coherence across the eight XCDs (each has its own L2): everything one item
// writes for another item of the same launch (op outputs, quantised rows,
// scales) is written with device-scope stores and read with device-scope
// loads, and a completion count is bumped only after the item's stores have
// completed (s_waitcnt + barrier).  No cache-wide fences.  A workgroup that
// has seen an op complete remembers it (one LDS bit), so later items that
// depend on the same op skip the poll.
//
// The last workgroup to finish resets the counters, so the next launch
// (stream order) starts from zero without a memset.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include "xtern_device.h"
#include "xtern_internal.h"

namespace xt {

namespace {

constexpr int kSW = 8;                 // waves per workgroup
constexpr int kSNT = kSW * 64;         // threads per workgroup
constexpr int kDescWords = sizeof(StackOpDev) / 4;
static_assert(kDescWords <= 64 && sizeof(StackOpDev) % 4 == 0, "a descriptor is one wave load");

// Counter slots, 128 bytes apart: exit count, error flag, spares, then the
// GEMV completions of every op, then the quantiser completions.
__device__ __forceinline__ unsigned* ctr_at(unsigned* c, int slot) { return c + slot * 32; }
constexpr int kCtrExit = 1, kCtrError = 2, kCtrDone0 = 4;

// Buffer resources (uniform).  num_records bounds every access whose vector
// offset (plus instruction offset) is past it: such a load returns zeros and
// reads no memory.  The scalar offset is not part of that check, so every
// offset here goes in the vector offset and the scalar offset stays 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr unsigned kOutOfRange = 0x80000000u;  // an offset past every resource
constexpr int kAuxStream = 2;   // cache policy: non-temporal (weights, read once)
constexpr int kAuxCoh = 16;     // cache policy: device scope (data written in the launch)
// (voff: the lane's part, below 2^31; off: the uniform part, or kOutOfRange)
__device__ __forceinline__ v4i ld_coh16(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned off = 0) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff + off, 0, kAuxCoh);
}
__device__ __forceinline__ v4i ld_w16(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff + off, 0, kAuxStream);
}
// Stores through a buffer resource (the descriptor's pointers carry no
// address space, and flat accesses would also count against LDS waits).
__device__ __forceinline__ void st_buf(__amdgpu_buffer_rsrc_t r, unsigned off, unsigned v, bool coh) {
    if (coh) __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kAuxCoh);
    else __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
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

constexpr int kDescLdsWords = kStackDescLdsBytes / 4;
constexpr int kKnownWords = kStackMaxOps * 2 / 32 + 1;

struct Shared {
    v4i red[kSW][kStackRowGroupsMax][64];
    unsigned desc[kDescLdsWords];          // every op descriptor
    unsigned items[kStackMaxWgItems];      // this workgroup's items, in order
    unsigned known[kKnownWords];           // completions this workgroup has seen
    unsigned last;
};

static_assert(kStackRowGroupsMax * 64 >= 16 * 17, "a wave's reduction stage holds its activation slice");

__device__ __forceinline__ unsigned* done_ctr(const StackArgs& a, int op) {
    return ctr_at(a.ctr, kCtrDone0 + op);
}
__device__ __forceinline__ unsigned* qdone_ctr(const StackArgs& a, int op) {
    return ctr_at(a.ctr, kCtrDone0 + a.nops + op);
}

// An op descriptor held as one vector register: lane k holds dword k (from
// the LDS copy).  Fields come out with v_readlane at a uniform (possibly
// computed) lane, straight into scalar registers.  (A descriptor struct in
// registers with a computed index into one of its arrays lands in scratch
// memory, and a scratch load waits for every memory operation in flight.)
struct OpRef {
    unsigned v;
    __device__ __forceinline__ int i(unsigned off) const {
        return (int)__builtin_amdgcn_readlane(v, (int)(off / 4));
    }
    template <typename T>
    __device__ __forceinline__ T* ptr(unsigned off) const {
        const uint32_t lo = __builtin_amdgcn_readlane(v, (int)(off / 4));
        const uint32_t hi = __builtin_amdgcn_readlane(v, (int)(off / 4 + 1));
        return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
    }
};
#define OPF(field) ((unsigned)offsetof(StackOpDev, field))
// Call with every lane of the wave active: lane k reads dword k, and a field
// read from a lane that skipped the load would be whatever that register
// held before.
__device__ __forceinline__ OpRef load_op(const Shared& sh, int opi) {
    const int lane = threadIdx.x & 63;
    unsigned v = sh.desc[opi * kDescWords + min(lane, kDescWords - 1)];
    // pins the read here: otherwise the compiler may move it into a branch
    // that uses the descriptor, where only some lanes execute it
    asm volatile("" : "+v"(v));
    return OpRef{v};
}
// Values the compiler cannot prove wave-uniform, moved to scalar registers
// (a buffer resource or scalar offset built from a vector register turns
// every load into a loop over the distinct values).
template <typename T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Wait (lane 0 of this wave; no workgroup barrier) until counter `slot`
// (an op's GEMV completions: slot = op; its quantiser rows: nops + op)
// reaches target, unless this workgroup has already seen it get there.
__device__ __forceinline__ void wave_wait(const StackArgs& a, Shared& sh, int slot, unsigned target) {
    const unsigned bit = 1u << (slot & 31);
    if (sh.known[slot >> 5] & bit) return;  // (uniform: an LDS word read by every lane)
    if ((threadIdx.x & 63) == 0) {
        wait_count(ctr_at(a.ctr, kCtrDone0 + slot), target, ctr_at(a.ctr, kCtrError), a.spin_limit);
        atomicOr(&sh.known[slot >> 5], bit);
    }
    __builtin_amdgcn_wave_barrier();
}

// Quantiser item: rows r0 .. r0 + kSW - 1 of op's input (one row per wave)
// into q / inv (quantization.rs:95-195): pass 1 the row's absmax, pass 2
// quantise and store (the row is read twice; no barrier).  per_item: the
// completion bumps each GEMV item of the op it depends on makes (one, or
// one per wave in the M = 1 kernel).
__device__ void quant_item(const StackArgs& a, Shared& sh, const OpRef& d, int opi, int r0,
                           unsigned per_item) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int K = d.i(OPF(K)), n4 = K >> 2, ldq = d.i(OPF(ldq)), M = a.M;
    const int rows = min(kSW, M - r0);
    const int dep = d.i(OPF(dep));
    if (dep >= 0) wave_wait(a, sh, dep, (unsigned)d.i(OPF(dep_items)) * per_item);
    const int m = r0 + min(wave, rows - 1);
    // one row per resource: pieces past K read as zero
    const __amdgpu_buffer_rsrc_t xr = rsrc(d.ptr<const float>(OPF(x)) + (size_t)m * K, (unsigned)(K * 4));
    float mx = 0.0f;
    for (int f0 = 0; f0 < n4; f0 += 4 * 64) {
        v4i r[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) r[u] = ld_coh16(xr, (unsigned)(f0 + u * 64 + lane) * 16u);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(__int_as_float(r[u][e])));
    }
    const float rmx = __int_as_float(wave_reduce_bits(__float_as_int(mx), [](int p, int q) {
        return __float_as_int(fmaxf(__int_as_float(p), __int_as_float(q)));
    }));
    const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
    const float invs = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;
    const __amdgpu_buffer_rsrc_t qr = rsrc(d.ptr<int8_t>(OPF(q)) + (size_t)m * ldq, (unsigned)ldq);
    const bool mine = wave < rows;
    auto body = [&](auto mode_c) {
        for (int f0 = 0; f0 < ldq / 4; f0 += 64) {  // one 256-column chunk per trip
            const int f = f0 + lane;
            const v4i r = ld_coh16(xr, (unsigned)f * 16u);  // zeros past K: code 0
            unsigned w = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                w |= (unsigned)(quant_one(__int_as_float(r[t]), scale, decltype(mode_c)::value,
                                          4 * f + t < kmain) & 255) << (8 * t);
            if (mine) st_buf(qr, (unsigned)f * 4u, w, true);
        }
    };
    if (a.mode == XT_QUANT_AVX512) body(std::integral_constant<int, XT_QUANT_AVX512>{});
    else body(std::integral_constant<int, XT_QUANT_SCALAR>{});
    if (mine && lane == 0)
        st_buf(rsrc(d.ptr<float>(OPF(inv)), (unsigned)(M * 4)), (unsigned)m * 4u, __float_as_uint(invs), true);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(qdone_ctr(a, opi), (unsigned)rows, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// GEMV item: row groups G0 .. G0 + RG - 1 of projection p over all of K,
// for every token.  Wave w multiplies chunks w, w + kSW, ... (NCW of them at
// most), reading the rows the op's quantiser items wrote.
template <int NCW, int RG>
__device__ void gemv_item(const StackArgs& a, Shared& sh, const OpRef& d, int opi, int blk,
                          int pos) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int g = lane >> 4, j = lane & 15;
    const int np = d.i(OPF(nproj));
    const int ge0 = d.i(OPF(gend)), ge1 = d.i(OPF(gend) + 4), ge2 = d.i(OPF(gend) + 8);
    const int p = (np > 1 && blk >= ge0) + (np > 2 && blk >= ge1) + (np > 3 && blk >= ge2);
    const int b0 = p == 0 ? 0 : d.i(OPF(gend) + 4 * (p - 1));
    const int G0 = (blk - b0) * RG;
    const int N = d.i(OPF(N) + 4 * p), NG = (N + 15) >> 4;
    const int nch = d.i(OPF(nch)), M = a.M;
    const bool pub = d.i(OPF(pub)) != 0;
    const __amdgpu_buffer_rsrc_t wr =
        rsrc(d.ptr<const uint8_t>(OPF(tiles) + 8 * p), (unsigned)(NG * nch * 1024));
    const unsigned voff = (unsigned)lane * 16u;
    v4i wv[NCW][RG];
#pragma unroll
    for (int t = 0; t < NCW; ++t) {
        const int c = wave + t * kSW;
#pragma unroll
        for (int r = 0; r < RG; ++r)  // (rows past N and chunks past K: zeros, no memory read)
            wv[t][r] = ld_w16(wr, voff, c < nch ? (unsigned)(((G0 + r) * nch + c) * 1024) : kOutOfRange);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int o = (G0 + min(wave, RG - 1)) * 16 + j;
    const float wscale = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        rsrc(d.ptr<const float>(OPF(ws) + 8 * p), (unsigned)(N * 4)), (unsigned)min(o, N - 1) * 4u, 0, 0));
    wave_wait(a, sh, a.nops + opi, (unsigned)M);

    const int ntb = (M + 15) >> 4;
    for (int tb = 0; tb < ntb; ++tb) {
        // the previous block's sums are read (its reduction stage doubles as
        // this block's activation slice)
        if (tb > 0) __syncthreads();
        const int mt = min(16, M - 16 * tb);  // tokens of this block
        float invr[4];
        v4i aq[NCW][4];
        {
            const int ldq = d.i(OPF(ldq));
            const __amdgpu_buffer_rsrc_t qr = rsrc(d.ptr<const int8_t>(OPF(q)), (unsigned)(M * ldq));
            const __amdgpu_buffer_rsrc_t ir = rsrc(d.ptr<const float>(OPF(inv)), (unsigned)(M * 4));
            // Each load covers 4 token rows x 256 contiguous bytes of a
            // chunk (a load spanning the 16 rows at the row stride kept the
            // address path stalled on translation); chunk by chunk the rows go
            // through this wave's part of the reduction stage (rows padded by
            // one piece) and come back as the MFMA fragments of lane (g, j):
            // row j, pieces 4 s + g.  A wave's LDS accesses complete in order.
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
                const int c = min(wave + t * kSW, nch - 1);
#pragma unroll
                for (int u = 0; u < 4; ++u) {  // (rows past the block: zeros, no memory read)
                    const int r = 4 * u + (lane >> 4);
                    aq[t][u] = ld_coh16(qr, r < mt ? (unsigned)((size_t)(16 * tb + r) * ldq + c * 256 + (lane & 15) * 16)
                                                   : kOutOfRange);
                }
            }
            v4i* slice = &sh.red[wave][0][0];  // 16 x 17 pieces of the wave's 8 x 64
#pragma unroll
            for (int t = 0; t < NCW; ++t) {
#pragma unroll
                for (int u = 0; u < 4; ++u) slice[(4 * u + (lane >> 4)) * 17 + (lane & 15)] = aq[t][u];
                __asm__ volatile("" ::: "memory");
#pragma unroll
                for (int s = 0; s < 4; ++s) aq[t][s] = slice[j * 17 + 4 * s + g];
                __asm__ volatile("" ::: "memory");
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                invr[r] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    ir, (unsigned)(16 * tb + min(4 * g + r, mt - 1)) * 4, 0, kAuxCoh));
        }
        // (the weights stay packed across token blocks: without this the
        // compiler hoists every decoded weight out of the loop)
#pragma unroll
        for (int t = 0; t < NCW; ++t)
#pragma unroll
            for (int r = 0; r < RG; ++r) asm volatile("" : "+v"(wv[t][r]));
        v4i acc[RG];
#pragma unroll
        for (int r = 0; r < RG; ++r) acc[r] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NCW; ++t) {
            // (chunks past K: the loads above clamp to the last chunk, so
            // those waves skip it)
            const bool live = wave + t * kSW < nch;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const v4i x = (live && j < mt) ? aq[t][s] : v4i{0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < RG; ++r) {
                    v4i b = decode4(wv[t][r][s]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) b[e] = signed_codes(b[e]);
                    acc[r] = mfma(x, b, acc[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RG; ++r) sh.red[wave][r][lane] = acc[r];
        __syncthreads();
        if (wave < RG && G0 + wave < NG && o < N) {
            v4i sum = sh.red[0][wave][lane];
#pragma unroll
            for (int w = 1; w < kSW; ++w) sum += sh.red[w][wave][lane];
            const __amdgpu_buffer_rsrc_t yr = rsrc(d.ptr<float>(OPF(y) + 8 * p), (unsigned)(M * N * 4));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 4 * g + r;
                // layers.rs:294 -- (dot as f32 * inv_scale) * w_scale; device-scope
                // stores only where another op of the launch reads the output
                const float v = __fmul_rn(__fmul_rn((float)sum[r], invr[r]), wscale);
                if (i < mt) st_buf(yr, (unsigned)((16 * tb + i) * N + o) * 4u, __float_as_uint(v), pub);
            }
        }
    }
    if (pub) {  // another op reads these outputs inside the launch
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(done_ctr(a, opi), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __syncthreads();  // the reduction stage is read before the next item writes it
    }
}

// (two waves per SIMD: two workgroups per CU)
__global__ __launch_bounds__(kSNT, 2) void stack_kernel(const StackArgs a) {
    __shared__ Shared sh;
    // this workgroup's items and (when they fit) every op descriptor into LDS
    const int i0 = a.sched_off[blockIdx.x], n = a.sched_off[blockIdx.x + 1] - i0;
    for (int i = threadIdx.x; i < n; i += kSNT) sh.items[i] = a.sched[i0 + i];
    for (int i = threadIdx.x; i < a.nops * kDescWords; i += kSNT)
        sh.desc[i] = reinterpret_cast<const unsigned*>(a.ops)[i];
    for (int i = threadIdx.x; i < kKnownWords; i += kSNT) sh.known[i] = 0u;
    __syncthreads();
    for (int k = 0; k < n; ++k) {
        const unsigned it = __builtin_amdgcn_readfirstlane(sh.items[k]);
        const int opi = (int)(it >> 20), local = (int)(it & 0xfffff);
        const OpRef op = load_op(sh, opi);
        const int nq = op.i(OPF(nq));
        if (local < nq) {
            quant_item(a, sh, op, opi, local * kSW, 1u);
        } else {
            const int blk = local - nq;
            // (row groups per item as the host dealt them: stack_gemv_rg)
            if ((op.i(OPF(nch)) + kSW - 1) / kSW <= 2) gemv_item<2, 8>(a, sh, op, opi, blk, i0 + k);
            else gemv_item<4, 4>(a, sh, op, opi, blk, i0 + k);
        }
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
            st_coh(done_ctr(a, i), 0u);
            st_coh(qdone_ctr(a, i), 0u);
        }
        if (threadIdx.x == 0) st_coh(ctr_at(a.ctr, kCtrExit), 0u);
    }
}

}  // namespace

int stack_threads() { return kSNT; }
int stack_max_chunks() { return 4 * kSW; }
int stack_rows_per_quant_item() { return kSW; }
int stack_gemv_rg(int nch) { return (nch + kSW - 1) / kSW <= 2 ? 8 : 4; }

hipError_t launch_stack(const StackArgs& a, int blocks, hipStream_t s) {
    hipLaunchKernelGGL(stack_kernel, dim3(blocks), dim3(kSNT), 0, s, a);
    return hipGetLastError();
}

hipError_t stack_blocks_per_cu(int* n) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, reinterpret_cast<const void*>(stack_kernel), kSNT, 0);
}

}  // namespace xt
