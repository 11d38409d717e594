// Streaming decode stack (M = 1 .. 32 tokens): a whole list of ternary
// projections in one launch, every wave walking its own sequence of tasks.
//
// Reference behaviour: the layer loop of the BitNet decode step
// (src/models/llama/mod.rs:420-470) calls TernaryLinear::forward /
// fused_forward_qkv / fused_forward_mlp per projection, each bit-exact with
// TernaryLinear::forward (src/bit1_58/layers.rs:262-313): per-token absmax
// quantisation (quantization.rs:95-195), the exact i32 dot of `dot_row`
// (:216-231) over pack4 / pack5 / sparse weights, (f32)dot * inv * w_scale.
//
// Work list.  The host flattens the ops into tasks: (M > 1) one quantiser task per
// op and token (the token's f32 input row -> i8 row, its exact sum and
// inverse scale) and one task per block of consecutive 16-row groups of one
// projection (at M = 1 the group tasks quantise the row themselves:
// ss_mblock_q1).  Every task follows the tasks it waits for: an op's
// quantiser tasks (or, at M = 1, its group tasks) come after the last group
// of the op its input comes from, its groups after its quantiser tasks.  The host deals the list out to the
// waves in list order, each task to the wave with the least work so far
// (weight bytes), and every wave runs its tasks in list order.  The grid is
// no larger than what is resident at once, so the wave holding the earliest
// unfinished task is running and has its inputs, and the launch always
// finishes.  Waits are bounded anyway: one that gives up sets a flag for the
// host, and all later waits of the launch return at once.
//
// A group task walks its block of R row groups chunk by chunk (ss_mblock;
// ss_mblock_q1 at M = 1): one step loads the R groups' tiles of a chunk and
// the chunk's pieces of the op's M quantised rows, stages the pieces in the
// wave's own LDS region (no barrier: a wave's LDS accesses complete in
// order) and runs the R groups' MFMAs on the same A fragments.  Every wave
// keeps its own loads in flight, with no workgroup-wide phases: R = 8 at two
// waves per SIMD keeps 64 KB of weights in flight per CU (the token forms
// and their measurements are listed with the instantiations below).
//
// Coherence across the eight XCDs (each has its own L2): quantised rows are
// written with device-scope stores and counted once the stores have
// completed; readers load them only after the count shows all M tokens
// done (see ss_mblock).  Outputs other ops read inside the launch are
// written with device-scope stores and counted the same way.  The last wave
// out resets the counts, so the next launch starts from zero without a
// memset.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "xtern_device.h"
#include "xtern_internal.h"

namespace xt {

namespace {

constexpr int kSsW = 4;   // waves per workgroup
constexpr int kSsKnownWords = kSStackMaxOps / 32 + 1;

__device__ __forceinline__ unsigned* ss_ctr(unsigned* c, int slot) { return c + slot * 32; }
constexpr int kSsExit = 1, kSsError = 2, kSsDone0 = 4;
constexpr int kSsQuant = 1, kSsPub = 2, kSsPack5 = 4;  // SStackTask::flags

__device__ __forceinline__ unsigned ss_ld_coh(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ss_st_coh(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-scope 16-byte loads and 4-byte stores through buffer resources
// (cache policy 16: coherent across the XCDs' L2s).  Offsets past the
// resource read zeros without a memory access.
constexpr int kSsCoh = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ss_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i ss_ld_coh16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSsCoh);
}
__device__ __forceinline__ void ss_st_coh4(__amdgpu_buffer_rsrc_t r, unsigned off, unsigned v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kSsCoh);
}

// Lane 0 waits until *c >= target (bounded; see the file comment).
__device__ __forceinline__ void ss_wait(unsigned* c, unsigned target, unsigned* err, int limit) {
    for (int n = 0; ss_ld_coh(c) < target; ++n) {
        if (n >= limit) {
            ss_st_coh(err, 1u);
            break;
        }
        if ((n & 63) == 63 && ss_ld_coh(err)) break;
        __builtin_amdgcn_s_sleep(2);
    }
}

// Pointers read from a task record are generic; loads and stores through
// them are given the global address space explicitly, so they are not flat
// accesses (a flat access counts against the LDS wait counter too, and every
// LDS read of the wave would then wait for the weight loads in flight).
typedef __attribute__((address_space(1))) const v4i gv4i;
typedef __attribute__((address_space(1))) const float gfloat;
typedef __attribute__((address_space(1))) float gfloat_w;
__device__ __forceinline__ v4i ss_ld_tile(const uint8_t* p) {
    return __builtin_nontemporal_load((gv4i*)(uintptr_t)p);
}

__device__ __forceinline__ v4i ss_lds16(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) v4i*>((uintptr_t)addr);
}

// A task record, as uniform values (see SStackTask).
struct Rec {
    const uint8_t* tiles;  // group: the group's first tile; quantiser: the f32 input row
    const float* ws;       // group: w_scales of its 16 rows
    float* y;              // group: outputs of its 16 rows
    int8_t* q;             // the op's i8 row, then its sum and inverse scale
    int opi, flags, nch, nrows, K, ldq, dep, dep_groups, ngroups;
};
// A record is loaded one task ahead, dword k into lane k (one register),
// and its fields are read out with readlane when its task starts (reading
// them right after the load would wait for it there).
__device__ __forceinline__ unsigned ss_rec_load(const SStackTask* t) {
    const int lane = threadIdx.x & 63;
    return reinterpret_cast<const unsigned*>(t)[lane & 15];
}
__device__ __forceinline__ Rec ss_rec(unsigned w) {
    auto u = [&](int k) { return (uint32_t)__builtin_amdgcn_readlane((int)w, k); };
    auto ptr = [&](int k) { return (uint64_t)u(k) | ((uint64_t)u(k + 1) << 32); };
    Rec r;
    r.tiles = reinterpret_cast<const uint8_t*>(ptr(0));
    r.ws = reinterpret_cast<const float*>(ptr(2));
    r.y = reinterpret_cast<float*>(ptr(4));
    r.q = reinterpret_cast<int8_t*>(ptr(6));
    r.opi = (int)u(8);
    r.flags = (int)u(9) & 0xffff;
    r.ngroups = (int)(u(9) >> 16);
    r.nch = (int)u(10);
    r.nrows = (int)u(11);
    r.K = (int)u(12);
    r.ldq = (int)u(13);
    r.dep = (int)u(14);
    r.dep_groups = (int)u(15);
    return r;
}

// A quantiser task (one wave, one token of an op): quantization.rs:95-195 on
// the f32 row -> i8 row (zero from K to ldq), its exact sum and its inverse
// scale; the op's count of quantised tokens goes up by one.
template <int MODE>
__device__ void ss_quant(const SStackArgs& a, const Rec& r) {
    const int lane = threadIdx.x & 63;
    const int K = r.K, n4 = K >> 2;
    const bool coh = r.dep >= 0;  // the input is written inside the launch
    if (coh && lane == 0)
        ss_wait(ss_ctr(a.ctr, kSsDone0 + r.dep), (unsigned)r.dep_groups, ss_ctr(a.ctr, kSsError), a.spin_limit);
    __builtin_amdgcn_wave_barrier();
    // pieces past K read as zero; an input written before the launch takes
    // ordinary cached loads
    const __amdgpu_buffer_rsrc_t xr = ss_rsrc(r.tiles, (unsigned)(K * 4));
    auto load4 = [&](int f) -> float4 {
        const v4i v = coh ? ss_ld_coh16(xr, (unsigned)f * 16u)
                          : __builtin_amdgcn_raw_buffer_load_b128(xr, (unsigned)f * 16u, 0, 0);
        return make_float4(__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]),
                           __int_as_float(v[3]));
    };
    // the row in rounds of kSsQ pieces per lane, all of a round's loads in
    // flight at once; a row of at most one round stays in
    // registers for the second pass (12: K <= 3072 in one round, and the
    // kernel stays within 128 VGPRs, four waves per SIMD)
    constexpr int kSsQ = 12;
    const int rounds = (n4 + 64 * kSsQ - 1) / (64 * kSsQ);
    float4 v[kSsQ];
    float mx = 0.0f;
    for (int rd = 0; rd < rounds; ++rd) {
#pragma unroll
        for (int u = 0; u < kSsQ; ++u) v[u] = load4((rd * kSsQ + u) * 64 + lane);
#pragma unroll
        for (int u = 0; u < kSsQ; ++u)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    }
    const float rmx = __int_as_float(wave_reduce_bits(__float_as_int(mx), [](int p, int q) {
        return __float_as_int(fmaxf(__int_as_float(p), __int_as_float(q)));
    }));
    const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
    const float invs = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;
    int rs = 0;
    const __amdgpu_buffer_rsrc_t qr = ss_rsrc(r.q, (unsigned)r.ldq);
    const int n4q = r.ldq / 4;  // (ldq >= K: the i8 row is zero from K on)
    const int qrounds = (n4q + 64 * kSsQ - 1) / (64 * kSsQ);
    for (int rd = 0; rd < qrounds; ++rd) {
        if (rounds > 1 || rd > 0) {  // (uniform) reload: the registers hold one round only
#pragma unroll
            for (int u = 0; u < kSsQ; ++u) v[u] = load4((rd * kSsQ + u) * 64 + lane);
        }
#pragma unroll
        for (int u = 0; u < kSsQ; ++u) {
            const int f = (rd * kSsQ + u) * 64 + lane;
            const float e4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            unsigned w = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                w |= (unsigned)(quant_one(e4[t], scale, MODE, 4 * f + t < kmain) & 255) << (8 * t);
            rs = __builtin_amdgcn_sdot4((int)w, 0x01010101, rs, false);
            // (pieces past ldq land out of the resource: no store)
            ss_st_coh4(qr, f < n4q ? (unsigned)f * 4u : 0x80000000u, w);
        }
    }
    rs = wave_reduce_bits(rs, [](int p, int q) { return p + q; });
    if (lane == 0) {  // the token's sum, and its inverse scale M slots later
        const __amdgpu_buffer_rsrc_t sr = ss_rsrc(r.ws, (unsigned)(4 * a.M + 4));
        ss_st_coh4(sr, 0u, (unsigned)rs);
        ss_st_coh4(sr, (unsigned)(4 * a.M), __float_as_uint(invs));
    }
    __builtin_amdgcn_s_waitcnt(0);  // (vmcnt and lgkmcnt 0: every store has completed)
    if (lane == 0)
        __hip_atomic_fetch_add(ss_ctr(a.ctr, kSsDone0 + a.nops + r.opi), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// A group task (M up to 32 tokens): a block of r.ngroups (<= R) consecutive
// 16-row groups of one projection, walked chunk by chunk: each step loads
// the block's tiles of one chunk (one per group) and the chunk's 16-byte
// pieces of the M quantised rows, puts the pieces in this wave's LDS region
// (16 token rows of CH bytes, padded) and multiplies every group's tile with
// the same A fragments, so the activation bytes are read once per block
// rather than once per group.  The rows are read with ordinary loads, and
// only after the op's count shows all M tokens quantised: nothing on this
// XCD has read those lines during the launch before (the L2s start a launch
// empty of them), every token's row starts on its own 128-byte line (the
// host pads the row pitch), so its L2 holds no stale copy, and later tasks
// of the op on the XCD hit in it.
//
// MT: token rows the LDS region holds (4 for M <= 4, 8, 16, or 32: two
// blocks of 16 tokens, each weight tile decoded once per k-step for both
// blocks' MFMAs).  PF: the next chunk's activation pieces are loaded during
// this step (registers allowing: MT <= 8), so a step stages its pieces in
// LDS and reads its A fragments while its tiles are still in flight.
// R: 16-row groups per task, at most (the host deals blocks of R).
template <int FMT, int MT, bool PF, int R>
__device__ void ss_mblock(const SStackArgs& a, const Rec& r, uint32_t areg, unsigned* known) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    constexpr int LDR = CH + 16;       // LDS bytes per token row of a chunk
    constexpr int PR = CH / 16;        // 16-byte pieces per token row of a chunk
    constexpr int kAP = (MT * PR + 63) / 64;  // pieces per lane for MT token rows
    constexpr int TB = (MT + 15) / 16;        // 16-token MFMA blocks
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int M = a.M, nch = r.nch, opi = r.opi, ldq = r.ldq, N = r.K;
    const int ng = r.ngroups;
    unsigned* const qdone = ss_ctr(a.ctr, kSsDone0 + a.nops + opi);
    // all M tokens quantised before any row load (see above)
    if (!((known[opi >> 5] >> (opi & 31)) & 1u)) {
        if (lane == 0) ss_wait(qdone, (unsigned)M, ss_ctr(a.ctr, kSsError), a.spin_limit);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) atomicOr(&known[opi >> 5], 1u << (opi & 31));
    }
    // Loaded now, used by the epilogue (loaded there, they would stall every
    // task's end on a memory latency with nothing else in flight): lane l <
    // 2M slot l of the op's M row sums and M inverse scales (device-scope
    // loads: those slots share lines that quantiser tasks on other XCDs
    // wrote); lane l the w_scales of rows l and l + 64 of the block.
    const int trows = (ng - 1) * 16 + r.nrows;
    const __amdgpu_buffer_rsrc_t sr = ss_rsrc(r.q + (size_t)M * ldq, (unsigned)(8 * M));
    const int sv = (int)__builtin_amdgcn_raw_buffer_load_b32(sr, lane < 2 * M ? 4u * lane : 0x80000000u, 0, kSsCoh);
    constexpr int WH = (R * 16 + 63) / 64;  // registers for the block's w_scales: lane l, row l + 64 h
    int wv[WH];
#pragma unroll
    for (int h = 0; h < WH; ++h) wv[h] = __float_as_int(((gfloat*)(uintptr_t)r.ws)[min(lane + 64 * h, trows - 1)]);
    // the activation pieces of one chunk: piece p = lane + 64 u is token
    // p / PR, bytes (p % PR) * 16; tokens >= M read nothing (outside the
    // resource) and leave rows of the LDS region the outputs never use
    const __amdgpu_buffer_rsrc_t qr = ss_rsrc(r.q, (unsigned)(M * ldq));
    auto ptok = [&](int u) { return (lane + 64 * u) / PR; };
    auto pcol = [&](int u) { return ((lane + 64 * u) % PR) * 16; };
    // block tb's A fragment: token row 16 tb + j (rows >= MT: the last row
    // again, never stored)
    auto abase = [&](int tb) { return areg + (uint32_t)(min(16 * tb + j, MT - 1) * LDR + g * 16); };
    const uint8_t* const tl = reinterpret_cast<const uint8_t*>(r.tiles) + lane * 16;
    auto load_act = [&](v4i* ap, int c) {  // (chunks past nch read nothing)
#pragma unroll
        for (int u = 0; u < kAP; ++u) {
            const int tk = ptok(u);
            const unsigned go = (tk < M && c < nch) ? (unsigned)(tk * ldq + pcol(u) + c * CH) : 0x80000000u;
            ap[u] = __builtin_amdgcn_raw_buffer_load_b128(qr, go, 0, 0);
        }
    };
    v4i acc[TB][R];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int gi = 0; gi < R; ++gi) acc[tb][gi] = v4i{0, 0, 0, 0};
    v4i ap[kAP];
    if constexpr (PF) load_act(ap, 0);
    for (int c = 0; c < nch; ++c) {
        v4i wb[R], apn[kAP];
#pragma unroll
        for (int gi = 0; gi < R; ++gi)  // (groups past the block: its last group again, unused)
            wb[gi] = ss_ld_tile(tl + ((size_t)min(gi, ng - 1) * nch + c) * kTileBytes);
        if constexpr (PF) load_act(apn, c + 1);
        else load_act(ap, c);
        // (every load of the step is issued before anything waits for one)
        __builtin_amdgcn_sched_barrier(0);
        // (the previous chunk's LDS reads were issued before these writes,
        // and a wave's LDS accesses complete in order)
#pragma unroll
        for (int u = 0; u < kAP; ++u)
            if (64 * (u + 1) <= MT * PR || ptok(u) < MT)  // (the region holds MT rows)
                *reinterpret_cast<__attribute__((address_space(3))) v4i*>(
                    (uintptr_t)(areg + (uint32_t)(ptok(u) * LDR + pcol(u)))) = ap[u];
        v4i af[TB][STEPS];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int st = 0; st < STEPS; ++st) af[tb][st] = ss_lds16(abase(tb) + st * 64);
        // (the LDS stage goes ahead of the weight decode: its wait for the
        // first tile would otherwise come first and hold the stage back)
        __builtin_amdgcn_sched_barrier(0);
        // (all R groups are multiplied: no branch for the compiler to sink
        // loads into; products of groups past the block are never stored)
#pragma unroll
        for (int gi = 0; gi < R; ++gi) {
            if constexpr (FMT == XT_PACK5) {
                int E[4], O[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    E[q] = wb[gi][q] & 0x00ff00ff;
                    O[q] = ((unsigned)wb[gi][q] >> 8) & 0x00ff00ff;
                }
#pragma unroll
                for (int st = 0; st < STEPS; ++st) {
                    v4i b;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int pE = E[q] * 3, pO = O[q] * 3;
                        b[q] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                        E[q] = pE & 0x00ff00ff;
                        O[q] = pO & 0x00ff00ff;
                    }
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) acc[tb][gi] = mfma(af[tb][st], b, acc[tb][gi]);
                }
            } else {
#pragma unroll
                for (int st = 0; st < STEPS; ++st) {
                    const v4i b = decode4(wb[gi][st]);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) acc[tb][gi] = mfma(af[tb][st], b, acc[tb][gi]);
                }
            }
        }
        if constexpr (PF) {
#pragma unroll
            for (int u = 0; u < kAP; ++u) ap[u] = apn[u];
        }
    }
    // this lane's outputs: tokens 16 tb + 4g .. + 3, row j of each group
    float wsc[R];
#pragma unroll
    for (int gi = 0; gi < R; ++gi)  // (rows past trows are never stored)
        wsc[gi] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (min(gi * 16 + j, trows - 1) & 63), wv[(gi * 16) >> 6]));

    // acc[tb][gi][t]: token 16 tb + 4g + t, row j of group gi; the MFMAs took
    // codes w + 1, so the token's sum comes off (layers.rs:340: (dot as f32 *
    // inv) * w_scale)
    const bool pub = (r.flags & kSsPub) != 0;
    const __amdgpu_buffer_rsrc_t yr = ss_rsrc(r.y, (unsigned)(((M - 1) * N + trows) * 4));
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        int rs[4];
        float inv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int tk = min(16 * tb + 4 * g + t, M - 1);
            rs[t] = __builtin_amdgcn_ds_bpermute(4 * tk, sv);
            inv[t] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (tk + M), sv));
        }
#pragma unroll
        for (int gi = 0; gi < R; ++gi) {  // (gi >= ng: groups past the block, predicated)
            const int row = gi * 16 + j;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int tk = 16 * tb + 4 * g + t;
                if (gi < ng && tk < M && row < trows) {
                    const float v = __fmul_rn(__fmul_rn((float)(acc[tb][gi][t] - rs[t]), inv[t]), wsc[gi]);
                    if (pub) ss_st_coh4(yr, (unsigned)((tk * N + row) * 4), __float_as_uint(v));
                    else ((gfloat_w*)(uintptr_t)r.y)[(size_t)tk * N + row] = v;
                }
            }
        }
    }
    if (pub) {  // another op reads these outputs inside the launch
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0)
            __hip_atomic_fetch_add(ss_ctr(a.ctr, kSsDone0 + opi), (unsigned)ng, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// M = 1: a group task that quantises its op's row itself (no quantiser
// tasks, no quantised-row buffer).  It waits only for the op its input comes
// from (if any), takes the row's absmax in one pass over the f32 row (rounds
// of kQ1 pieces per lane in flight), then quantises each chunk's pieces as
// it walks the chunks (the next chunk's f32 pieces load during the current
// step), stages the chunk's i8 bytes in its LDS row and runs the R groups'
// MFMAs on them; the row's exact sum is summed on the way.  Each task reads
// the op's row from L2 twice (25-50 % above its weight bytes), against three
// device-scope hops per dependency when quantiser tasks publish the rows.
// (x is read with ordinary loads: written before the launch, or by the op it
// depends on, whose count this task has seen complete; each 128-byte line of
// that op's output is written by one task only.)
template <int FMT, int MODE, int R>
__device__ void ss_mblock_q1(const SStackArgs& a, const Rec& r, uint32_t areg, unsigned* known) {
    constexpr int STEPS = (FMT == XT_PACK5) ? 5 : 4;
    constexpr int CH = STEPS * 64;
    constexpr int XP = (CH / 4 + 63) / 64;  // f32 pieces (float4) per lane per chunk: 1, or 2 for Pack5
    constexpr int kQ1 = 14;                 // absmax pass: pieces per lane per round
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int nch = r.nch, K = r.K, ng = r.ngroups, dep = r.dep;
    (void)j;
    if (dep >= 0 && !((known[dep >> 5] >> (dep & 31)) & 1u)) {
        if (lane == 0)
            ss_wait(ss_ctr(a.ctr, kSsDone0 + dep), (unsigned)r.dep_groups, ss_ctr(a.ctr, kSsError), a.spin_limit);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) atomicOr(&known[dep >> 5], 1u << (dep & 31));
    }
    const int trows = (ng - 1) * 16 + r.nrows;
    constexpr int WH = (R * 16 + 63) / 64;  // registers for the block's w_scales: lane l, row l + 64 h
    int wv[WH];
#pragma unroll
    for (int h = 0; h < WH; ++h) wv[h] = __float_as_int(((gfloat*)(uintptr_t)r.ws)[min(lane + 64 * h, trows - 1)]);
    const uint8_t* const tl = reinterpret_cast<const uint8_t*>(r.tiles) + lane * 16;
    auto load_tiles = [&](v4i* wb, int c) {
#pragma unroll
        for (int gi = 0; gi < R; ++gi)  // (groups past the block: its last group again, unused)
            wb[gi] = ss_ld_tile(tl + ((size_t)min(gi, ng - 1) * nch + c) * kTileBytes);
    };
    // the first chunk's tiles go out with the absmax pass
    v4i wb[R];
    load_tiles(wb, 0);
    const __amdgpu_buffer_rsrc_t xr = ss_rsrc(r.q, (unsigned)(K * 4));  // (pieces past K: zeros)
    const int n4 = (K + 3) >> 2;
    float mx = 0.0f;
    for (int f0 = 0; f0 < n4; f0 += 64 * kQ1) {
        v4i v[kQ1];
#pragma unroll
        for (int u = 0; u < kQ1; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, (unsigned)(f0 + u * 64 + lane) * 16u, 0, 0);
#pragma unroll
        for (int u = 0; u < kQ1; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(__int_as_float(v[u][e])));
    }
    const float rmx = __int_as_float(wave_reduce_bits(__float_as_int(mx), [](int p, int q) {
        return __float_as_int(fmaxf(__int_as_float(p), __int_as_float(q)));
    }));
    const float scale = (rmx > 0.0f) ? __fdiv_rn(127.0f, rmx) : 1.0f;
    const float invs = (rmx > 0.0f) ? __fdiv_rn(rmx, 127.0f) : 1.0f;
    const int kmain = (K / 16) * 16;
    // chunk c's f32 pieces of this lane: piece lane + 64 u (16 bytes of i8
    // columns 4 (lane + 64 u) .. + 3 of the chunk)
    auto load_x = [&](v4i* xp, int c) {
#pragma unroll
        for (int u = 0; u < XP; ++u) {
            const int pc = lane + 64 * u;
            const bool in = pc < CH / 4 && c < nch;
            xp[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, in ? (unsigned)(c * CH + 4 * pc) * 4u : 0x80000000u, 0, 0);
        }
    };
    v4i xc[XP];
    load_x(xc, 0);
    int rs = 0;
    v4i acc[R];
#pragma unroll
    for (int gi = 0; gi < R; ++gi) acc[gi] = v4i{0, 0, 0, 0};
    for (int c = 0; c < nch; ++c) {
        v4i xn[XP];
        if (c > 0) load_tiles(wb, c);  // (uniform)
        load_x(xn, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        // this chunk's i8 bytes into the LDS row (layers.rs quantisation:
        // quantization.rs:95-195), then the A fragments of row 0
#pragma unroll
        for (int u = 0; u < XP; ++u) {
            const int pc = lane + 64 * u;
            if (64 * (u + 1) <= CH / 4 || pc < CH / 4) {
                unsigned w = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int col = c * CH + 4 * pc + t;
                    w |= (unsigned)(quant_one(__int_as_float(xc[u][t]), scale, MODE, col < kmain) & 255) << (8 * t);
                }
                rs = __builtin_amdgcn_sdot4((int)w, 0x01010101, rs, false);
                *reinterpret_cast<__attribute__((address_space(3))) unsigned*>((uintptr_t)(areg + 4u * pc)) = w;
            }
        }
        v4i af[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) af[st] = ss_lds16(areg + (uint32_t)(g * 16 + st * 64));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gi = 0; gi < R; ++gi) {
            if constexpr (FMT == XT_PACK5) {
                int E[4], O[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    E[q] = wb[gi][q] & 0x00ff00ff;
                    O[q] = ((unsigned)wb[gi][q] >> 8) & 0x00ff00ff;
                }
#pragma unroll
                for (int st = 0; st < STEPS; ++st) {
                    v4i b;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int pE = E[q] * 3, pO = O[q] * 3;
                        b[q] = (int)__builtin_amdgcn_perm((unsigned)pO, (unsigned)pE, 0x07030501u);
                        E[q] = pE & 0x00ff00ff;
                        O[q] = pO & 0x00ff00ff;
                    }
                    acc[gi] = mfma(af[st], b, acc[gi]);
                }
            } else {
#pragma unroll
                for (int st = 0; st < STEPS; ++st) acc[gi] = mfma(af[st], decode4(wb[gi][st]), acc[gi]);
            }
        }
#pragma unroll
        for (int u = 0; u < XP; ++u) xc[u] = xn[u];
    }
    rs = wave_reduce_bits(rs, [](int p, int q) { return p + q; });
    // acc[gi][0] of lanes 0-15: the token, row j of group gi; the MFMAs took
    // codes w + 1, so the row's sum comes off (layers.rs:340)
    const bool pub = (r.flags & kSsPub) != 0;
    const __amdgpu_buffer_rsrc_t yr = ss_rsrc(r.y, (unsigned)(trows * 4));
#pragma unroll
    for (int gi = 0; gi < R; ++gi) {
        // (groups past the block: gi >= ng, uniform; a predicate, not a
        // break, so that the loop unrolls and acc stays in registers)
        const int row = gi * 16 + (lane & 15);
        const int rw = min(row, trows - 1);  // (gi * 16 / 64 is uniform: the register is known)
        const float wsc = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (rw & 63), wv[(gi * 16) >> 6]));
        if (gi < ng && lane < 16 && row < trows) {
            const float v = __fmul_rn(__fmul_rn((float)(acc[gi][0] - rs), invs), wsc);
            if (pub) ss_st_coh4(yr, (unsigned)(row * 4), __float_as_uint(v));
            else ((gfloat_w*)(uintptr_t)r.y)[row] = v;
        }
    }
    if (pub) {  // another op reads these outputs inside the launch
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0)
            __hip_atomic_fetch_add(ss_ctr(a.ctr, kSsDone0 + r.opi), (unsigned)ng, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// MT: the token form (see ss_mblock).  Three waves per SIMD: up to 168
// registers for a task's tiles, activation pieces, A fragments and the four
// groups' accumulators.
template <int MT, int R, int WPE>
__global__ __launch_bounds__(kSsW * 64) __attribute__((amdgpu_waves_per_eu(WPE))) void sstack_kernel(const SStackArgs a) {
    __shared__ unsigned known[kSsKnownWords];  // ops this workgroup has seen quantised
    extern __shared__ __align__(16) uint8_t rows[];  // [kSsW][a.row_bytes]: each wave's i8 row
    for (int i = threadIdx.x; i < kSsKnownWords; i += kSsW * 64) known[i] = 0u;
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int TW = gridDim.x * kSsW;
    const int gw = blockIdx.x * kSsW + wave;
    const uint32_t areg = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(rows + wave * a.row_bytes);
    // each task's record is loaded one task ahead
    const int t0 = a.woff[gw], t1 = a.woff[gw + 1];
    unsigned nxt = 0;
    if (t0 < t1) nxt = ss_rec_load(a.tasks + t0);
    for (int t = t0; t < t1; ++t) {
        const Rec cur = ss_rec(nxt);
        if (t + 1 < t1) nxt = ss_rec_load(a.tasks + t + 1);
        if (cur.flags & kSsQuant) {
            if (a.mode == XT_QUANT_AVX512) ss_quant<XT_QUANT_AVX512>(a, cur);
            else ss_quant<XT_QUANT_SCALAR>(a, cur);
        } else if constexpr (MT == 1) {
            if (cur.flags & kSsPack5) {
                if (a.mode == XT_QUANT_AVX512) ss_mblock_q1<XT_PACK5, XT_QUANT_AVX512, R>(a, cur, areg, known);
                else ss_mblock_q1<XT_PACK5, XT_QUANT_SCALAR, R>(a, cur, areg, known);
            } else {
                if (a.mode == XT_QUANT_AVX512) ss_mblock_q1<XT_PACK4, XT_QUANT_AVX512, R>(a, cur, areg, known);
                else ss_mblock_q1<XT_PACK4, XT_QUANT_SCALAR, R>(a, cur, areg, known);
            }
        } else if (cur.flags & kSsPack5) {
            ss_mblock<XT_PACK5, MT, MT <= 8, R>(a, cur, areg, known);
        } else {
            ss_mblock<XT_PACK4, MT, MT <= 8, R>(a, cur, areg, known);
        }
    }
    // the last wave out resets the counts for the next launch (its own
    // bumps, like everyone's, were performed before its exit is counted)
    __builtin_amdgcn_s_waitcnt(0);
    unsigned old = 0;
    if ((threadIdx.x & 63) == 0)
        old = __hip_atomic_fetch_add(ss_ctr(a.ctr, kSsExit), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == (unsigned)TW - 1) {
        for (int i = threadIdx.x & 63; i < 2 * a.nops; i += 64) ss_st_coh(ss_ctr(a.ctr, kSsDone0 + i), 0u);
        if ((threadIdx.x & 63) == 0) ss_st_coh(ss_ctr(a.ctr, kSsExit), 0u);
    }
}

}  // namespace

// LDS beyond the static part: every wave's region for one chunk of the
// form's token rows.
static size_t ss_dyn_lds(int row_bytes) { return (size_t)kSsW * row_bytes; }

// Token forms: rows of the LDS region, groups per task, waves per SIMD.
// M = 1: eight groups per task at two waves per SIMD (183 registers) ran the
// C4 list in 108.5 us against 114 us with four at three (and six at three:
// 117 us); more bytes per step per wave beat more waves here.  M = 2 .. 4
// likewise (121 independent C0 ops at M = 4: 120 against 125.6 us); an
// 8-token form with eight groups and the next chunk's pieces in flight took
// the M = 8 C4 list from 152 to 146 us.  The 16-token form: eight groups at
// two waves per SIMD 171.7 us on the C4 list at M = 16 against 175.5 with
// four at three (six at two: 197.8; eight with the next chunk's pieces in
// flight: 174.2).  The 32-token form (two 16-token MFMA blocks per tile):
// six groups 255 us on the C4 list against 293 with four and 275 with seven
// (eight spill registers).  Ten or twelve groups at two waves per SIMD
// (204-253 registers): M = 1 / 8 C4 lists 127 / 168 and 136 / 159 us
// against 112-114 / 145 with eight.
constexpr int kSsF4R = 8, kSsF4W = 2;
constexpr int kSsF1R = 8, kSsF1W = 2;
constexpr int kSsF8R = 8, kSsF8W = 2;
constexpr int kSsF16R = 8, kSsF16W = 2;
constexpr int kSsF32R = 6, kSsF32W = 2;
// Base-3 forms (Pack5 tiles are most of the stack's bytes), M <= 16.  A
// Pack5 tile's decode is five multiply-mask-permute rounds per dword and
// k-step against Pack4's one permute, so the VALU work per tile is several
// times Pack4's and more waves hide it better than more groups per wave:
// four groups at three waves per SIMD ran the 26-layer BitNet-3B Pack5 stack
// in 194 / 194 / 199 us at M = 1 / 4 / 8 against 247 / 230 / 254 us with the
// Pack4 forms (two groups at four waves: 218 / 225 / 226 us; three groups at
// four waves for M = 1 and three at three above: 203 / 211 / 216 us; five
// at three: 192 / 203 / 228 us; six at three: 249 / 227 / 230 us).
constexpr int kSsP5R = 4, kSsP5W = 3;
// (Pack5 at M = 32 keeps four groups: 408 us on that stack against 478 with
// six)
constexpr int kSsP32R = 4;
int sstack_lds_rows(int M) { return M == 1 ? 1 : (M <= 4 ? 4 : (M <= 8 ? 8 : (M <= 16 ? 16 : 32))); }
int sstack_groups_per_task(int M, bool p5) {
    if (p5) return M <= 16 ? kSsP5R : kSsP32R;
    return M == 1 ? kSsF1R : (M <= 4 ? kSsF4R : (M <= 8 ? kSsF8R : (M <= 16 ? kSsF16R : kSsF32R)));
}
bool sstack_quant_tasks(int M) { return M > 1; }

static const void* ss_fn(int M, bool p5) {
    if (p5 && M == 1) return reinterpret_cast<const void*>(sstack_kernel<1, kSsP5R, kSsP5W>);
    if (p5 && M <= 4) return reinterpret_cast<const void*>(sstack_kernel<4, kSsP5R, kSsP5W>);
    if (p5 && M <= 8) return reinterpret_cast<const void*>(sstack_kernel<8, kSsP5R, kSsP5W>);
    if (p5 && M <= 16) return reinterpret_cast<const void*>(sstack_kernel<16, kSsP5R, kSsP5W>);
    if (p5) return reinterpret_cast<const void*>(sstack_kernel<32, kSsP32R, kSsF32W>);
    if (M == 1) return reinterpret_cast<const void*>(sstack_kernel<1, kSsF1R, kSsF1W>);
    if (M <= 4) return reinterpret_cast<const void*>(sstack_kernel<4, kSsF4R, kSsF4W>);
    if (M <= 8) return reinterpret_cast<const void*>(sstack_kernel<8, kSsF8R, kSsF8W>);
    if (M <= 16) return reinterpret_cast<const void*>(sstack_kernel<16, kSsF16R, kSsF16W>);
    return reinterpret_cast<const void*>(sstack_kernel<32, kSsF32R, kSsF32W>);
}

hipError_t launch_sstack(const SStackArgs& a, int blocks, hipStream_t s) {
    if (a.M < 1 || a.M > kSStackMaxM) return hipErrorInvalidValue;
    void* args[] = {const_cast<SStackArgs*>(&a)};
    return hipLaunchKernel(ss_fn(a.M, a.pack5 != 0), dim3(blocks), dim3(kSsW * 64), args, ss_dyn_lds(a.row_bytes), s);
}

hipError_t sstack_blocks_per_cu(int M, bool p5, int row_bytes, int* n) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, ss_fn(M, p5), kSsW * 64, ss_dyn_lds(row_bytes));
}

int sstack_waves_per_block() { return kSsW; }

}  // namespace xt
