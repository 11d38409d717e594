// Device helpers shared by the xtern kernels (xtern_kernels.hip,
// xtern_sstack.hip, xtern_gstream.hip, xtern_xs.hip): the quantiser's per-element rounding, DPP wave reductions,
// load flavours, the Pack4 decode and the i8 MFMA.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xtern.h"

namespace xt {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Activation quantiser
// ---------------------------------------------------------------------------

// One element of quantize_f32_to_i8.  `main_lane` selects, in AVX-512 mode,
// the vector body (quantization.rs:128-136: min/max clamp in MINPS/MAXPS
// operand order, then CVTPS2DQ round-half-even, NaN -> 0) versus the scalar
// tail (:138-142: round half away from zero, clamp, `as i8`).  Scalar mode is
// :189-192 (round half away; Rust max/min send NaN to -127).
__device__ __forceinline__ int quant_one(float x, float scale, int mode, bool main_lane) {
    const float s = __fmul_rn(x, scale);
    if (mode == XT_QUANT_AVX512) {
        if (main_lane) {
            float t = (127.0f < s) ? 127.0f : s;
            t = (-127.0f > t) ? -127.0f : t;
            return (t != t) ? 0 : (int)__builtin_rintf(t);
        }
        const float r = roundf(s);
        const float c = (r > 127.0f) ? 127.0f : ((r < -127.0f) ? -127.0f : r);
        return (c != c) ? 0 : (int)c;
    }
    float r = roundf(s);
    if (r != r) return -127;
    r = (r < -127.0f) ? -127.0f : r;
    r = (r > 127.0f) ? 127.0f : r;
    return (int)r;
}

// Wave reductions over DPP (gfx9 row_shr within rows of 16, then
// row_bcast:15 / row_bcast:31 into the following rows; lane 63 ends with the
// full result, which readlane broadcasts).  Lanes without a source read the
// identity (`old` = 0: the sum identity, and the max identity for the
// non-negative values the quantisers reduce).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_id(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}
template <typename Op>
__device__ __forceinline__ int wave_reduce_bits(int v, Op op) {
    v = op(v, dpp_id<0x111, 0xf>(v));
    v = op(v, dpp_id<0x112, 0xf>(v));
    v = op(v, dpp_id<0x114, 0xf>(v));
    v = op(v, dpp_id<0x118, 0xf>(v));
    v = op(v, dpp_id<0x142, 0xa>(v));
    v = op(v, dpp_id<0x143, 0xc>(v));
    return __builtin_amdgcn_readlane(v, 63);
}

struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OrOp {
    __device__ int operator()(int a, int b) const { return a | b; }
};
struct AddOp {
    __device__ int operator()(int a, int b) const { return a + b; }
};

// Workgroup reduction: DPP inside each wave, then the per-wave values
// through LDS.  MaxOp is only used on non-negative values (absmax).
// NW: waves of the workgroup when known at compile time (0: from blockDim,
// an extra kernel-argument load).
template <int NW = 0, typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T* smem) {
    int bits;
    if constexpr (sizeof(T) == 4 && __is_same(T, float)) {
        bits = wave_reduce_bits(__float_as_int(v), [op](int x, int y) {
            return __float_as_int(op(__int_as_float(x), __int_as_float(y)));
        });
        v = __int_as_float(bits);
    } else {
        v = (T)wave_reduce_bits((int)v, [op](int x, int y) { return (int)op((T)x, (T)y); });
    }
    const int wave = threadIdx.x >> 6, nw = NW > 0 ? NW : (int)(blockDim.x >> 6);
    if ((threadIdx.x & 63) == 0) smem[wave] = v;
    __syncthreads();
    T r = smem[0];
    for (int w = 1; w < nw; ++w) r = op(r, smem[w]);
    __syncthreads();
    return r;
}


__device__ __forceinline__ v4i ld_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}
__device__ __forceinline__ v4i ld_cached(const int8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

// Workgroups are dispatched to the 8 XCDs round-robin in linear order, and
// each XCD has its own L2.  xcd_remap turns the linear workgroup id into a
// logical tile id so that every XCD owns a contiguous range of logical tiles
// (a bijection on [0, total)); callers order logical tiles so that tiles that
// share weights are adjacent and hence share an L2.
__device__ __forceinline__ int xcd_remap(int lin, int total) {
    const int q = total >> 3, r = total & 7;
    const int xcd = lin & 7, slot = lin >> 3;
    // branch-free: xcd * q + min(xcd, r) == the first tile of XCD xcd
    return xcd * q + min(xcd, r) + slot;
}

// Pack4 tile dword -> four code dwords (columns 4jj..4jj+3 in byte order).
__device__ __forceinline__ v4i decode4(int x) {
    v4i b;
    b[0] = x & 0x03030303;
    b[1] = (x >> 2) & 0x03030303;
    b[2] = (x >> 4) & 0x03030303;
    b[3] = (x >> 6) & 0x03030303;
    return b;
}

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int signed_codes(int c) {
    // byte i of the result = byte c_i of 0x000100ff: codes 0..3 -> -1, 0, +1, 0
    return (int)__builtin_amdgcn_perm(0u, 0x000100ffu, (unsigned)c);
}

}  // namespace xt
