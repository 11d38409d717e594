// Measurement kernels for bench.py --peaks (libxtern_diag.so, not part of the
// product ABI): the ceilings the product kernels are judged against, measured
// on the box rather than taken from the data sheet.
//   xtd_read        streaming read of a buffer (16-byte nontemporal loads,
//                   eight in flight per lane), one XOR per workgroup written
//   xtd_mfma_i8     back-to-back v_mfma_i32_32x32x32_i8 (or 16x16x64) on four
//                   independent accumulators per wave, no memory traffic
//   xtd_empty       an empty kernel of a given grid (launch floor)
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kReadThreads = 512;
constexpr int kReadUnroll = 8;

__global__ __launch_bounds__(kReadThreads) void read_kernel(const v4i* __restrict__ p, size_t n16,
                                                             unsigned* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * kReadThreads;
    size_t i = (size_t)blockIdx.x * kReadThreads + threadIdx.x;
    v4i acc = {0, 0, 0, 0};
    for (; i + (kReadUnroll - 1) * stride < n16; i += kReadUnroll * stride) {
        v4i v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
    unsigned x = (unsigned)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]);
    // one store per workgroup keeps the loads live
    __shared__ unsigned red[kReadThreads / 64];
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned r = 0;
        for (int w = 0; w < kReadThreads / 64; ++w) r ^= red[w];
        sink[blockIdx.x] = r;
    }
}

template <int SHAPE>
__global__ __launch_bounds__(256) void mfma_kernel(int iters, int seed, int* __restrict__ sink) {
    // operands from the seed so the compiler cannot fold the chain
    const int a0 = seed * 0x01010101 + threadIdx.x;
    if constexpr (SHAPE == 32) {
        v4i a = {a0, a0 ^ 0x5a5a5a5a, a0 * 3, a0 + 7};
        v4i b = {a0 + 1, a0 * 5, a0 ^ 0x33, a0 - 9};
        v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
        }
        int s = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) s += c0[k] ^ c1[k] ^ c2[k] ^ c3[k];
        if (s == 0x12345678) sink[blockIdx.x] = s;
    } else {
        v4i a = {a0, a0 ^ 0x5a5a5a5a, a0 * 3, a0 + 7};
        v4i b = {a0 + 1, a0 * 5, a0 ^ 0x33, a0 - 9};
        v4i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c3, 0, 0, 0);
        }
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) s += c0[k] ^ c1[k] ^ c2[k] ^ c3[k];
        if (s == 0x12345678) sink[blockIdx.x] = s;
    }
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// Streaming read of `bytes` (a multiple of 16) at `p` over `blocks`
// workgroups of 512 threads; sink holds `blocks` unsigned.
int xtd_read(const void* p, size_t bytes, int blocks, unsigned* sink, void* stream) {
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(kReadThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const v4i*>(p), bytes / 16,
                       sink);
    return (int)hipGetLastError();
}

// `blocks` workgroups of 4 waves, each wave issuing 4 * iters MFMAs.
// shape 32: v_mfma_i32_32x32x32_i8 (65536 ops each), 16: 16x16x64 (32768).
int xtd_mfma_i8(int shape, int blocks, int iters, int* sink, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (shape == 32)
        hipLaunchKernelGGL(mfma_kernel<32>, dim3(blocks), dim3(256), 0, s, iters, 1, sink);
    else
        hipLaunchKernelGGL(mfma_kernel<16>, dim3(blocks), dim3(256), 0, s, iters, 1, sink);
    return (int)hipGetLastError();
}

int xtd_empty(int blocks, int threads, void* stream) {
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(threads), 0,
                       static_cast<hipStream_t>(stream));
    return (int)hipGetLastError();
}

}  // extern "C"
