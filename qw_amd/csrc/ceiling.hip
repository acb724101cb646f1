// ceiling.hip - the box's memory ceilings, measured the way the decode path
// uses memory (libqwceil.so, loaded by bench.py only; not part of the C ABI
// in include/qwattn.h).
//
//   qwc_read: every byte of a buffer read once with 128-bit loads and folded
//             into a per-thread XOR (the result is stored only when it equals
//             a value the caller never passes, so the loads cannot be dropped
//             and nothing is written in practice). Workgroup b of `blocks`
//             reads 4 KB pieces b, b + blocks, ... with `unroll` pieces in
//             flight a wave: the decode kernel's interleaved deal.
//   qwc_copy: dst = src, 128-bit loads and stores, grid-stride.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ __launch_bounds__(512) void read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                   uint32_t never, uint32_t* __restrict__ sink) {
    // a wave reads 1 KB runs (64 lanes x 16 B); the workgroup's waves cover
    // consecutive runs
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int64_t runs = n16 / 64;
    const int64_t stride = (int64_t)gridDim.x * nw;
    uint32_t x = 0;
    int64_t r = (int64_t)blockIdx.x * nw + wave;
    for (; r + (UNROLL - 1) * stride < runs; r += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v[u] = src[(r + u * stride) * 64 + lane];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; r < runs; r += stride) {
        const u32x4 v = src[r * 64 + lane];
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (x == never) sink[blockIdx.x * blockDim.x + threadIdx.x] = x;
}

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

}  // namespace

extern "C" {

// bytes: a multiple of 1024; blocks: workgroups (512 threads each);
// unroll: 1, 2, 4 or 8 runs in flight a wave. Returns 0 or a hipError_t.
int qwc_read(const void* buf, int64_t bytes, uint32_t* sink, int blocks, int unroll,
             hipStream_t stream) {
    if (!buf || !sink || bytes <= 0 || bytes % 1024 != 0 || blocks <= 0) return (int)hipErrorInvalidValue;
    const int64_t n16 = bytes / 16;
    const uint32_t never = 0x9E3779B9u;
    switch (unroll) {
        case 1: hipLaunchKernelGGL(read_kernel<1>, dim3(blocks), dim3(512), 0, stream, (const u32x4*)buf, n16, never, sink); break;
        case 2: hipLaunchKernelGGL(read_kernel<2>, dim3(blocks), dim3(512), 0, stream, (const u32x4*)buf, n16, never, sink); break;
        case 4: hipLaunchKernelGGL(read_kernel<4>, dim3(blocks), dim3(512), 0, stream, (const u32x4*)buf, n16, never, sink); break;
        case 8: hipLaunchKernelGGL(read_kernel<8>, dim3(blocks), dim3(512), 0, stream, (const u32x4*)buf, n16, never, sink); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// bytes: a multiple of 16.
int qwc_copy(void* dst, const void* src, int64_t bytes, int blocks, hipStream_t stream) {
    if (!dst || !src || bytes <= 0 || bytes % 16 != 0 || blocks <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, stream, (const u32x4*)src, (u32x4*)dst,
                       bytes / 16);
    return (int)hipGetLastError();
}

}  // extern "C"
