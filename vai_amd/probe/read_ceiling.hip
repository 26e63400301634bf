// read_ceiling.hip -- measurement kernel, not part of the product library: a
// plain streaming read of `bytes` (16-byte non-temporal loads, every load of a
// lane issued before any is used), the ceiling an HBM-bound kernel of the same
// size can reach on this GPU. bench.py times it like the GEMV (rotating
// buffers, one launch per step inside a HIP graph).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef float float4v __attribute__((ext_vector_type(4)));

// Wave w of the grid reads LOADS * 1 KB chunks starting at chunk w * LOADS,
// then strides by the grid's wave count (a single pass when the grid covers
// the buffer).
template <int LOADS>
__global__ void read_kernel(const float4v* __restrict__ src, size_t chunks, float* sink)
{
    const int lane = threadIdx.x & 63;
    const size_t waves = (size_t)gridDim.x * (blockDim.x >> 6);
    float s = 0.f;
    for (size_t w = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); w * LOADS < chunks; w += waves) {
        const float4v* p = src + w * LOADS * 64 + lane;
        float4v v[LOADS];
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            v[i] = (w * LOADS + i < chunks) ? __builtin_nontemporal_load(p + i * 64) : (float4v)0.f;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
    }
    if (s == 1234.5f) sink[0] = s;   // keeps the loads; never true for the zero-filled buffers used
}

extern "C" int vai_probe_read(const void* src, size_t bytes, int grid, int threads, int loads, float* sink,
                              hipStream_t stream)
{
    if (bytes % 1024 || (threads != 256 && threads != 512 && threads != 1024) || grid <= 0) return 1;
    const size_t chunks = bytes / 1024;
    const float4v* p = (const float4v*)src;
    switch (loads) {
    case 4: hipLaunchKernelGGL(read_kernel<4>, dim3(grid), dim3(threads), 0, stream, p, chunks, sink); break;
    case 8: hipLaunchKernelGGL(read_kernel<8>, dim3(grid), dim3(threads), 0, stream, p, chunks, sink); break;
    case 16: hipLaunchKernelGGL(read_kernel<16>, dim3(grid), dim3(threads), 0, stream, p, chunks, sink); break;
    case 32: hipLaunchKernelGGL(read_kernel<32>, dim3(grid), dim3(threads), 0, stream, p, chunks, sink); break;
    default: return 1;
    }
    return (int)hipGetLastError();
}

// The write counterpart: wave w stores STORES * 1 KB chunks from chunk
// w * STORES with 16-byte non-temporal stores (the form the scores kernel's
// hidden tiles use), the ceiling for a kernel bound by writing its output.
template <int STORES>
__global__ void write_kernel(float4v* __restrict__ dst, size_t chunks)
{
    const int lane = threadIdx.x & 63;
    const size_t waves = (size_t)gridDim.x * (blockDim.x >> 6);
    const float4v v = (float4v)(-1.f);
    for (size_t w = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); w * STORES < chunks; w += waves) {
        float4v* p = dst + w * STORES * 64 + lane;
#pragma unroll
        for (int i = 0; i < STORES; ++i)
            if (w * STORES + i < chunks) __builtin_nontemporal_store(v, p + i * 64);
    }
}

extern "C" int vai_probe_write(void* dst, size_t bytes, int grid, int threads, int stores, hipStream_t stream)
{
    if (bytes % 1024 || (threads != 256 && threads != 512 && threads != 1024) || grid <= 0) return 1;
    const size_t chunks = bytes / 1024;
    float4v* p = (float4v*)dst;
    switch (stores) {
    case 4: hipLaunchKernelGGL(write_kernel<4>, dim3(grid), dim3(threads), 0, stream, p, chunks); break;
    case 8: hipLaunchKernelGGL(write_kernel<8>, dim3(grid), dim3(threads), 0, stream, p, chunks); break;
    case 16: hipLaunchKernelGGL(write_kernel<16>, dim3(grid), dim3(threads), 0, stream, p, chunks); break;
    default: return 1;
    }
    return (int)hipGetLastError();
}

__global__ void empty_kernel(float* sink)
{
    if (threadIdx.x == 1023) sink[0] = 0.f;
}

// An empty kernel: the fixed cost of one launch of `grid` workgroups in a graph.
extern "C" int vai_probe_empty(int grid, int threads, float* sink, hipStream_t stream)
{
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(threads), 0, stream, sink);
    return (int)hipGetLastError();
}
