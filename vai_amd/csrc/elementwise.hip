// elementwise.hip -- the memory-bound passes around the GEMM: the split-K fold
// with the Linear epilogue (/root/reference/vai/shaders/linear-reduce.comp) and
// GatedMul (/root/reference/vai/shaders/gated-mul.comp).
#include "device_common.h"
#include "kernels.h"

namespace vai_dev {

// O = s*epi(sum_z P[z] + B) (+R); P fp32 [splits, M, N]. With gated_H > 0 the
// partials are [splits, M, 2H] and O[m,j] = gate_epi(g + bg) * (u + bu).
__global__ __launch_bounds__(256) void linear_reduce_kernel(
    void* out, int o_dt, const float* __restrict__ P, uint32_t splits, size_t MN,
    const void* bias, int b_dt, uint32_t bias_rep, const void* res, uint32_t res_rep,
    uint32_t epi, uint32_t order, float s, uint32_t H, uint32_t gate_epi, uint32_t N)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (H == 0) {
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += stride) {
            float acc = bias ? ld(bias, b_dt, bias_rep ? i % bias_rep : i) : 0.f;
            for (uint32_t z = 0; z < splits; ++z) acc += P[(size_t)z * MN + i];
            const float r = res ? ld(res, o_dt, res_rep ? i % res_rep : i) : 0.f;
            st(out, o_dt, i, finish(acc, r, epi, order, s));
        }
    } else {
        // MN counts outputs [M, H]; partial rows are 2H wide.
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += stride) {
            const size_t m = i / H, j = i % H;
            const size_t PW = (size_t)(MN / H) * 2 * H;
            float g = bias ? ld(bias, b_dt, j) : 0.f, u = bias ? ld(bias, b_dt, H + j) : 0.f;
            for (uint32_t z = 0; z < splits; ++z) {
                g += P[z * PW + m * 2 * H + j];
                u += P[z * PW + m * 2 * H + H + j];
            }
            st(out, o_dt, i, epilogue(g, gate_epi) * u);
        }
    }
}

// Four consecutive outputs per thread (MN, bias and residual repeats
// multiples of 4, 16-byte aligned partials): 16-byte partial loads and one
// 8- or 16-byte store, the repeat offsets computed once per four outputs.
__global__ __launch_bounds__(256) void linear_reduce4_kernel(
    void* out, int o_dt, const float* __restrict__ P, uint32_t splits, size_t MN,
    const void* bias, int b_dt, uint32_t bias_rep, const void* res, uint32_t res_rep,
    uint32_t epi, uint32_t order, float s)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x * 4;
    for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < MN; i += stride) {
        // the bias first, then the planes in split order (linear-reduce.comp:90-93)
        const size_t bi = bias_rep ? i % bias_rep : i, ri = res_rep ? i % res_rep : i;
        float4v acc = (float4v)0.f;
        if (bias)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = ld(bias, b_dt, bi + k);
        for (uint32_t z = 0; z < splits; ++z) acc += *(const float4v*)(P + (size_t)z * MN + i);
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float r = res ? ld(res, o_dt, ri + k) : 0.f;
            v[k] = finish(acc[k], r, epi, order, s);
        }
        if (o_dt == DT_F16) {
            typedef half_t half4t __attribute__((ext_vector_type(4)));
            const half4t h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
            *(half4t*)((half_t*)out + i) = h;
        } else {
            *(float4v*)((float*)out + i) = float4v{v[0], v[1], v[2], v[3]};
        }
    }
}

hipError_t linear_reduce_launch(void* out, int o_dtype, const float* partials, uint32_t splits, size_t MN,
                                const void* bias, int b_dtype, uint32_t bias_repeat,
                                const void* residual, uint32_t residual_repeat,
                                uint32_t epi, uint32_t order, float s, uint32_t gated_H, uint32_t gate_epi,
                                uint32_t N, hipStream_t st)
{
    const bool vec4 = gated_H == 0 && MN % 4 == 0 && bias_repeat % 4 == 0 && residual_repeat % 4 == 0 &&
                      ((uintptr_t)partials % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                      ((uintptr_t)bias % 16) == 0 && ((uintptr_t)residual % 16) == 0;
    if (vec4) {
        const size_t want = (MN / 4 + 255) / 256;
        const uint32_t blocks = (uint32_t)(want < 65536 ? (want ? want : 1) : 65536);
        hipLaunchKernelGGL(linear_reduce4_kernel, dim3(blocks), dim3(256), 0, st, out, o_dtype, partials, splits, MN,
                           bias, b_dtype, bias_repeat, residual, residual_repeat, epi, order, s);
        return hipGetLastError();
    }
    const size_t want = (MN + 255) / 256;
    const uint32_t blocks = (uint32_t)(want < 65536 ? (want ? want : 1) : 65536);
    hipLaunchKernelGGL(linear_reduce_kernel, dim3(blocks), dim3(256), 0, st, out, o_dtype, partials, splits, MN,
                       bias, b_dtype, bias_repeat, residual, residual_repeat, epi, order, s, gated_H, gate_epi, N);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void gated_mul_kernel(void* out, int o_dt, const void* in, int i_dt,
                                                        size_t total, uint32_t H, uint32_t epi)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const size_t row = e / H, src = row * 2 * H + (e - row * H);
        st(out, o_dt, e, epilogue(ld(in, i_dt, src), epi) * ld(in, i_dt, src + H));
    }
}

hipError_t gated_mul_launch(void* out, int o_dtype, const void* in, int i_dtype, uint32_t rows, uint32_t H,
                            uint32_t epi, hipStream_t s)
{
    const size_t total = (size_t)rows * H;
    const size_t want = (total + 255) / 256;
    const uint32_t blocks = (uint32_t)(want < 65536 ? (want ? want : 1) : 65536);
    hipLaunchKernelGGL(gated_mul_kernel, dim3(blocks), dim3(256), 0, s, out, o_dtype, in, i_dtype, total, H, epi);
    return hipGetLastError();
}

}   // namespace vai_dev
