// device_common.h -- dtype access and epilogue math shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace vai_dev {

// Calls f(std::integral_constant<int, I>{}) for I = 0..N-1, fully unrolled at
// compile time (register arrays indexed by I stay registers).
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
        (f(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, N>{});
}

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float8v __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

enum : int { DT_F32 = 0, DT_F16 = 1 };

__device__ __forceinline__ float ld(const void* p, int dt, size_t i)
{
    return dt == DT_F16 ? (float)((const half_t*)p)[i] : ((const float*)p)[i];
}
__device__ __forceinline__ void st(void* p, int dt, size_t i, float v)
{
    if (dt == DT_F16) ((half_t*)p)[i] = (half_t)v;   // round-to-nearest-even
    else ((float*)p)[i] = v;
}

// Epilogues of vai::Epilogue, as the reference's activation.h states them
// (/root/reference/vai/shaders/common/activation.h:19-58): GELU (erf) through
// Abramowitz-Stegun 7.1.26, GELU-tanh, SiLU, sigmoid. exp and reciprocal use
// the hardware v_exp_f32 / v_rcp_f32 (about 1 ulp each): the reference's own
// tier for these is 1e-4 relative, and IEEE exp + division made the GEMM
// epilogue VALU-bound. tanh(y) = 1 - 2 / (e^{2y} + 1) saturates to +-1 for
// large |y| (e^{2y} = inf gives 1 - 0) and keeps an absolute error of a few
// ulp of 1 near 0.
// A pointer every lane holds the same value of, moved to scalar registers:
// a buffer resource built from it then stays scalar (a resource the compiler
// cannot prove uniform is used through a readfirstlane loop around every
// load).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p)
{
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float erf_as(float x)
{
    const float t = fast_rcp(1.0f + 0.3275911f * fabsf(x));
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t
                     + 0.254829592f) * t;
    const float s = x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f);
    return s * (1.0f - p * fast_exp(-x * x));
}

__device__ __forceinline__ float fast_tanh(float y)
{
    return 1.0f - 2.0f * fast_rcp(fast_exp(2.0f * y) + 1.0f);
}

__device__ __forceinline__ float epilogue(float x, uint32_t epi)
{
    switch (epi) {
    case 1: return x > 0.f ? x : 0.f;
    case 2: return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
    case 3: return 0.5f * x * (1.0f + fast_tanh(0.79788456080286535f * (x + 0.044715f * x * x * x)));
    case 4: return x * fast_rcp(1.0f + fast_exp(-x));
    case 5: return fast_rcp(1.0f + fast_exp(-x));
    default: return x;
    }
}

// s * epi(acc + r) (before) or s * epi(acc) + r (after): linear-slab.comp:236-242.
__device__ __forceinline__ float finish(float acc, float r, uint32_t epi, uint32_t order, float s)
{
    return order == 1 ? s * epilogue(acc + r, epi) : s * epilogue(acc, epi) + r;
}

// One Linear output O[o] = s * epi(v + B) (+R), the bias and residual read
// with their repeats. A plain Linear (no bias, residual or epilogue, scale 1,
// fp32 output) branches straight to its store: in a GEMV every wave reaches
// its epilogue at about the same moment at the end, and running through the
// general code (repeat divisions, dtype and epilogue switches) cost about
// 0.15 us per launch.
struct OutputSpec {
    void* out;
    const void* bias;
    const void* residual;
    int o_dtype, b_dtype;
    uint32_t bias_repeat, residual_repeat, epilogue, residual_order;
    float scale;
};

__device__ __forceinline__ void store_output_general(const OutputSpec& q, size_t o, float v)
{
    const float b = q.bias ? ld(q.bias, q.b_dtype, q.bias_repeat ? o % q.bias_repeat : o) : 0.f;
    const float r = q.residual ? ld(q.residual, q.o_dtype, q.residual_repeat ? o % q.residual_repeat : o) : 0.f;
    st(q.out, q.o_dtype, o, finish(v + b, r, q.epilogue, q.residual_order, q.scale));
}

__device__ __forceinline__ void store_output(const OutputSpec& q, size_t o, float v)
{
    if (!q.bias && !q.residual && q.epilogue == 0 && q.scale == 1.0f && q.o_dtype == DT_F32) {
        ((float*)q.out)[o] = v;
        return;
    }
    store_output_general(q, o, v);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// One butterfly exchange across lane bit O (16 or 32) in a single VALU
// instruction, no LDS: v_permlane{16,32}_swap exchanges the O-lane halves
// with bit O set in `a` with those with bit O clear in `b`, so afterwards the
// two registers hold, per lane, the pair (lane, lane ^ O) of a (lanes with
// bit O clear) or of b (lanes with bit O set); their sum is
//   a[l] + a[l ^ O] where bit O of l is clear, b[l] + b[l ^ O] where it is set.
//
// Written as inline asm: the compiler's builtins for these instructions
// return the first register twice here (the second result is lost). The
// s_nops give the VALU writes before and the reads after the wait states the
// compiler cannot insert around an asm block.
template <int O>
__device__ __forceinline__ void lane_swap(float& a, float& b)
{
    static_assert(O == 16 || O == 32, "row or half-wave exchange");
    if constexpr (O == 16)
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    else
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

template <int O>
__device__ __forceinline__ float swap_sum(float a, float b)
{
    lane_swap<O>(a, b);
    return a + b;
}

// max(x[l], x[l ^ 32]) in every lane, by the same swap.
__device__ __forceinline__ float swap_max32(float x)
{
    float y = x;
    lane_swap<32>(x, y);
    return fmaxf(x, y);
}

}   // namespace vai_dev
