// gemm_acc16.hip -- Linear with an fp16 accumulator (Linear::setAccDtype(Fp16)).
//
// The reference's scalar tile kernel with accType fp16
// (/root/reference/vai/shaders/linear-tile.comp:55,71,292-320) keeps its sums
// in float16 and walks each split's K span in 4-wide steps from the span's
// start, each step one nested fma chain
//     sum = fma(a[k], b[k], fma(a[k+1], b[k+1], fma(a[k+2], b[k+2], fma(a[k+3], b[k+3], sum))))
// i.e. k+3 first, every fma rounded to fp16 (elements past the span's end
// are zero). The sums are clamped to +-65504 and then finished in fp32 like
// any partial (bias, epilogue, residual, scale; split planes via the reduce).
// That order depends on nothing but the split span, so this kernel repeats it
// exactly: every output is bit-identical to the same chain on the CPU.
//
// gfx950's matrix cores only accumulate in fp32, so this path uses v_fma_f16
// on the vector ALUs: a 64x64 output tile per workgroup, operands staged as
// fp16 in LDS 32 k at a time (fp32 operands are rounded to fp16 first, the
// tile contract), each thread holding 4x4 outputs (x2 when gated: the gate
// and up sums of one output column).
#include "device_common.h"
#include "kernels.h"

namespace vai_dev {
namespace {

constexpr int TM = 64, TN = 64, TK = 32, LDK = TK + 2;   // +2 halves: rows land on different banks

template <bool GATED>
__global__ __launch_bounds__(256) void gemm_acc16_kernel(GemmParams p)
{
    constexpr int G = GATED ? 2 : 1;
    __shared__ half_t As[TM][LDK];
    __shared__ half_t Bs[G][TN][LDK];
    const uint32_t ncols = GATED ? p.H : p.N;
    const uint32_t m0 = blockIdx.y * TM, n0 = blockIdx.x * TN, split = blockIdx.z;
    const uint32_t kbeg = split * p.split_size;
    const uint32_t kend = min(p.K, kbeg + p.split_size);
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;   // outputs (ty + 16i, tx + 16j)

    half_t acc[G][4][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[g][i][j] = (half_t)0.f;

    for (uint32_t kb = kbeg; kb < kend; kb += TK) {
        // stage: 64 rows x 32 k per operand, 8 elements per thread
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int idx = threadIdx.x * 8 + e, r = idx / TK, c = idx % TK;
            const uint32_t k = kb + c;
            const uint32_t ra = m0 + r, rb = n0 + r;
            As[r][c] = (ra < p.M && k < kend) ? (half_t)ld(p.A, p.a_dtype, (size_t)ra * p.K + k) : (half_t)0.f;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t wrow = rb + (g ? p.H : 0u);
                Bs[g][r][c] = (rb < ncols && k < kend) ? (half_t)ld(p.B, p.b_dtype, (size_t)wrow * p.K + k)
                                                       : (half_t)0.f;
            }
        }
        __syncthreads();
#pragma unroll 2
        for (int c = 0; c < TK; c += 4) {
            half_t a[4][4], b[G][4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) a[i][q] = As[ty + 16 * i][c + q];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) b[g][j][q] = Bs[g][tx + 16 * j][c + q];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        half_t s = acc[g][i][j];
                        s = __builtin_fmaf16(a[i][3], b[g][j][3], s);
                        s = __builtin_fmaf16(a[i][2], b[g][j][2], s);
                        s = __builtin_fmaf16(a[i][1], b[g][j][1], s);
                        s = __builtin_fmaf16(a[i][0], b[g][j][0], s);
                        acc[g][i][j] = s;
                    }
        }
        __syncthreads();
    }

    // clamp to +-65504 (linear-tile.comp:317-321); a NaN sum stays NaN (GLSL
    // leaves clamp of a NaN undefined: keeping it makes the fault visible)
    const float lim = 65504.f;
    const auto clamp16 = [lim](float x) { return x != x ? x : fminf(fmaxf(x, -lim), lim); };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = m0 + ty + 16 * i;
        if (row >= p.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t col = n0 + tx + 16 * j;
            if (col >= ncols) continue;
            const float v = clamp16((float)acc[0][i][j]);
            if constexpr (GATED) {
                const float u = clamp16((float)acc[G - 1][i][j]);
                if (p.splits > 1) {
                    float* P = (float*)p.C + (size_t)split * p.M * (2 * p.H);
                    P[(size_t)row * 2 * p.H + col] = v;
                    P[(size_t)row * 2 * p.H + p.H + col] = u;
                } else {
                    float g = v, uu = u;
                    if (p.bias) {
                        g += ld(p.bias, p.bias_dtype, col);
                        uu += ld(p.bias, p.bias_dtype, p.H + col);
                    }
                    st(p.C, p.c_dtype, (size_t)row * p.H + col, epilogue(g, p.epilogue) * uu);
                }
            } else {
                const size_t o = (size_t)row * p.N + col;
                if (p.splits > 1) {
                    ((float*)p.C)[(size_t)split * p.M * p.N + o] = v;
                } else {
                    const float b = p.bias ? ld(p.bias, p.bias_dtype, p.bias_repeat ? o % p.bias_repeat : o) : 0.f;
                    const float r = p.residual ? ld(p.residual, p.residual_dtype,
                                                    p.residual_repeat ? o % p.residual_repeat : o) : 0.f;
                    st(p.C, p.c_dtype, o, finish(v + b, r, p.epilogue, p.residual_order, p.scalar_scale));
                }
            }
        }
    }
}

}   // namespace

hipError_t gemm_acc16_launch(const GemmParams& p, bool gated, hipStream_t s)
{
    const uint32_t ncols = gated ? p.H : p.N;
    const dim3 grid((ncols + TN - 1) / TN, (p.M + TM - 1) / TM, p.splits);
    if (gated) hipLaunchKernelGGL(gemm_acc16_kernel<true>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_acc16_kernel<false>, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}   // namespace vai_dev
