// mfma_rate.cpp -- the matrix-core ceiling of this GPU for fp16 MFMA work,
// and how it depends on the operand data: 256 workgroups x 4 waves (one wave
// per SIMD) issue back-to-back v_mfma_f32_32x32x16_f16 on 16 independent
// accumulators, once with constant operands and once with random ones
// (U(-1,1) fp16). Prints TFLOP/s for each of three timed runs. Then the
// fp32 matrix rate (v_mfma_f32_16x16x4_f32 and v_mfma_f32_32x32x2_f32, random
// operands), the ceiling of the fp32 Linear path.
//
//   mfma_rate [iters]
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
template <bool RANDOM>
__global__ __launch_bounds__(256, 1) void mf(const half8* src, float16v* out, int iters) {
  half8 a[4], b[4];
  for (int i = 0; i < 4; ++i) {
    if (RANDOM) { a[i] = src[(blockIdx.x * 256 + threadIdx.x) * 8 + i]; b[i] = src[(blockIdx.x * 256 + threadIdx.x) * 8 + 4 + i]; }
    else { a[i] = (half8)(_Float16)(threadIdx.x * 0.001f); b[i] = (half8)(_Float16)1.0f; }
  }
  float16v acc[4][4];
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  float16v s = (float16v)0.f;
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) s += acc[i][j];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
typedef float float4v __attribute__((ext_vector_type(4)));
// fp32: 16 independent accumulators per wave, 16x16x4 (4 regs) or 32x32x2
// (16 regs) shapes.
template <bool BIG>
__global__ __launch_bounds__(256, 1) void mf32(const float* src, float* out, int iters) {
  float a[4], b[4];
  for (int i = 0; i < 4; ++i) { a[i] = src[(blockIdx.x * 256 + threadIdx.x) * 8 + i]; b[i] = src[(blockIdx.x * 256 + threadIdx.x) * 8 + 4 + i]; }
  float s = 0.f;
  if constexpr (BIG) {
    float16v acc[4][4];
    for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  } else {
    float4v acc[4][4];
    for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) acc[i][j] = (float4v)0.f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) for (int r = 0; r < 4; ++r) s += acc[i][j][r];
  }
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
#define CHECK(x)                                                                  \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));               \
            return 1;                                                             \
        }                                                                         \
    } while (0)

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 4000;
  const size_t n = 256 * 256 * 8 * 8;   // halves: 8 half8 operands per thread
  half8* src;
  CHECK(hipMalloc(&src, n * 2));
  {
    _Float16* h = (_Float16*)malloc(n * 2);
    unsigned s = 1;
    for (size_t i = 0; i < n; ++i) { s = s * 1664525u + 1013904223u; h[i] = (_Float16)((((s >> 9) & 0xFFFF) / 32768.0f - 1.0f)); }
    CHECK(hipMemcpy(src, h, n * 2, hipMemcpyHostToDevice));
    free(h);
  }
  float16v* o;
  CHECK(hipMalloc(&o, 256 * 256 * sizeof(float16v)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int v = 0; v < 2; ++v) {
    auto k = v ? mf<true> : mf<false>;
    hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src, o, 10);
    CHECK(hipDeviceSynchronize());
    for (int rep = 0; rep < 3; ++rep) {
      CHECK(hipEventRecord(e0));
      hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src, o, iters);
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      const double flops = 256.0 * 4 * iters * 16 * 32768.0;
      printf("%s operands: %.3f ms, %.1f TFLOP/s\n", v ? "random" : "constant", ms, flops / ms / 1e9);
    }
  }
  float* src32;
  CHECK(hipMalloc(&src32, 256 * 256 * 8 * 4));
  {
    float* h = (float*)malloc(256 * 256 * 8 * 4);
    unsigned s = 7;
    for (size_t i = 0; i < 256 * 256 * 8; ++i) { s = s * 1664525u + 1013904223u; h[i] = ((s >> 9) & 0xFFFF) / 32768.0f - 1.0f; }
    CHECK(hipMemcpy(src32, h, 256 * 256 * 8 * 4, hipMemcpyHostToDevice));
    free(h);
  }
  const int iters32 = iters / 4 > 0 ? iters / 4 : 1;
  for (int v = 0; v < 2; ++v) {
    auto k = v ? mf32<true> : mf32<false>;
    hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src32, (float*)o, 10);
    CHECK(hipDeviceSynchronize());
    for (int rep = 0; rep < 3; ++rep) {
      CHECK(hipEventRecord(e0));
      hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src32, (float*)o, iters32);
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      const double flops = 256.0 * 4 * iters32 * 16 * (v ? 4096.0 : 2048.0);
      printf("fp32 %s random operands: %.3f ms, %.1f TFLOP/s\n", v ? "32x32x2" : "16x16x4", ms, flops / ms / 1e9);
    }
  }
  return 0;
}
