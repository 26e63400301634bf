// scores.hip -- attention scores S = scale * Q K^T with the causal mask, fp16
// Q/K, fp32 S (the Q.K^T stage of /root/reference/vai/shaders/attention.comp:
// 155-182 and attention-fa.comp:581-591; mask rule of common/causal_mask.h).
//
// The work is bound by writing S (4 bytes per score against ~2 flop/byte of
// MFMA work per head-dim element), so the kernel is built around the store:
//  * one workgroup per 128x128 tile of one head; tiles the mask hides
//    entirely are written as -inf and never touch Q, K or the matrix cores;
//  * Q and K rows are copied global->LDS (buffer_load ... lds) in 64-wide
//    head-dim stages, double buffered; 4 waves x (64x64 of 32x32x16 MFMAs);
//    68 KB of LDS, so two workgroups share a CU and one's stores overlap the
//    other's loads (measured on MI355X: one workgroup per CU with all of
//    head_dim in flight is 40% slower, 32-wide stages x 4 is 7% slower);
//  * the accumulators are staged through LDS and written with scale and mask
//    applied, 16 bytes per lane, whole 512-byte row segments per wave.
#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

namespace sc {
constexpr int T = 128, BK = 64, CH = BK / 8, RPW = 16 / CH;    // tile, stage depth, chunks per row
constexpr int SLAB = T * BK * 2;                               // one operand, one stage: 16 KB
constexpr int STAGE = 2 * SLAB;                                // Q + K
constexpr int LOADS = STAGE / (4 * 1024);                      // 1 KB copies per wave per stage
constexpr int EPS = T + 4;                                     // epilogue row stride (floats)
constexpr int NS = 2;                                          // double buffer
constexpr int LDS_BYTES = T * EPS * 4 > NS * STAGE ? T * EPS * 4 : NS * STAGE;
__device__ __forceinline__ int slot(int row, int chunk) { return row * CH + (chunk ^ ((row / RPW) % CH)); }
}

template <int N>
__device__ __forceinline__ void sc_wait_vmcnt()
{
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__global__ __launch_bounds__(256, 2) void scores_kernel(GemmParams p)
{
    using namespace sc;
    extern __shared__ half8 lds[];
    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, fr = lane & 31, fk = lane >> 5;
    const uint32_t m0 = blockIdx.y * T, n0 = blockIdx.x * T, bz = blockIdx.z;
    const uint32_t M = p.M, N = p.N, K = p.K;
    float* S = (float*)p.C + bz * p.c_batch_stride;

    // Tiles the mask hides entirely: -inf, 16 bytes per lane.
    {
        const int64_t first_q = (int64_t)m0 + p.causal_offset, last_q = first_q + T - 1;
        const bool hidden = (p.causal && (int64_t)n0 > last_q) ||
                            (p.span && (int64_t)n0 + T - 1 < first_q + 1 - (int64_t)p.span);
        if (hidden) {
            const float4v ninf = (float4v)(-__builtin_inff());
            const bool vec = (N % 4) == 0;
            for (int i = tid; i < T * (T / 4); i += 256) {
                const uint32_t r = m0 + i / (T / 4), c = n0 + (i % (T / 4)) * 4;
                if (r >= M) continue;
                if (vec && c + 3 < N) *(float4v*)(S + (size_t)r * N + c) = ninf;
                else for (int e = 0; e < 4; ++e) if (c + e < N) S[(size_t)r * N + c + e] = -__builtin_inff();
            }
            return;
        }
    }

    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const half_t*)p.A + bz * p.a_batch_stride), (short)0, (int)((size_t)M * K * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const half_t*)p.B + (bz / p.b_group) * p.b_batch_stride), (short)0, (int)((size_t)N * K * 2),
        0x00020000);
    // Copy i of wave w fills stage slots [(w*LOADS + i)*64, +64): Q rows first, then K rows.
    uint32_t off[LOADS];
    bool isk[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int s = (wave * LOADS + i) * 64 + lane;
        isk[i] = s >= T * CH;
        const int ss = isk[i] ? s - T * CH : s;
        const int row = ss / CH, ch = (ss % CH) ^ ((row / RPW) % CH);
        const uint32_t g = min((isk[i] ? n0 : m0) + row, (isk[i] ? N : M) - 1);
        off[i] = (g * K + ch * 8) * 2;
    }
    const int ktiles = (int)(K / BK);
    auto issue = [&](int kt) {
        LDS_AS char* dst = lds_base + (kt % NS) * STAGE + wave * LOADS * 1024;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            if (isk[i])
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(dst + i * 1024), 16, off[i], kt * BK * 2, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (LDS_AS void*)(dst + i * 1024), 16, off[i], kt * BK * 2, 0, 0);
        }
    };

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (float16v)0.f;

    // Up to NS stages in flight from the start; each later stage is issued
    // into the slot the stage before it freed.
    const int first = min(ktiles, NS);
    for (int kt = 0; kt < first; ++kt) issue(kt);
    for (int kt = 0; kt < ktiles; ++kt) {
        const int later = min(ktiles, kt + NS) - 1 - kt;      // stages issued after kt
        switch (later) {
        case 0: sc_wait_vmcnt<0>(); break;
        case 1: sc_wait_vmcnt<LOADS>(); break;
        case 2: sc_wait_vmcnt<2 * LOADS>(); break;
        default: sc_wait_vmcnt<3 * LOADS>(); break;
        }
        __builtin_amdgcn_s_barrier();
        const half8* q = (const half8*)(lds_base + (kt % NS) * STAGE);
        const half8* k = q + T * CH;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int ch = ks * 2 + fk;
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = q[slot(wm * 64 + i * 32 + fr, ch)];
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = k[slot(wn * 64 + j * 32 + fr, ch)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + NS < ktiles) {
            // every wave is done reading this slot before it is refilled
            __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
            __builtin_amdgcn_s_barrier();
            issue(kt + NS);
        }
    }
    __syncthreads();

    // Epilogue through LDS: D[i][j] of a fragment is lane j + 32*((i/4)%2), register (i%4) + 4*(i/8).
    float* ep = (float*)(lds_base);
    static_for<2>([&](auto I) __attribute__((always_inline)) {
        static_for<2>([&](auto J) __attribute__((always_inline)) {
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int i = I, j = J, r = R;
                ep[(wm * 64 + i * 32 + 8 * (r / 4) + 4 * fk + (r % 4)) * EPS + wn * 64 + j * 32 + fr] = acc[i][j][r];
            });
        });
    });
    __syncthreads();
    const int c4 = (tid & 31) * 4;
    const uint32_t col = n0 + c4;
    const bool vec = (N % 4) == 0 && col + 3 < N;
    for (int rl = tid >> 5; rl < T; rl += 8) {
        const uint32_t row = m0 + rl;
        if (row >= M) break;
        const float4v v = *(const float4v*)(ep + rl * EPS + c4);
        const int64_t pos = (int64_t)row + p.causal_offset;
        float out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = (int64_t)col + e;
            const bool hide = (p.causal && c > pos) || (p.span && pos >= (int64_t)p.span && c < pos + 1 - (int64_t)p.span);
            out[e] = hide ? -__builtin_inff() : v[e] * p.scalar_scale;
        }
        if (vec) *(float4v*)(S + (size_t)row * N + col) = (float4v){out[0], out[1], out[2], out[3]};
        else
            for (int e = 0; e < 4; ++e) if (col + e < N) S[(size_t)row * N + col + e] = out[e];
    }
}

bool scores_fast_ok(const GemmParams& p)
{
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % 64 == 0 &&
           (uint64_t)p.M * p.K * 2 < (1ull << 31) && (uint64_t)p.N * p.K * 2 < (1ull << 31) &&
           ((uintptr_t)p.A % 16) == 0 && ((uintptr_t)p.B % 16) == 0;
}

hipError_t scores_launch(const GemmParams& p, hipStream_t s)
{
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)scores_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           sc::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr = true;
    }
    dim3 grid((p.N + sc::T - 1) / sc::T, (p.M + sc::T - 1) / sc::T, p.batch);
    hipLaunchKernelGGL(scores_kernel, grid, dim3(256), sc::LDS_BYTES, s, p);
    return hipGetLastError();
}

}   // namespace vai_dev
