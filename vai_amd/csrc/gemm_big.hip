// gemm_big.hip -- the prefill GEMM: fp16 x fp16 -> fp32 accumulate on
// v_mfma_f32_32x32x16_f16 with 256x256 workgroup tiles, for the shapes where
// the MFMA pipes, not HBM, bound the work (the Linear tile path at large M
// and the fused gate/up projection).
//
// Layout and schedule for gfx950:
//  * 4 waves per workgroup, each owning a 128x128 block = 4x4 fragments of
//    32x32 (256 fp32 accumulators per lane, in AGPRs). LDS bytes per MFMA
//    flop are then half of what a 64x64 wave tile needs.
//  * K advances in 32-wide stages through a ring of 4 LDS stages (32 KB each:
//    a 256x32 slab of A and of B). Global memory is copied straight into LDS
//    (global_load_lds_dwordx4, no VGPR round trip), three stages ahead of the
//    MFMAs, so ~1.5 us of load latency hides behind the matrix cores. Each
//    wave waits only for its own copies of the stage it is about to read
//    (s_waitcnt vmcnt) and one s_barrier makes the other waves' copies
//    visible; no LDS fence is needed because the copies are the only writes.
//  * A slab row is 64 bytes = 4 chunks of 16 B; chunk c of row r is stored
//    at chunk c ^ ((r >> 2) & 3). The 16 lanes that one LDS cycle serves
//    (rows r..r+15 of a fragment, one chunk) then hit 16 distinct 16-byte
//    bank groups of the 256-byte bank window.
//  * Workgroups are dispatched round-robin over the 8 XCDs. The launch index
//    is remapped so that one XCD's resident workgroups share A and B slabs in
//    its L2 (8 M-tiles x 4 N-tiles per round at the config-3 shape).
#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

namespace big {
constexpr int BM = 256, BN = 256, BK = 32, STAGES = 4;
constexpr int CH = BK / 8;                         // 16-byte chunks per slab row
constexpr int SLAB_BYTES = BM * BK * 2;            // one operand, one stage
constexpr int STAGE_BYTES = 2 * SLAB_BYTES;        // A + B
constexpr int LOADS = (2 * SLAB_BYTES) / (4 * 1024);   // 1 KB wave copies per wave per stage
}

__device__ __forceinline__ int big_slot(int row, int chunk) { return row * big::CH + (chunk ^ ((row >> 2) & 3)); }

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Four consecutive outputs (row, col..col+3) of a Linear: bias, epilogue,
// residual, scale, then one 16- (fp32) or 8-byte (fp16) store when aligned.
__device__ __forceinline__ void store_linear4(const GemmParams& p, uint32_t row, uint32_t col, float4v v)
{
    const size_t o = (size_t)row * p.N + col;
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const size_t oe = o + e;
        const float b = p.bias ? ld(p.bias, p.bias_dtype, p.bias_repeat ? oe % p.bias_repeat : oe) : 0.f;
        const float rr = (p.residual && col + e < p.N)
            ? ld(p.residual, p.residual_dtype, p.residual_repeat ? oe % p.residual_repeat : oe) : 0.f;
        out[e] = finish(v[e] + b, rr, p.epilogue, p.residual_order, p.scalar_scale);
    }
    if (col + 3 < p.N && (o & 3) == 0) {
        if (p.c_dtype == DT_F16) {
            half4 h = {(half_t)out[0], (half_t)out[1], (half_t)out[2], (half_t)out[3]};
            *(half4*)((half_t*)p.C + o) = h;
        } else {
            *(float4v*)((float*)p.C + o) = (float4v){out[0], out[1], out[2], out[3]};
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (col + e < p.N) st(p.C, p.c_dtype, o + e, out[e]);
    }
}

// Four consecutive gated outputs O[row, jo..jo+3] = epi(g + bg) * (u + bu).
__device__ __forceinline__ void store_gated4(const GemmParams& p, uint32_t row, uint32_t jo, float4v g, float4v u)
{
    const size_t o = (size_t)row * p.H + jo;
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float ge = g[e], ue = u[e];
        if (p.bias && jo + e < p.H) {
            ge += ld(p.bias, p.bias_dtype, jo + e);
            ue += ld(p.bias, p.bias_dtype, p.H + jo + e);
        }
        out[e] = epilogue(ge, p.epilogue) * ue;
    }
    if (jo + 3 < p.H && (o & 3) == 0) {
        if (p.c_dtype == DT_F16) {
            half4 h = {(half_t)out[0], (half_t)out[1], (half_t)out[2], (half_t)out[3]};
            *(half4*)((half_t*)p.C + o) = h;
        } else {
            *(float4v*)((float*)p.C + o) = (float4v){out[0], out[1], out[2], out[3]};
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (jo + e < p.H) st(p.C, p.c_dtype, o + e, out[e]);
    }
}

template <bool GATED>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(GemmParams p)
{
    using namespace big;
    extern __shared__ half8 lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware tile order: launch index L runs on XCD L % 8.
    const uint32_t tiles_m = (p.M + BM - 1) / BM;
    const uint32_t tiles_n = gridDim.x / tiles_m;
    uint32_t tm, tn;
    {
        const uint32_t L = blockIdx.x, total = gridDim.x;
        if (total % 8 == 0 && tiles_m <= 8 && (8 % tiles_m) == 0 && tiles_n % 8 == 0) {
            const uint32_t xcd = L % 8, local = L / 8;
            tm = local % tiles_m;
            tn = xcd * (tiles_n / 8) + local / tiles_m;
        } else {
            tm = L % tiles_m;
            tn = L / tiles_m;
        }
    }
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t M = p.M, K = p.K;

    // This lane's source for each of its LOADS copies per stage. Copy i of
    // wave w fills LDS slots [(w*LOADS + i)*64, +64) of the stage: the first
    // half of the copies cover the A slab, the second the B slab. Slot s of
    // a slab holds row s/CH, physical chunk s%CH = logical chunk ^ swizzle.
    const _Float16* src[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int slot = (wave * LOADS + i) * 64 + lane;           // stage-wide slot
        const bool is_b = slot >= BM * CH;
        const int s = is_b ? slot - BM * CH : slot;
        const int row = s / CH, pch = s % CH, ch = pch ^ ((row >> 2) & 3);
        if (!is_b) {
            const uint32_t gm = min(m0 + row, M - 1);               // tail rows: any valid row, never stored
            src[i] = (const _Float16*)p.A + (size_t)gm * K + ch * 8;
        } else {
            uint32_t gn;
            if constexpr (GATED) {
                // logical column -> W row: wave column wn covers 64 output columns,
                // fragments 0-1 their gate rows and 2-3 the matching up rows
                const int w_n = row / 128, within = row % 128, fn = within / 32, j = within % 32;
                const uint32_t jo = min(tn * (BN / 2) + w_n * 64 + (fn & 1) * 32 + j, p.H - 1);
                gn = jo + (fn >= 2 ? p.H : 0u);
            } else {
                gn = min(n0 + row, p.N - 1);
            }
            src[i] = (const _Float16*)p.B + (size_t)gn * K + ch * 8;
        }
    }
    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;
    auto issue = [&](int kt) {
        LDS_AS char* dst = lds_base + (kt % STAGES) * STAGE_BYTES + wave * LOADS * 1024;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(src[i] + (size_t)kt * BK), (LDS_AS void*)(dst + i * 1024),
                                             16, 0, 0);
    };

    float16v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;

    const int ktiles = (int)(K / BK);
    // Prologue: stages 0..STAGES-2 in flight.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < ktiles) issue(s);

    const int fr = lane & 31, fk = lane >> 5;
    for (int kt = 0; kt < ktiles; ++kt) {
        // Own copies of stage kt done (later stages may still fly), then all waves'.
        const int ahead = min(ktiles - 1 - kt, STAGES - 2);   // stages issued after kt
        if (ahead >= 2) wait_vmcnt<2 * LOADS>();
        else if (ahead == 1) wait_vmcnt<LOADS>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        // The ring slot of stage kt-1 is free: every wave has passed this barrier.
        if (kt + STAGES - 1 < ktiles) issue(kt + STAGES - 1);

        const half8* a = (const half8*)(lds_base + (kt % STAGES) * STAGE_BYTES);
        const half8* b = a + BM * CH;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            half8 af[4], bf[4];
            const int ch = ks * 2 + fk;
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = a[big_slot(wm * 128 + i * 32 + fr, ch)];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = b[big_slot(wn * 128 + j * 32 + fr, ch)];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }

    // Epilogue, staged through the now idle LDS one 32-row fragment band at a
    // time: each wave writes its 32x128 band (row stride 132 floats, so the
    // two half-waves' rows fall in different banks), then reads it back by
    // rows and stores 16 bytes per lane. D[i][j] of a fragment sits in lane
    // j + 32*((i/4)%2), register (i%4) + 4*(i/8).
    __builtin_amdgcn_s_barrier();
    constexpr int EPS = 132;
    float* ep = (float*)(lds_base + wave * (32 * EPS * 4));
    const uint32_t rbase = m0 + wm * 128;
    static_for<4>([&](auto I) __attribute__((always_inline)) {
        constexpr int i = I;
        static_for<4>([&](auto J) __attribute__((always_inline)) {
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int j = J, r = R;
                ep[(8 * (r / 4) + 4 * fk + (r % 4)) * EPS + j * 32 + fr] = acc[i][j][r];
            });
        });
        __builtin_amdgcn_wave_barrier();
        if constexpr (GATED) {
            const int c4 = (lane & 15) * 4;
            const uint32_t jo = tn * (BN / 2) + wn * 64 + c4;
            for (int rl = lane >> 4; rl < 32; rl += 4) {
                const float4v g = *(const float4v*)(ep + rl * EPS + c4);
                const float4v u = *(const float4v*)(ep + rl * EPS + 64 + c4);
                const uint32_t row = rbase + i * 32 + rl;
                if (row < M) store_gated4(p, row, jo, g, u);
            }
        } else {
            const int c4 = (lane & 31) * 4;
            const uint32_t col = n0 + wn * 128 + c4;
            for (int rl = lane >> 5; rl < 32; rl += 2) {
                const float4v v = *(const float4v*)(ep + rl * EPS + c4);
                const uint32_t row = rbase + i * 32 + rl;
                if (row < M) store_linear4(p, row, col, v);
            }
        }
        __builtin_amdgcn_wave_barrier();
    });
}

bool gemm_big_ok(const GemmParams& p, bool gated)
{
    const uint32_t ncols = gated ? 2 * p.H : p.N;
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % big::BK == 0 && p.splits == 1 && p.batch == 1 &&
           ((uintptr_t)p.A % 16 == 0) && ((uintptr_t)p.B % 16 == 0) &&
           (size_t)((p.M + 255) / 256) * ((ncols + 255) / 256) >= 128;
}

hipError_t gemm_big_launch(const GemmParams& p, bool gated, hipStream_t s)
{
    const uint32_t tiles_m = (p.M + big::BM - 1) / big::BM;
    const uint32_t tiles_n = gated ? (p.H + big::BN / 2 - 1) / (big::BN / 2) : (p.N + big::BN - 1) / big::BN;
    const size_t lds = (size_t)big::STAGES * big::STAGE_BYTES;
    auto kern = gated ? gemm_big_kernel<true> : gemm_big_kernel<false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[gated]) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set[gated] = true;
    }
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(256), lds, s, p);
    return hipGetLastError();
}

}   // namespace vai_dev
