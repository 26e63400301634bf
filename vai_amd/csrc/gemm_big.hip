// gemm_big.hip -- the prefill GEMM: fp16 x fp16 -> fp32 accumulate on
// v_mfma_f32_32x32x16_f16 with 256x256 workgroup tiles, for the shapes where
// the MFMA pipes, not HBM, bound the work (the Linear tile path at large M
// and the fused gate/up projection).
//
// Layout and schedule for gfx950:
//  * 4 waves per workgroup, each owning a 128x128 block = 4x4 fragments of
//    32x32 (256 fp32 accumulators per lane, in AGPRs). LDS bytes per MFMA
//    flop are then half of what a 64x64 wave tile needs.
//  * K advances in 64-wide stages through 2 LDS stages (64 KB each: a 256x64
//    slab of A and of B). Global memory is copied straight into LDS
//    (global_load_lds_dwordx4, no VGPR round trip) one stage ahead of the
//    MFMAs. Each wave waits only for its own copies of the stage it is about
//    to read (s_waitcnt vmcnt) and one s_barrier per stage makes the other
//    waves' copies visible; no LDS fence is needed because the copies are the
//    only writes. Measured on MI355X: 32-wide stages x 4 (more lookahead,
//    twice the barriers) is ~3% slower; streaming B from L2 into VGPRs to
//    halve LDS traffic is ~25% slower (L2->CU traffic doubles for B).
//  * Slab rows are CH 16-byte chunks; chunk c of row r is stored at
//    chunk c ^ ((r / RPW) % CH), RPW = rows per 256-byte bank window. The 16
//    lanes one LDS cycle serves (16 rows of a fragment, one chunk) then hit 16
//    distinct 16-byte bank groups.
//  * Workgroups are dispatched round-robin over the 8 XCDs. The launch index
//    is remapped so that one XCD's resident workgroups share A and B slabs in
//    its L2 (8 M-tiles x 4 N-tiles per round at the config-3 shape).
#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

namespace big {
constexpr int BM = 256, BN = 256;
// K per LDS stage and ring depth (the kernel is a template over both).
template <int BK, int STAGES> struct Cfg {
    static constexpr int CH = BK / 8;                          // 16-byte chunks per slab row
    static constexpr int SLAB_BYTES = BM * BK * 2;             // one operand, one stage
    static constexpr int STAGE_BYTES = 2 * SLAB_BYTES;         // A + B
    static constexpr int LOADS = STAGE_BYTES / (4 * 1024);     // 1 KB wave copies per wave per stage
    static constexpr int RPW = 16 / CH;                        // slab rows per 256-byte bank window
    // chunk c of row r lives at chunk c ^ ((r / RPW) % CH): the 16 lanes an
    // LDS cycle serves (16 consecutive rows, one chunk) hit 16 distinct
    // 16-byte bank groups.
    static __device__ __forceinline__ int slot(int row, int chunk) { return row * CH + (chunk ^ ((row / RPW) % CH)); }
};
}

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
    if (col + 3 < p.N && (p.N & 3) == 0) {   // wave-uniform: every row start is 16-byte aligned
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
    if (jo + 3 < p.H && (p.H & 3) == 0) {
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

__device__ __forceinline__ void wait_lgkmcnt0()
{
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

template <bool GATED, int BK, int STAGES>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(GemmParams p)
{
    using namespace big;
    typedef Cfg<BK, STAGES> C;
    constexpr int CH = C::CH, STAGE_BYTES = C::STAGE_BYTES, LOADS = C::LOADS, KS = BK / 16;
    extern __shared__ half8 lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform, kept in an SGPR
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
        const int row = s / CH, pch = s % CH, ch = pch ^ ((row / C::RPW) % CH);
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
    const int ktiles = (int)(K / BK);
    // Copies stage kt into ring slot kt % STAGES. Past the last stage the
    // source is clamped to it: the copy is harmless (its slot is never read
    // again) and keeps the number of copies in flight fixed, so every wait
    // below is a compile-time vmcnt.
    auto issue = [&](int kt) {
        const int ksrc = min(kt, ktiles - 1);
        LDS_AS char* dst = lds_base + (kt % STAGES) * STAGE_BYTES + wave * LOADS * 1024;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(src[i] + (size_t)ksrc * BK), (LDS_AS void*)(dst + i * 1024),
                                             16, 0, 0);
    };
    const int fr = lane & 31, fk = lane >> 5;
    // Fragment reads of one 16-wide k substep of a stage.
    auto read_frags = [&](int kt, int ks, half8* af, half8* bf) {
        const half8* a = (const half8*)(lds_base + (kt % STAGES) * STAGE_BYTES);
        const half8* b = a + BM * CH;
        const int ch = ks * 2 + fk;
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = a[C::slot(wm * 128 + i * 32 + fr, ch)];
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = b[C::slot(wn * 128 + j * 32 + fr, ch)];
    };

    float16v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;
    // Half of a substep's 16 MFMAs: fragment rows i = 2h, 2h+1.
    auto mfma_half = [&](const half8* af, const half8* bf, int h) {
#pragma unroll
        for (int i = 2 * h; i < 2 * h + 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    };

    // Prologue: all STAGES slots in flight, then stage 0 landed everywhere.
#pragma unroll
    for (int st = 0; st < STAGES; ++st) issue(st);
    wait_vmcnt<(STAGES - 1) * LOADS>();
    __builtin_amdgcn_s_barrier();
    half8 fa[2][4], fb[2][4];   // fragments of the current and the next 16-wide substep
    read_frags(0, 0, fa[0], fb[0]);

    for (int kt = 0; kt + 1 < ktiles; ++kt) {
        static_for<KS>([&](auto Q) __attribute__((always_inline)) {
            constexpr int q = Q, cur = q & 1, nxt = cur ^ 1;
            if constexpr (q + 1 < KS) {
                // MFMAs on substep q while substep q + 1's fragments load.
                read_frags(kt, q + 1, fa[nxt], fb[nxt]);
                mfma_half(fa[cur], fb[cur], 0);
                mfma_half(fa[cur], fb[cur], 1);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // 1 LDS read
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                __builtin_amdgcn_sched_barrier(0);   // substeps do not mix
            } else {
                // Last substep: half its MFMAs cover the stage barrier; after it
                // slot kt is free for stage kt + STAGES and stage kt + 1 is read.
                mfma_half(fa[cur], fb[cur], 0);
                __builtin_amdgcn_sched_barrier(0);       // these MFMAs stay ahead of the barrier
                wait_lgkmcnt0();                         // this wave's reads of slot kt are done
                wait_vmcnt<(STAGES - 2) * LOADS>();      // its copies of stage kt + 1 have landed
                __builtin_amdgcn_s_barrier();
                issue(kt + STAGES);
                read_frags(kt + 1, 0, fa[nxt], fb[nxt]);
                mfma_half(fa[cur], fb[cur], 1);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                    __builtin_amdgcn_sched_group_barrier(0x020, LOADS / 8, 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    }
    // Last stage (KS is even, so its substep 0 fragments sit in fa[0]).
    static_for<KS>([&](auto Q) __attribute__((always_inline)) {
        constexpr int q = Q, cur = q & 1, nxt = cur ^ 1;
        if constexpr (q + 1 < KS) read_frags(ktiles - 1, q + 1, fa[nxt], fb[nxt]);
        mfma_half(fa[cur], fb[cur], 0);
        mfma_half(fa[cur], fb[cur], 1);
    });
    wait_vmcnt<0>();   // the clamped copies must land before LDS is reused

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

#ifndef VAI_BIG_BK
#define VAI_BIG_BK 64
#define VAI_BIG_STAGES 2
#endif
constexpr int kBigBK = VAI_BIG_BK, kBigStages = VAI_BIG_STAGES;

bool gemm_big_ok(const GemmParams& p, bool gated)
{
    const uint32_t ncols = gated ? 2 * p.H : p.N;
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % kBigBK == 0 && p.splits == 1 && p.batch == 1 &&
           ((uintptr_t)p.A % 16 == 0) && ((uintptr_t)p.B % 16 == 0) &&
           (size_t)((p.M + 255) / 256) * ((ncols + 255) / 256) >= 128;
}

hipError_t gemm_big_launch(const GemmParams& p, bool gated, hipStream_t s)
{
    const uint32_t tiles_m = (p.M + big::BM - 1) / big::BM;
    const uint32_t tiles_n = gated ? (p.H + big::BN / 2 - 1) / (big::BN / 2) : (p.N + big::BN - 1) / big::BN;
    const size_t lds = (size_t)kBigStages * big::Cfg<kBigBK, kBigStages>::STAGE_BYTES;
    auto kern = gated ? gemm_big_kernel<true, kBigBK, kBigStages> : gemm_big_kernel<false, kBigBK, kBigStages>;
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
