// gemm_f32.hip -- the fp32 Linear for problems too small to fill the chip
// with ordinary output tiles (the GPT-2 c_fc shape: X[128,768] W[3072,768]):
// fp32 x fp32 -> fp32 on v_mfma_f32_16x16x4_f32, the path linear-tile.comp
// runs with fp32 staging (stageF32) in the reference.
//
// fp32 matrix cores deliver 1/16 of the fp16 rate, so a small fp32 GEMM is
// bound by how many SIMDs stay busy, not by bytes. One workgroup (8 waves,
// two per SIMD, so that one wave's MFMAs cover the other's waits) owns a
// 32 x 16*NF output tile and the full K: the waves split K eight ways and
// their partial tiles are summed once through LDS, so no split-K partials go
// to memory and there is no second launch. NF (at most 3: the eight rings
// fill the 160 KB of LDS) is chosen at plan time so that the tile count lands
// on (a multiple of) the CU count. (Four waves with three-stage rings: 8.87
// against 8.68-8.71 us on config 1, both builds in one run.)
//
// Operand staging: each wave streams its own K range through a private ring
// of LDS stages (no workgroup barrier in the loop). A stage is 32 k of the
// tile's 32 A rows and 16*NF B rows, 128 bytes per row, copied global -> LDS
// by buffer_load ... lds so that every copy instruction reads eight whole
// 128-byte lines (loading MFMA fragments straight into registers reads 16
// half-lines per instruction and ran 2x slower, bound by the vector memory
// path). The 16-byte chunks of row r sit at chunk ^ (r % 8), so the fragment
// reads (16 rows, one chunk) hit distinct banks. The 16x16x4 fp32 MFMA takes
// one A and one B value per lane (row/column l % 16, k-slot l / 16); a lane
// reads 4 consecutive k as one 16-byte chunk and feeds them to 4 MFMAs, so
// the k order is 4*(l/16) + q on both operands and every product is still
// summed once. Rows past M or N read as zero through the buffer resource's
// range check.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

namespace vai_dev {

namespace f32k {
constexpr int WAVES = 8;   // two per SIMD: one's MFMAs cover the other's waits
constexpr int SLOTS = 2;   // LDS stages per wave (one copy ahead)
constexpr int KC = 32;     // k per stage: 128 bytes of each row
}

typedef float float4v __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

// s_waitcnt with only vmcnt (or only lgkmcnt) constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void f32k_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void f32k_wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

template <int NF>
constexpr size_t f32k_stage_bytes() { return (size_t)(32 + 16 * NF) * 128; }
template <int NF>
constexpr size_t f32k_lds_bytes()
{
    const size_t ring = (size_t)f32k::WAVES * f32k::SLOTS * f32k_stage_bytes<NF>();
    const size_t red = (size_t)f32k::WAVES * 2 * NF * 4 * 64 * 4;
    return ring > red ? ring : red;
}

// fp32 output, no residual, bias absent or one [N] row: the activation is
// compile-time (EPI 6: the runtime epilogue code).
template <int NF, uint32_t EPI>
__device__ __forceinline__ void f32k_store(const GemmParams& p, const float (&v)[NF], const float (&cbias)[NF],
                                           uint32_t row, uint32_t col)
{
    const uint32_t M = p.M, N = p.N;
    const float s = p.scalar_scale;
    if (row >= M) return;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const uint32_t c = col + j * 16;
        if (c < N) ((float*)p.C)[(size_t)row * N + c] = s * epilogue(v[j] + cbias[j], EPI == 6 ? p.epilogue : EPI);
    }
}

template <int NF>
__global__ __launch_bounds__(64 * f32k::WAVES) void gemm_f32_kernel(GemmParams p)
{
    using namespace f32k;
    constexpr int BM = 32, BN = 16 * NF;
    constexpr int A_LOADS = 32 * 8 / 64, B_LOADS = 16 * NF * 8 / 64, LOADS = A_LOADS + B_LOADS;
    constexpr uint32_t STAGE = f32k_stage_bytes<NF>();
    extern __shared__ float4v lds_raw[];
    LDS_AS char* lds = (LDS_AS char*)(LDS_AS void*)lds_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    // Workgroups go round-robin over the 8 XCDs; give each XCD a contiguous
    // run of tiles, column-major, so the M-tiles sharing a weight slab share
    // one L2.
    uint32_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    const uint32_t tm = __builtin_amdgcn_readfirstlane(t % tiles_m);
    const uint32_t tn = __builtin_amdgcn_readfirstlane(t / tiles_m);

    const uint32_t r0 = tm * BM, c0 = tn * BN;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const float*)p.A + (size_t)r0 * K), (short)0, (int)((M - r0) * K * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const float*)p.B + (size_t)c0 * K), (short)0, (int)((N - c0) * K * 4), 0x00020000);
    // Copy slot s = instruction*64 + lane holds row s/8, physical chunk s%8
    // = logical chunk ^ (row % 8): its global byte offset within a stage.
    const uint32_t crow = lane / 8, cch = (lane % 8) ^ (crow % 8);
    const uint32_t coff = (crow * K + cch * 4) * 4;   // + instruction * 8 rows
    const uint32_t row8 = 8 * K * 4;

    // Wave w runs stages [c_lo, c_hi) of the K/32 stages.
    const int chunks = (int)(K / KC);
    const int c_lo = wave * chunks / WAVES, c_hi = (wave + 1) * chunks / WAVES;
    const int n = c_hi - c_lo;
    LDS_AS char* ring = lds + (size_t)wave * SLOTS * STAGE;

    // The fast epilogue's bias (one [N] row) for this thread's NF columns
    // c0 + lane % 16 + 16 j, loaded now, unconditionally (columns clamped),
    // so that its latency hides behind the K loop instead of following it.
    float cbias[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) cbias[j] = 0.f;
    if (p.bias) {
        if (p.bias_dtype == DT_F16) {
#pragma unroll
            for (int j = 0; j < NF; ++j) cbias[j] = (float)((const half_t*)p.bias)[min(c0 + (lane & 15) + 16 * j, N - 1)];
        } else {
#pragma unroll
            for (int j = 0; j < NF; ++j) cbias[j] = ((const float*)p.bias)[min(c0 + (lane & 15) + 16 * j, N - 1)];
        }
    }

    float4v acc[2][NF];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc[i][j] = (float4v)0.f;

    // Stages past the wave's range copy its last stage again (never read),
    // so the number of copies in flight, and every wait, is fixed.
    auto issue = [&](int slot, int c) __attribute__((always_inline)) {
        const int kb = (min(c, c_hi - 1)) * KC * 4;
        LDS_AS char* dst = ring + slot * STAGE;
#pragma unroll
        for (int u = 0; u < A_LOADS; ++u)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (LDS_AS void*)(dst + u * 1024), 16, (int)(coff + u * row8), kb,
                                                     0, 0);
#pragma unroll
        for (int u = 0; u < B_LOADS; ++u)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (LDS_AS void*)(dst + (A_LOADS + u) * 1024), 16,
                                                     (int)(coff + u * row8), kb, 0, 0);
    };
    // Fragment reads: lane l takes row (16*f + l%16), logical chunk h*4 + l/16.
    // Half h of a stage (16 of its 32 k) goes into register set h; the
    // next stage's first half is read while this stage's second half runs
    // its MFMAs, so no stage starts on an LDS read latency.
    const uint32_t fr = lane & 15, fc = lane >> 4;
    float4v fa[2][2], fb[2][NF];
    auto read = [&](int slot, auto H) __attribute__((always_inline)) {
        constexpr int h = decltype(H)::value;
        LDS_AS const char* src = ring + slot * STAGE;
        const uint32_t off = (fr * 8 + ((h * 4 + fc) ^ (fr % 8))) * 16;
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[h][i] = *(LDS_AS const float4v*)(src + off + i * 16 * 128);
#pragma unroll
        for (int j = 0; j < NF; ++j) fb[h][j] = *(LDS_AS const float4v*)(src + 32 * 128 + off + j * 16 * 128);
    };
    auto mma = [&](auto H) __attribute__((always_inline)) {
        constexpr int h = decltype(H)::value;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NF; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[h][i][q], fb[h][j][q], acc[i][j], 0, 0, 0);
    };
    if (n > 0) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) issue(s, c_lo + s);
        f32k_wait_vmcnt<(SLOTS - 1) * LOADS>();   // stage 0 has landed
        read(0, std::integral_constant<int, 0>{});
        int slot = 0;
        for (int c = 0; c < n; ++c) {
            const int next = slot + 1 == SLOTS ? 0 : slot + 1;
            read(slot, std::integral_constant<int, 1>{});
            mma(std::integral_constant<int, 0>{});
            if (c + 1 < n) {
                // stage c + 1 has landed: stages up to c + SLOTS - 1 were
                // issued, and only the SLOTS - 2 after c + 1 may be in flight
                f32k_wait_vmcnt<(SLOTS - 2) * LOADS>();
                read(next, std::integral_constant<int, 0>{});
            }
            mma(std::integral_constant<int, 1>{});
            f32k_wait_lgkmcnt0();                      // every read of this slot has returned
            issue(slot, c_lo + c + SLOTS);
            slot = next;
        }
    }
    f32k_wait_vmcnt<0>();   // the clamped copies land before the ring is reused
    __syncthreads();
    float (*red)[2 * NF * 4][64] = (float (*)[2 * NF * 4][64])lds_raw;

    // The WAVES partial tiles meet in LDS; every thread then finishes NF
    // outputs. Thread (wave w, lane l) takes register r = w % 4 of the
    // fragments (w / 4, j): row 16 (w / 4) + 4 (l / 16) + r, column 16 j + l % 16.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(i * NF + j) * 4 + r][lane] = acc[i][j][r];
    __syncthreads();
    static_assert(WAVES == 8, "two fragment rows x four registers");
    const int fi = wave >> 2, fr4 = wave & 3;
    const uint32_t col_l = lane & 15, row_l = fi * 16 + (lane >> 4) * 4 + fr4;
    float v[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) a += red[w][(fi * NF + j) * 4 + fr4][lane];
        v[j] = a;
    }
    const bool plain = p.c_dtype == 0 && !p.residual && (!p.bias || p.bias_repeat == N);
    if (plain) {
        switch (p.epilogue) {
        case 0: f32k_store<NF, 0>(p, v, cbias, r0 + row_l, c0 + col_l); break;
        case 3: f32k_store<NF, 3>(p, v, cbias, r0 + row_l, c0 + col_l); break;
        case 4: f32k_store<NF, 4>(p, v, cbias, r0 + row_l, c0 + col_l); break;
        default: f32k_store<NF, 6>(p, v, cbias, r0 + row_l, c0 + col_l); break;
        }
        return;
    }
    const uint32_t row = r0 + row_l;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const uint32_t col = c0 + j * 16 + col_l;
        if (row < M && col < N) {
            const size_t o = (size_t)row * N + col;
            const float bb = p.bias ? ld(p.bias, p.bias_dtype, p.bias_repeat ? o % p.bias_repeat : o) : 0.f;
            const float res = p.residual
                ? ld(p.residual, p.residual_dtype, p.residual_repeat ? o % p.residual_repeat : o) : 0.f;
            st(p.C, p.c_dtype, o, finish(v[j] + bb, res, p.epilogue, p.residual_order, p.scalar_scale));
        }
    }
}

// fp32 operands, K a multiple of 32 (a stage's 128 bytes stay inside a row), and
// 32-bit buffer offsets.
bool gemm_f32_ok(const GemmParams& p)
{
    return p.a_dtype == 0 && p.b_dtype == 0 && p.K % 32 == 0 && p.K >= 32 && p.batch == 1 && p.splits == 1 &&
           (uint64_t)p.M * p.K * 4 < (1ull << 31) && (uint64_t)p.N * p.K * 4 < (1ull << 31);
}

// Column fragments per tile: the NF whose tile count fills the CUs in the
// fewest rounds of per-tile work (a round costs NF fragment columns).
int gemm_f32_nf(uint32_t M, uint32_t N, uint32_t cus)
{
    int best = 1;
    uint64_t best_cost = ~0ull;
    for (int nf = 3; nf >= 1; --nf) {   // NF = 4 would need 192 KB of LDS rings
        const uint64_t tiles = (uint64_t)((M + 31) / 32) * ((N + 16 * nf - 1) / (16 * nf));
        const uint64_t cost = (tiles + cus - 1) / cus * nf;
        if (cost < best_cost) { best_cost = cost; best = nf; }
    }
    return best;
}

template <int NF>
static hipError_t f32k_launch(const GemmParams& p, hipStream_t s)
{
    // The ring takes up to 144 KB: above the default dynamic LDS limit.
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)gemm_f32_kernel<NF>, (int)f32k_lds_bytes<NF>());
    if (e != hipSuccess) return e;
    const uint32_t tiles = ((p.M + 31) / 32) * ((p.N + 16 * NF - 1) / (16 * NF));
    hipLaunchKernelGGL(gemm_f32_kernel<NF>, dim3(tiles), dim3(64 * f32k::WAVES), f32k_lds_bytes<NF>(), s, p);
    return hipGetLastError();
}

hipError_t gemm_f32_launch(const GemmParams& p, int nf, hipStream_t s)
{
    switch (nf) {
    case 1: return f32k_launch<1>(p, s);
    case 2: return f32k_launch<2>(p, s);
    case 3: return f32k_launch<3>(p, s);
    default: return hipErrorInvalidValue;
    }
}

}   // namespace vai_dev
