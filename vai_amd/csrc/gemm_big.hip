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
//    (buffer_load ... lds, no VGPR round trip; rows past the operand read as
//    zero) one stage ahead of the MFMAs. Each wave waits only for its own
//    copies of the stage it is about to read (s_waitcnt vmcnt) and one
//    s_barrier per stage makes the other waves' copies visible; no LDS fence
//    is needed because the copies are the only writes. Measured on MI355X:
//    32-wide stages x 4 (more lookahead, twice the barriers) is ~3% slower;
//    streaming B from L2 into VGPRs to halve LDS traffic is ~25% slower (L2->CU
//    traffic doubles for B).
//  * Slab rows are CH 16-byte chunks; chunk c of row r is stored at
//    chunk c ^ ((r / RPW) % CH), RPW = rows per 256-byte bank window. The 16
//    lanes one LDS cycle serves (16 rows of a fragment, one chunk) then hit 16
//    distinct 16-byte bank groups.
//  * Persistent: at most one workgroup per CU, each walking its tiles as one
//    stream of K stages. The next tile's first copies are in flight while a
//    finished tile is written straight from the accumulators (two 128-byte
//    row segments per store instruction, no LDS round trip), and those stores
//    drain behind the next tile's MFMAs.
//  * Workgroups are dispatched round-robin over the 8 XCDs. Tile indices are
//    remapped so that one XCD's resident workgroups share A and B slabs in
//    its L2 (8 M-tiles x 4 N-tiles per round at the config-3 shape).
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"
#include "tile_store.h"

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

// Keeps a substep's MFMA operands allocated until all of its MFMAs have
// issued: the fragment reads interleaved with those MFMAs then cannot be
// given a register an issued-but-not-started MFMA still has to read.
__device__ __forceinline__ void keep_operands(const half8 (&a)[4], const half8 (&b)[4])
{
    asm volatile("" ::"v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
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

// Persistent: a grid of at most one workgroup per CU walks its tiles as one
// continuous stream of K stages, so the copies of a tile's first stages are
// in flight while the previous tile's accumulators are written out, and the
// output stores drain behind the next tile's MFMAs.
template <bool GATED, int BK, int STAGES>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(GemmParams p)
{
    using namespace big;
    typedef Cfg<BK, STAGES> C;
    constexpr int CH = C::CH, STAGE_BYTES = C::STAGE_BYTES, LOADS = C::LOADS, KS = BK / 16;
    static_assert(4 * LOADS * 64 == 2 * BM * CH, "copies cover one stage");
    extern __shared__ half8 lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform, kept in an SGPR
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t M = p.M, K = p.K;

    const uint32_t G = gridDim.x;
    const TileOrder order = TileOrder::make((M + BM - 1) / BM, GATED ? (p.H + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN, G);
    const uint32_t total = order.tiles_m * order.tiles_n;
    const int ktiles = (int)(K / BK);
    const int my_tiles = __builtin_amdgcn_readfirstlane((int)((total - blockIdx.x + G - 1) / G));
    const int S = my_tiles * ktiles;   // K stages this workgroup runs

    // Copies: waves 0-1 fill the A slab of a stage, waves 2-3 the B slab; copy
    // i of wave w fills slots [(w*LOADS + i)*64, +64). Slot s of a slab holds
    // row s/CH, physical chunk s%CH = logical chunk ^ swizzle. The per-lane
    // byte offsets do not depend on the tile: the tile and the stage enter as
    // one wave-uniform offset. Rows past M (A) or past N / 2H (B) lie beyond
    // the buffer's extent and read as zero; gated tail columns read rows whose
    // outputs are never stored.
    const bool is_b = wave >= 2;
    uint32_t voff[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int slot = ((wave & 1) * LOADS + i) * 64 + lane;
        const int row = slot / CH, pch = slot % CH, ch = pch ^ ((row / C::RPW) % CH);
        uint32_t r = row;
        if constexpr (GATED) {
            // logical column -> W row: wave column w_n covers 64 output columns,
            // fragments 0-1 their gate rows and 2-3 the matching up rows
            const int w_n = row / 128, within = row % 128, fn = within / 32, j = within % 32;
            const uint32_t jo = w_n * 64 + (fn & 1) * 32 + j;
            r = is_b ? jo + (fn >= 2 ? p.H : 0u) : (uint32_t)row;
        }
        voff[i] = (r * K + ch * 8) * 2;
    }
    const uint32_t tile_rows_b = GATED ? BN / 2 : BN;   // W rows one N-tile advances by (gate half)

    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;
    // Copies stage g of the stream into ring slot g % STAGES. Past the last
    // stage the source is clamped to it: the copy is harmless (its slot is
    // never read again) and keeps the number of copies in flight fixed, so
    // every wait below is a compile-time vmcnt.
    auto issue = [&](int g) __attribute__((always_inline)) {
        const int gs = min(g, S - 1);
        const int r = gs / ktiles;
        const int kt = __builtin_amdgcn_readfirstlane(gs - r * ktiles);   // uniform (the divisions run on VALU)
        uint32_t tm, tn;
        order.of(blockIdx.x + (uint32_t)r * G, tm, tn);
        tm = __builtin_amdgcn_readfirstlane(tm);
        tn = __builtin_amdgcn_readfirstlane(tn);
        // The resource starts at the tile's first row (of A, or of W) and ends
        // at the operand's last row: rows past it are out of bounds (read as
        // zero) through the per-lane offset alone.
        const uint32_t row0 = is_b ? tn * tile_rows_b : tm * BM;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const half_t*)(is_b ? p.B : p.A) + (size_t)row0 * K), (short)0,
            (int)(((is_b ? p.N : M) - row0) * K * 2), 0x00020000);
        LDS_AS char* dst = lds_base + (g % STAGES) * STAGE_BYTES + wave * LOADS * 1024;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)(dst + i * 1024), 16, (int)voff[i],
                                                     (int)((uint32_t)kt * BK * 2), 0, 0);
    };
    const int fr = lane & 31, fk = lane >> 5;
    // Fragment rows of one wave are fr + 32*i (+ 128*wave row): the swizzle
    // term (row / RPW) % CH is the same for all of them, so each 16-wide k
    // substep needs one LDS address per slot and the fragments sit at
    // immediate offsets from it.
    static_assert((32 / C::RPW) % CH == 0, "fragment rows share the swizzle");
    const int swz = (fr / C::RPW) % CH;
    auto read_frags = [&](int g, int ks, half8* af, half8* bf) __attribute__((always_inline)) {
        const int ch = (ks * 2 + fk) ^ swz;
        LDS_AS const char* a = lds_base + (g % STAGES) * STAGE_BYTES + ((wm * 128 + fr) * CH + ch) * 16;
        LDS_AS const char* b = lds_base + (g % STAGES) * STAGE_BYTES + BM * CH * 16 + ((wn * 128 + fr) * CH + ch) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = *(LDS_AS const half8*)(a + i * 32 * CH * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = *(LDS_AS const half8*)(b + j * 32 * CH * 16);
    };

    // Writes a finished tile straight from the accumulators. D[i][j] of a
    // 32x32 fragment sits in lane j + 32*((i/4)%2), register (i%4) + 4*(i/8):
    // for each register a half-wave holds 32 consecutive columns of one row,
    // so every store instruction writes two 128-byte row segments.
    // Prologue: all STAGES slots in flight, then stage 0 landed everywhere.
#pragma unroll
    for (int st = 0; st < STAGES; ++st) issue(st);
    wait_vmcnt<(STAGES - 1) * LOADS>();
    __builtin_amdgcn_s_barrier();
    half8 fa[2][4], fb[2][4];   // fragments of the current and the next 16-wide substep
    read_frags(0, 0, fa[0], fb[0]);

    int g = 0;
    for (int r = 0; r < my_tiles; ++r) {
        float cb[4];
        {
            uint32_t tm, tn;
            order.of(blockIdx.x + (uint32_t)r * G, tm, tn);
            tile_col_bias<GATED>(p, tn, wn, fr, cb);
        }
        float16v acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;
        // Half of a substep's 16 MFMAs: fragment rows i = 2h, 2h+1.
        auto mfma_half = [&](const half8* af, const half8* bf, int h) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 2 * h; i < 2 * h + 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        };

        for (int kt = 0; kt < ktiles; ++kt, ++g) {
            static_for<KS>([&](auto Q) __attribute__((always_inline)) {
                constexpr int q = Q, cur = q & 1, nxt = cur ^ 1;
                if constexpr (q + 1 < KS) {
                    // MFMAs on substep q while substep q + 1's fragments load.
                    read_frags(g, q + 1, fa[nxt], fb[nxt]);
                    mfma_half(fa[cur], fb[cur], 0);
                    mfma_half(fa[cur], fb[cur], 1);
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // 1 LDS read
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                    __builtin_amdgcn_sched_barrier(0);   // substeps do not mix
                    keep_operands(fa[cur], fb[cur]);
                } else {
                    // Last substep: half its MFMAs cover the stage barrier; after it
                    // slot g is free for stage g + STAGES and stage g + 1 is read.
                    mfma_half(fa[cur], fb[cur], 0);
                    __builtin_amdgcn_sched_barrier(0);       // these MFMAs stay ahead of the barrier
                    wait_lgkmcnt0();                         // this wave's reads of slot g are done
                    wait_vmcnt<(STAGES - 2) * LOADS>();      // its copies of stage g + 1 have landed
                    __builtin_amdgcn_s_barrier();
                    issue(g + STAGES);
                    read_frags(g + 1, 0, fa[nxt], fb[nxt]);
                    mfma_half(fa[cur], fb[cur], 1);
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                        __builtin_amdgcn_sched_group_barrier(0x020, LOADS / 8, 1);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    keep_operands(fa[cur], fb[cur]);
                }
            });
        }
        {
            // (tile indices made wave-uniform: the store resource built from
            // them then lives in SGPRs, not in a waterfall loop per store)
            uint32_t tm, tn;
            order.of(blockIdx.x + (uint32_t)r * G, tm, tn);
            tile_store<GATED>(p, acc, cb, __builtin_amdgcn_readfirstlane(tm), __builtin_amdgcn_readfirstlane(tn), wm,
                              wn, fr, fk);
        }
    }
    wait_vmcnt<0>();   // the clamped copies land before the workgroup retires
}

#ifndef VAI_BIG_BK
#define VAI_BIG_BK 64
#define VAI_BIG_STAGES 2
#endif
constexpr int kBigBK = VAI_BIG_BK, kBigStages = VAI_BIG_STAGES;

bool gemm_big_ok(const GemmParams& p, bool gated)
{
    const uint32_t ncols = gated ? 2 * p.H : p.N;
    // byte offsets into A and W are 32-bit buffer offsets
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % kBigBK == 0 && p.splits == 1 && p.batch == 1 &&
           (size_t)p.M * p.K * 2 < (1u << 31) && (size_t)ncols * p.K * 2 < (1u << 31) &&
           (size_t)((p.M + 255) / 256) * ((ncols + 255) / 256) >= 128;
}

hipError_t gemm_big_launch(const GemmParams& p, bool gated, hipStream_t s)
{
    const uint32_t tiles_m = (p.M + big::BM - 1) / big::BM;
    const uint32_t tiles_n = gated ? (p.H + big::BN / 2 - 1) / (big::BN / 2) : (p.N + big::BN - 1) / big::BN;
    const size_t lds = (size_t)kBigStages * big::Cfg<kBigBK, kBigStages>::STAGE_BYTES;
    auto kern = gated ? gemm_big_kernel<true, kBigBK, kBigStages> : gemm_big_kernel<false, kBigBK, kBigStages>;
    static PerDevice lds_once[2];
    hipError_t e = set_max_lds(lds_once[gated], (const void*)kern, (int)lds);
    if (e != hipSuccess) return e;
    // one workgroup per CU at most (the kernel walks its tiles)
    int cus = 0;
    if ((e = device_cus(&cus)) != hipSuccess) return e;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t grid = std::min<uint32_t>(tiles, (uint32_t)cus);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, s, p);
    return hipGetLastError();
}

}   // namespace vai_dev
