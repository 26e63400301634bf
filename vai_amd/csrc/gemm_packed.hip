// gemm_packed.hip -- the prefill GEMM with a pre-packed weight: fp16 x fp16
// -> fp32 accumulate on v_mfma_f32_32x32x16_f16, 256x256 workgroup tiles,
// for the Linear tile path at large M and the fused gate/up projection.
//
// Why a packed weight: with both operands staged in LDS, the copies into LDS
// plus the fragment reads out of it exceed what LDS delivers per MFMA cycle
// on gfx950, and the MFMAs wait on LDS. Here only the activation operand A
// goes through LDS; the weight streams from global memory (L2) straight into
// VGPRs in MFMA fragment order. That needs W in a fragment-major layout,
// prepared once per weight (the reference's Linear prepares its weights once
// too, linear.h:2291-2704):
//
//   logical 32-column block lb, K chunk kc (8 halves), row r of the block:
//     packed[lb][kc][r][0..7] = W[src_row(lb, r)][kc*8 .. kc*8+7]
//
// so one wave's fragment of one 16-wide k substep (32 rows x 2 chunks) is
// 1 KB of contiguous memory: lane l reads bytes l*16 .. l*16+15. Logical
// columns follow the tile layout of tile_store.h (for gated weights each
// 128-column group is 64 gate rows then the 64 matching up rows); blocks past
// N (or H) are zero.
//
// Schedule (per workgroup, 4 waves, one workgroup per CU, persistent):
//  * A: 256x64 fp16 stages (32 KB) copied global -> LDS (buffer_load ... lds)
//    into a ring of 3 slots, two stages ahead; swizzled like gemm_big.hip.
//  * B: each wave loads its 128 columns x 64 k (16 KB) of stage g + 1 into
//    VGPRs at the start of stage g (16 x 1 KB loads), double buffered.
//  * Per stage and wave: 64 MFMAs, 16 LDS fragment reads, 8 LDS copies, 16
//    global loads; one s_barrier per stage.
#include <algorithm>

#include "device_common.h"
#include "kernels.h"
#include "tile_store.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

namespace pk {
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int CH = BK / 8;                 // 16-byte chunks per A slab row
constexpr int RPW = 16 / CH;               // slab rows per 256-byte LDS bank window
constexpr int SLOTS = 3;                   // A ring depth
constexpr int A_STAGE = BM * BK * 2;       // 32 KB
constexpr int A_LOADS = A_STAGE / (4 * 1024);   // 1 KB copies per wave per stage
constexpr int B_LOADS = 16;                // 16-byte fragment loads per lane per stage
constexpr size_t LDS_BYTES = (size_t)SLOTS * A_STAGE;
}

// W row of logical block lb, row r (>= the row count when the block is padding).
__host__ __device__ inline uint32_t packed_src_row(uint32_t lb, uint32_t r, bool gated, uint32_t H, uint32_t N)
{
    if (!gated) {
        const uint32_t row = lb * 32 + r;
        return row < N ? row : 0xFFFFFFFFu;
    }
    const uint32_t t = lb / 8, w = (lb / 4) % 2, j = lb % 4;
    const uint32_t jo = t * 128 + w * 64 + (j & 1) * 32 + r;
    return jo < H ? jo + (j >= 2 ? H : 0u) : 0xFFFFFFFFu;
}

__host__ __device__ inline uint32_t packed_blocks(uint32_t N, uint32_t H, bool gated)
{
    return gated ? (H + 127) / 128 * 8 : (N + 255) / 256 * 8;
}

// One thread per 16-byte chunk of the packed weight.
__global__ __launch_bounds__(256) void pack_linear_weight_kernel(half8* __restrict__ dst, const half_t* __restrict__ w,
                                                                 uint32_t N, uint32_t K, uint32_t H, int gated,
                                                                 uint64_t chunks)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= chunks) return;
    const uint32_t kcs = K / 8;
    const uint32_t r = (uint32_t)(idx % 32);
    const uint64_t rest = idx / 32;
    const uint32_t kc = (uint32_t)(rest % kcs);
    const uint32_t lb = (uint32_t)(rest / kcs);
    const uint32_t row = packed_src_row(lb, r, gated != 0, H, N);
    half8 v = (half8)(half_t)0;
    if (row != 0xFFFFFFFFu) v = *(const half8*)(w + (size_t)row * K + (size_t)kc * 8);
    dst[idx] = v;
}

size_t gemm_packed_weight_bytes(uint32_t N, uint32_t K, uint32_t H, bool gated)
{
    return (size_t)packed_blocks(N, H, gated) * K * 64;
}

hipError_t gemm_pack_weight(void* dst, const void* w, uint32_t N, uint32_t K, uint32_t H, bool gated, hipStream_t s)
{
    const uint64_t chunks = gemm_packed_weight_bytes(N, K, H, gated) / 16;
    const uint64_t blocks = (chunks + 255) / 256;
    hipLaunchKernelGGL(pack_linear_weight_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, (half8*)dst,
                       (const half_t*)w, N, K, H, gated ? 1 : 0, chunks);
    return hipGetLastError();
}

template <int N>
__device__ __forceinline__ void pk_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void pk_wait_lgkmcnt0()
{
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

template <bool GATED>
__global__ __launch_bounds__(256, 1) void gemm_packed_kernel(GemmParams p, const half_t* __restrict__ wp)
{
    using namespace pk;
    extern __shared__ half8 lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fk = lane >> 5;
    const uint32_t M = p.M, K = p.K, G = gridDim.x;
    const TileOrder order = TileOrder::make((M + BM - 1) / BM, GATED ? (p.H + 127) / 128 : (p.N + BN - 1) / BN, G);
    const uint32_t total = order.tiles_m * order.tiles_n;
    const int ktiles = (int)(K / BK);                      // even: the stage loop is unrolled by two
    // (a division expands to VALU code: read it back as the scalar it is)
    const int my_tiles = __builtin_amdgcn_readfirstlane((int)((total - blockIdx.x + G - 1) / G));

    // A stream position: the tile (tm, tn) and K step kt of a stage. The
    // stages a workgroup runs are its tiles' K steps back to back; copies past
    // the last stage repeat it (harmless, and the copy counts stay fixed).
    struct Pos { uint32_t tm, tn; int kt; };
    // A copies: copy i of wave w fills slab slots [(w*A_LOADS + i)*64, +64);
    // slot s holds row s/CH, physical chunk s%CH = logical chunk ^ swizzle.
    uint32_t voff[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int s = (wave * A_LOADS + i) * 64 + lane;
        const int row = s / CH, ch = (s % CH) ^ ((row / RPW) % CH);
        voff[i] = (uint32_t)(row * K + ch * 8) * 2;
    }
    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;

    auto issue_a = [&](int g, Pos at) __attribute__((always_inline)) {
#ifdef PK_NO_A
        if (g >= SLOTS) return;
#endif
        // The resource starts at the tile's first row and ends at A's last
        // row: rows past M are out of bounds (read as zero) through the
        // per-lane offset alone, whatever the scalar offset does.
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const half_t*)p.A + (size_t)at.tm * BM * K), (short)0, (int)((M - at.tm * BM) * K * 2), 0x00020000);
        LDS_AS char* dst = lds_base + (g % SLOTS) * A_STAGE + wave * A_LOADS * 1024;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)(dst + i * 1024), 16, (int)voff[i],
                                                     (int)(at.kt * BK * 2), 0, 0);
    };

    // A fragments of substep ks of stage g: rows wm*128 + i*32 + fr share the
    // swizzle term, so the four fragments sit at immediate offsets.
    static_assert((32 / RPW) % CH == 0, "fragment rows share the swizzle");
    const int swz = (fr / RPW) % CH;
    auto read_a = [&](int g, int ks, half8* af) __attribute__((always_inline)) {
#ifdef PK_NO_LDSREAD
        if (g > 0) return;
#endif
        const int ch = (ks * 2 + fk) ^ swz;
        LDS_AS const char* a = lds_base + (g % SLOTS) * A_STAGE + ((wm * 128 + fr) * CH + ch) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = *(LDS_AS const half8*)(a + i * 32 * CH * 16);
    };

    // B fragments of stage g: fragment (q, j) is 1 KB at block tn*8 + wn*4 + j,
    // chunk kt*8 + 2q; lane l reads its 16 bytes at l*16.
    const size_t blk = (size_t)K * 64;
    auto load_b = [&](Pos at, half8 (&fb)[4][4], int q) __attribute__((always_inline)) {
        const char* base =
            (const char*)wp + (size_t)(at.tn * 8 + wn * 4) * blk + (size_t)at.kt * 4096 + q * 1024 + lane * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[q][j] = *(const half8*)(base + j * blk);
    };

    auto mfma_rows = [&](float16v (&acc)[4][4], const half8* af, const half8 (&bq)[4], int i0, int i1)
        __attribute__((always_inline)) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bq[j], acc[i][j], 0, 0, 0);
    };

    half8 fa[2][4];
    half8 fb0[4][4], fb1[4][4];

    // One stage: MFMAs on (fa, cur) while the next stage's B loads into nxt
    // and the next substep's A fragments come out of LDS.
    // Position d stages after K step kt of the current tile.
    auto ahead = [&](Pos here, Pos next, bool has_next, int d) __attribute__((always_inline)) {
        Pos at = here;
        at.kt = here.kt + d;
        if (at.kt >= ktiles) {
            if (has_next) { at = next; at.kt = here.kt + d - ktiles; }
            else at.kt = ktiles - 1;
        }
        return at;
    };

    auto stage = [&](int g, Pos here, Pos next, bool has_next, float16v (&acc)[4][4], half8 (&cur)[4][4],
                     half8 (&nxt)[4][4]) __attribute__((always_inline)) {
        const Pos b_at = ahead(here, next, has_next, 1);
        static_for<4>([&](auto Q) __attribute__((always_inline)) {
            constexpr int q = Q, c = q & 1, n = c ^ 1;
            if constexpr (q < 3) {
#ifndef PK_NO_B
                load_b(b_at, nxt, q);
#endif
                read_a(g, q + 1, fa[n]);
                mfma_rows(acc, fa[c], cur[q], 0, 4);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load (B)
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read (A)
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                __builtin_amdgcn_sched_barrier(0);
            } else {
#ifndef PK_NO_B
                load_b(b_at, nxt, q);
#endif
                mfma_rows(acc, fa[c], cur[q], 0, 2);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                pk_wait_lgkmcnt0();                              // this wave's reads of slot g are done
                pk_wait_vmcnt<A_LOADS + 2 * B_LOADS>();          // A(g+1) landed: B(g), A(g+2), B(g+1) may not
                __builtin_amdgcn_s_barrier();
                issue_a(g + SLOTS, ahead(here, next, has_next, SLOTS));
                read_a(g + 1, 0, fa[n]);
                mfma_rows(acc, fa[c], cur[q], 2, 4);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 1);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    };

    // Tile r of this workgroup (uniform: the divisions in TileOrder expand to
    // VALU code, so the result is read back as a scalar).
    auto tile_pos = [&](int r) __attribute__((always_inline)) {
        uint32_t tm, tn;
        order.of(blockIdx.x + (uint32_t)r * G, tm, tn);
        return Pos{(uint32_t)__builtin_amdgcn_readfirstlane(tm), (uint32_t)__builtin_amdgcn_readfirstlane(tn), 0};
    };

    // Prologue: A stages 0..2 and B stage 0 of the first tile in flight
    // (ktiles >= 4); wait for A(0).
    // The issue order A(0), A(1), B(0), A(2) is the order the loop keeps
    // (A(g+1), B(g), A(g+2) are the youngest copies at the top of stage g),
    // so the compiler's waits for B registers come out the same on entry and
    // on the back edge.
    Pos here = tile_pos(0);
    issue_a(0, Pos{here.tm, here.tn, 0});
    issue_a(1, Pos{here.tm, here.tn, 1});
#pragma unroll
    for (int q = 0; q < 4; ++q) load_b(here, fb0, q);
#ifdef PK_NO_B
    for (int q = 0; q < 4; ++q) load_b(here, fb1, q);
#endif
    issue_a(2, Pos{here.tm, here.tn, 2});
    pk_wait_vmcnt<(SLOTS - 1) * A_LOADS + B_LOADS>();
    __builtin_amdgcn_s_barrier();
    read_a(0, 0, fa[0]);

    int g = 0;
    for (int r = 0; r < my_tiles; ++r) {
        here = tile_pos(r);
        const bool has_next = r + 1 < my_tiles;
        const Pos next = has_next ? tile_pos(r + 1) : here;
        float cb[4];
        tile_col_bias<GATED>(p, here.tn, wn, fr, cb);
        float16v acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = (float16v)0.f;
        // The tile's first and last stages are peeled: the inner loop's header
        // then only joins states with the same copies in flight, and the
        // compiler's waits for the B registers stay at their steady-state
        // counts (entering it from the previous tile's stores would make
        // them wait for the copies just issued).
        here.kt = 0;
        stage(g, here, next, has_next, acc, fb0, fb1);
        ++g;
        for (int kt = 1; kt + 1 < ktiles; kt += 2, g += 2) {
            here.kt = kt;
            stage(g, here, next, has_next, acc, fb1, fb0);
            here.kt = kt + 1;
            stage(g + 1, here, next, has_next, acc, fb0, fb1);
        }
        here.kt = ktiles - 1;
        stage(g, here, next, has_next, acc, fb1, fb0);
        ++g;
#ifdef PK_NO_EPI
        if (p.M == 12345)
#endif
        tile_store<GATED>(p, acc, cb, here.tm, here.tn, wm, wn, fr, fk);
    }
    pk_wait_vmcnt<0>();   // the clamped copies land before the workgroup retires
}

bool gemm_packed_ok(const GemmParams& p, bool gated)
{
    const uint32_t ncols = gated ? 2 * p.H : p.N;
    // K % 128: the stage loop runs two stages per trip; K >= 256: the copies
    // run at most one tile ahead
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % 128 == 0 && p.K >= 256 && p.splits == 1 &&
           p.batch == 1 &&
           (size_t)p.M * p.K * 2 < (1u << 31) &&
           (size_t)((p.M + 255) / 256) * ((ncols + 255) / 256) >= 128;
}

hipError_t gemm_packed_launch(const GemmParams& p, const void* packed, bool gated, hipStream_t s)
{
    const uint32_t tiles_m = (p.M + pk::BM - 1) / pk::BM;
    const uint32_t tiles_n = gated ? (p.H + 127) / 128 : (p.N + pk::BN - 1) / pk::BN;
    auto kern = gated ? gemm_packed_kernel<true> : gemm_packed_kernel<false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[gated]) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)pk::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set[gated] = true;
    }
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!cus[dev]) {
        hipError_t e = hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
    }
    const uint32_t grid = std::min<uint32_t>(tiles_m * tiles_n, (uint32_t)cus[dev]);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), pk::LDS_BYTES, s, p, (const half_t*)packed);
    return hipGetLastError();
}

}   // namespace vai_dev
