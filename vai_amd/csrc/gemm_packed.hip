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
// 1 KB of contiguous memory: lane l reads bytes l*16 .. l*16+15. Blocks past
// N (or H) are zero.
//
// Wave layout 1 x 4: wave w owns all 256 rows of the tile and logical
// columns w*64 .. w*64+63 (8 x 2 fragments of 32x32, 256 fp32 accumulators
// per lane in AGPRs). No wave loads what another loads, and every wave reads
// all eight A fragments of a substep from LDS. For gated weights a wave's two
// column fragments are the 32 gate rows and the 32 matching up rows of its
// 32 outputs.
//
// Schedule (per workgroup, 4 waves, one workgroup per CU, persistent):
//  * A: 256x64 fp16 stages (32 KB) copied global -> LDS (buffer_load ... lds)
//    into a ring of 3 slots, two stages ahead; swizzled like gemm_big.hip.
//  * B: each wave loads its 64 columns x 64 k (8 KB) of stage g + 1 into
//    VGPRs during stage g (8 x 1 KB loads), double buffered.
//  * Per stage and wave: 64 MFMAs, 32 LDS fragment reads, 8 LDS copies, 8
//    global loads; one s_barrier per stage.
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"
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
constexpr int B_LOADS = 8;                 // 16-byte fragment loads per lane per stage
constexpr size_t LDS_BYTES = (size_t)SLOTS * A_STAGE;
}

// W row of logical block lb, row r (0xFFFFFFFF when the block row is padding).
__host__ __device__ inline uint32_t packed_src_row(uint32_t lb, uint32_t r, bool gated, uint32_t H, uint32_t N)
{
    if (!gated) {
        const uint32_t row = lb * 32 + r;
        return row < N ? row : 0xFFFFFFFFu;
    }
    // tile t = lb / 8 covers outputs t*128.., wave w = (lb / 2) % 4 outputs
    // t*128 + w*32.., block lb % 2: 0 = gate rows, 1 = up rows
    const uint32_t t = lb / 8, w = (lb / 2) % 4, j = lb % 2;
    const uint32_t jo = t * 128 + w * 32 + r;
    return jo < H ? jo + (j ? H : 0u) : 0xFFFFFFFFu;
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

// ---- decode GEMV over the packed weight (M <= 8) ----------------------------
// In the packed layout one 32x32x16 MFMA B fragment (32 rows x 16 k) is 1 KB
// of contiguous memory, so the GEMV reads W in whole 1 KB pieces per load
// instruction and the matrix cores take the products: X is the A operand
// (rows >= M read as zero), each output row of W a column. A workgroup of 16
// waves owns one 32-row block; its K/16 fragments are split over the waves,
// each issuing all of its (up to 8) fragment loads before the X loads and the
// MFMAs, and the 16 partial 8x32 results meet in LDS. (Loading the MFMA layout
// from an unpacked W reads 16 rows x 64 B per instruction and measured about
// 1 us slower per 32 MiB; staging unpacked rows through LDS, 1.5-2 us.)
constexpr int GV_WAVES = 16, GV_FR = 8;

// EXACT: K/16 is a multiple of GV_WAVES * GV_FR, so every wave runs whole
// passes of GV_FR fragments with no guards (straight-line loads, per-fragment
// waits). Rows past M read X row 0 (a valid address); their results are
// never stored. A padding block (no row of W) skips its passes but still
// meets the barrier: no branch ahead of the loads, so the compiler fetches
// the kernel arguments in one batch.
template <bool EXACT>
__global__ __launch_bounds__(1024) void gemv_packed_kernel(SlabParams a, const half8* __restrict__ packed,
                                                           uint32_t H, int gated, float* __restrict__ ygated)
{
    __shared__ float part[GV_WAVES][8][33];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lb = blockIdx.x, K = a.K, M = a.M, N = a.N;
    // the arguments the loads need, fetched in one batch at entry (the
    // compiler otherwise fetches each behind the branch that first uses it)
    asm volatile("" ::"s"(packed), "s"(a.in), "s"(K), "s"(M), "s"(N), "s"(H), "s"(gated));
    const bool live = packed_src_row(lb, 0, gated != 0, H, N) != 0xFFFFFFFFu;   // uniform
    const uint32_t frags = K / 16, per = (frags + GV_WAVES - 1) / GV_WAVES;
    const uint32_t f0 = wave * per, f1 = live ? std::min(frags, f0 + per) : f0;
    const half8* wp = packed + (size_t)lb * frags * 64 + lane;   // fragment f at wp + 64 f
    const int xm = lane & 31, xg = lane >> 5;
    const half_t* xp = (const half_t*)a.in + (size_t)((uint32_t)xm < M ? xm : 0) * K + xg * 8;
    float16v acc0 = (float16v)0.f, acc1 = (float16v)0.f;
    for (uint32_t fb = f0; fb < f1; fb += GV_FR) {
        half8 wv[GV_FR], xv[GV_FR];
#pragma unroll
        for (int i = 0; i < GV_FR; ++i) {
            wv[i] = (EXACT || fb + i < f1) ? __builtin_nontemporal_load(wp + (size_t)(fb + i) * 64) : (half8)0;
            xv[i] = (EXACT || fb + i < f1) ? *(const half8*)(xp + (size_t)(fb + i) * 16) : (half8)0;
        }
        // every load of the pass in flight before the first MFMA (left alone,
        // the scheduler trades that for registers: load, wait, MFMA, ...)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < GV_FR; i += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xv[i], wv[i], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(xv[i + 1], wv[i + 1], acc1, 0, 0, 0);
        }
    }
    // rows 0..7 of the 32x32 result: register rr < 4 holds row rr + 4 (lane / 32), column lane % 32
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) part[wave][rr + 4 * xg][xm] = acc0[rr] + acc1[rr];
    __syncthreads();
    if (threadIdx.x >= 8 * 32) return;
    const uint32_t m = threadIdx.x / 32, n = threadIdx.x % 32;
    const uint32_t row = packed_src_row(lb, n, gated != 0, H, N);
    if (m >= M || row == 0xFFFFFFFFu) return;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < GV_WAVES; ++w) v += part[w][m][n];
    const size_t o = (size_t)m * N + row;
    if (gated) {   // the Linear output with its bias; the gating pass reads it
        ygated[o] = v + (a.bias ? ld(a.bias, a.b_dtype, a.bias_repeat ? o % a.bias_repeat : o) : 0.f);
        return;
    }
    store_output(OutputSpec{a.out, a.bias, a.residual, a.o_dtype, a.b_dtype, a.bias_repeat, a.residual_repeat,
                            a.epilogue, a.residual_order, a.scalar_scale},
                 o, v);
}

hipError_t gemv_packed_launch(const SlabParams& a, const void* packed, bool gated, float* ygated, hipStream_t s)
{
    const uint32_t H = gated ? a.N / 2 : 0;
    const uint32_t blocks = packed_blocks(a.N, H, gated);
    auto kern = (a.K / 16) % (GV_WAVES * GV_FR) == 0 ? gemv_packed_kernel<true> : gemv_packed_kernel<false>;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * GV_WAVES), 0, s, a, (const half8*)packed, H, gated ? 1 : 0,
                       ygated);
    return hipGetLastError();
}

// Keeps a substep's MFMA operands allocated until all of its MFMAs have
// issued: the fragment loads interleaved with those MFMAs then cannot be
// given a register an issued-but-not-started MFMA still has to read.
__device__ __forceinline__ void keep_operands(const half8 (&a)[8], const half8 (&b)[2])
{
    asm volatile("" ::"v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
                 "v"(b[0]), "v"(b[1]));
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

// ---- epilogue for the 1 x 4 layout ----------------------------------------
// D[i][j] of a 32x32 fragment sits in lane j + 32*((i/4)%2), register
// (i%4) + 4*(i/8): per register a half-wave holds 32 consecutive columns of
// one row. Row of fragment i, register rr: i*32 + (rr%4) + 8*(rr/4) + 4*fk.

// Bias of this lane's columns, loaded before the tile's K loop (a load still
// in flight at the epilogue would make the compiler wait for every copy
// issued after it). Gated: [0] gate bias, [1] up bias of the lane's output.
template <bool GATED>
__device__ __forceinline__ void pk_col_bias(const GemmParams& p, uint32_t tn, int w, int fr, float (&cb)[2])
{
    cb[0] = cb[1] = 0.f;
    if constexpr (GATED) {
        const uint32_t H = p.H, col = tn * 128 + w * 32 + fr;
        if (p.bias && col < H) {
            cb[0] = ld(p.bias, p.bias_dtype, col);
            cb[1] = ld(p.bias, p.bias_dtype, H + col);
        }
    } else {
        const uint32_t N = p.N, col0 = tn * 256 + w * 64 + fr;
        if (p.bias && p.bias_repeat == N) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (col0 + j * 32 < N) cb[j] = ld(p.bias, p.bias_dtype, col0 + j * 32);
        }
    }
}

// Fast path (fp32 output, the tile's columns inside the output, the bias one
// row): buffer stores from a resource that starts at the tile's first row and
// ends at the output's last row, so rows past M are dropped by the bounds
// check; the common activations are compile-time (6 = the runtime kind).
template <bool GATED, uint32_t EPI, bool F16OUT = false>
__device__ __forceinline__ void pk_store_fast(const GemmParams& p, float16v (&acc)[8][2], const float (&cb)[2],
                                              uint32_t tm, uint32_t tn, int w, int fr, int fk)
{
    const uint32_t ld_out = GATED ? p.H : p.N;
    const uint32_t rows_left = p.M - tm * 256;
    constexpr uint32_t ES = F16OUT ? 2 : 4;   // output element bytes
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((char*)p.C + (size_t)tm * 256 * ld_out * ES), (short)0,
        (int)std::min<size_t>((size_t)rows_left * ld_out * ES, 0x7FFFFFFF), 0x00020000);
    const uint32_t col0 = GATED ? tn * 128 + w * 32 + fr : tn * 256 + w * 64 + fr;
    const uint32_t lane_off = (4 * fk * ld_out + col0) * ES;
    const uint32_t row_bytes = ld_out * ES;
    const uint32_t epi = p.epilogue;
    const float s = p.scalar_scale;
    constexpr int JN = GATED ? 1 : 2;
    static_for<8>([&](auto I) __attribute__((always_inline)) {
        static_for<JN>([&](auto J) __attribute__((always_inline)) {
            constexpr int i = I, j = J;
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int rr = R;
                float v;
                if constexpr (GATED)
                    v = act<EPI>(agpr_read(acc[i][0][rr]) + cb[0], epi) * (agpr_read(acc[i][1][rr]) + cb[1]);
                else
                    v = s * act<EPI>(agpr_read(acc[i][j][rr]) + cb[j], epi);
                const uint32_t voff = lane_off + (uint32_t)(i * 32 + (rr % 4) + 8 * (rr / 4)) * row_bytes + j * 32 * ES;
                if constexpr (F16OUT)
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (half_t)v), out, (int)voff, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out, (int)voff, 0, 0);
            });
            __builtin_amdgcn_sched_barrier(0);   // 16 outputs at a time: few live registers
        });
    });
}

template <bool GATED>
__device__ __forceinline__ void pk_store_any(const GemmParams& p, float16v (&acc)[8][2], const float (&cb)[2],
                                             uint32_t tm, uint32_t tn, int w, int fr, int fk)
{
    const uint32_t M = p.M, row0 = tm * 256 + 4 * fk;
    if constexpr (GATED) {
        const uint32_t H = p.H, col = tn * 128 + w * 32 + fr;
        static_for<8>([&](auto I) __attribute__((always_inline)) {
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int i = I, rr = R;
                const uint32_t row = row0 + i * 32 + (rr % 4) + 8 * (rr / 4);
                const float g = agpr_read(acc[i][0][rr]), u = agpr_read(acc[i][1][rr]);
                if (row < M && col < H)
                    st(p.C, p.c_dtype, (size_t)row * H + col, epilogue(g + cb[0], p.epilogue) * (u + cb[1]));
            });
            __builtin_amdgcn_sched_barrier(0);
        });
    } else {
        const uint32_t N = p.N, col0 = tn * 256 + w * 64 + fr;
        static_for<8>([&](auto I) __attribute__((always_inline)) {
            static_for<2>([&](auto J) __attribute__((always_inline)) {
                constexpr int i = I, j = J;
                const uint32_t col = col0 + j * 32;
                static_for<16>([&](auto R) __attribute__((always_inline)) {
                    constexpr int rr = R;
                    const uint32_t row = row0 + i * 32 + (rr % 4) + 8 * (rr / 4);
                    const float a = agpr_read(acc[i][j][rr]);
                    if (row < M && col < N) {
                        const size_t o = (size_t)row * N + col;
                        // a bias other than one [N] row: read per element
                        const float bb = (p.bias && p.bias_repeat != N)
                            ? ld(p.bias, p.bias_dtype, p.bias_repeat ? o % p.bias_repeat : o) : cb[j];
                        const float res = p.residual
                            ? ld(p.residual, p.residual_dtype, p.residual_repeat ? o % p.residual_repeat : o) : 0.f;
                        st(p.C, p.c_dtype, o, finish(a + bb, res, p.epilogue, p.residual_order, p.scalar_scale));
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    }
}

template <bool GATED>
__device__ __forceinline__ void pk_store(const GemmParams& p, float16v (&acc)[8][2], const float (&cb)[2],
                                         uint32_t tm, uint32_t tn, int w, int fr, int fk)
{
    __builtin_amdgcn_sched_barrier(0);
    // Every accumulator passes through an (empty) asm first, so no MFMA can
    // be moved past this point into the epilogue's blocks; the s_nops then
    // give the last MFMA its result-to-read distance (the agpr_read asm is
    // opaque to the compiler's hazard checks).
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) asm volatile("" : "+a"(acc[i][j]));
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");   // MFMA result -> VALU read distance
    const bool cols_in = GATED ? tn * 128 + 128 <= p.H : tn * 256 + 256 <= p.N;
    const bool plain = GATED || (!p.residual && (!p.bias || p.bias_repeat == p.N));   // cb holds the bias
    if (cols_in && plain && p.c_dtype == DT_F32) {
        switch (p.epilogue) {
        case 4: pk_store_fast<GATED, 4>(p, acc, cb, tm, tn, w, fr, fk); break;   // SiLU
        case 3: pk_store_fast<GATED, 3>(p, acc, cb, tm, tn, w, fr, fk); break;   // GELU-tanh
        case 0: pk_store_fast<GATED, 0>(p, acc, cb, tm, tn, w, fr, fk); break;
        default: pk_store_fast<GATED, 6>(p, acc, cb, tm, tn, w, fr, fk); break;
        }
    } else if (cols_in && plain && p.c_dtype == DT_F16) {
        switch (p.epilogue) {
        case 4: pk_store_fast<GATED, 4, true>(p, acc, cb, tm, tn, w, fr, fk); break;   // SiLU
        case 0: pk_store_fast<GATED, 0, true>(p, acc, cb, tm, tn, w, fr, fk); break;
        default: pk_store_fast<GATED, 6, true>(p, acc, cb, tm, tn, w, fr, fk); break;
        }
    } else {
        pk_store_any<GATED>(p, acc, cb, tm, tn, w, fr, fk);
    }
}

// ---- the kernel ------------------------------------------------------------
template <bool GATED>
__global__ __launch_bounds__(256, 1) void gemm_packed_kernel(GemmParams p, const half_t* __restrict__ wp)
{
    using namespace pk;
    extern __shared__ half8 lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 31, fk = lane >> 5;
    const uint32_t M = p.M, K = p.K, G = gridDim.x;
    const TileOrder order = TileOrder::make((M + BM - 1) / BM, GATED ? (p.H + 127) / 128 : (p.N + BN - 1) / BN, G);
    const uint32_t total = order.tiles_m * order.tiles_n;
    // Work units: (tile, K split). With p.splits = S > 1 (not gated) unit
    // U covers tile U % total over K steps [s*ktiles, (s+1)*ktiles), s =
    // U / total, and writes its raw fp32 sums to partial plane s at p.C; a
    // reduce pass applies the epilogue.
    const uint32_t S = GATED ? 1u : p.splits, units = total * S;
    const int ktiles = (int)(K / S / BK);   // per unit: even, >= 4
    // (a division expands to VALU code: read it back as the scalar it is)
    const int my_tiles = __builtin_amdgcn_readfirstlane((int)((units - blockIdx.x + G - 1) / G));
    GemmParams up = p;   // the parameters a unit's epilogue sees
    if (S > 1) {
        up.bias = nullptr;
        up.residual = nullptr;
        up.epilogue = 0;
        up.scalar_scale = 1.f;
        up.c_dtype = DT_F32;
    }

    // A stream position: the unit's tile (tm, tn), its first K step kb and
    // the K step kt within the unit. The stages a workgroup runs are its
    // units' K steps back to back; copies past the last stage repeat it
    // (harmless, and the copy counts stay fixed).
    struct Pos { uint32_t tm, tn; int kt; int kb; uint32_t split; };

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
        // The resource starts at the tile's first row and ends at A's last
        // row: rows past M are out of bounds (read as zero) through the
        // per-lane offset alone, whatever the scalar offset does.
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const half_t*)p.A + (size_t)at.tm * BM * K), (short)0, (int)((M - at.tm * BM) * K * 2), 0x00020000);
        LDS_AS char* dst = lds_base + (g % SLOTS) * A_STAGE + wave * A_LOADS * 1024;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)(dst + i * 1024), 16, (int)voff[i],
                                                     (int)((at.kb + at.kt) * BK * 2), 0, 0);
    };

    // A fragments of substep ks of stage g: rows i*32 + fr share the swizzle
    // term, so the eight fragments sit at immediate offsets.
    static_assert((32 / RPW) % CH == 0, "fragment rows share the swizzle");
    const int swz = (fr / RPW) % CH;
    auto read_a = [&](int g, int ks, half8 (&af)[8]) __attribute__((always_inline)) {
        const int ch = (ks * 2 + fk) ^ swz;
        LDS_AS const char* a = lds_base + (g % SLOTS) * A_STAGE + (fr * CH + ch) * 16;
#pragma unroll
        for (int i = 0; i < 8; ++i) af[i] = *(LDS_AS const half8*)(a + i * 32 * CH * 16);
    };

    // B fragments of stage `at`, substep q: fragment j is 1 KB at block
    // tn*8 + wave*2 + j, chunk kt*8 + 2q; lane l reads its 16 bytes at l*16.
    const size_t blk = (size_t)K * 64;

    auto mfma_rows = [&](float16v (&acc)[8][2], const half8 (&af)[8], const half8 (&bq)[2], int i0, int i1)
        __attribute__((always_inline)) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bq[j], acc[i][j], 0, 0, 0);
    };

    half8 fa[2][8];
    half8 fb0[4][2], fb1[4][2];

    auto load_b = [&](struct Pos at, half8 (&fb)[4][2], int qq) __attribute__((always_inline)) {
        const char* base =
            (const char*)wp + (size_t)(at.tn * 8 + wave * 2) * blk + (size_t)(at.kb + at.kt) * 4096 + qq * 1024 +
            lane * 16;
#pragma unroll
        for (int j = 0; j < 2; ++j) fb[qq][j] = *(const half8*)(base + j * blk);
    };

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

    // One stage: MFMAs on (fa, cur) while the next stage's B loads into nxt
    // and the next substep's A fragments come out of LDS.
    auto stage = [&](int g, Pos here, Pos next, bool has_next, float16v (&acc)[8][2], half8 (&cur)[4][2],
                     half8 (&nxt)[4][2]) __attribute__((always_inline)) {
        const Pos b_at = ahead(here, next, has_next, 1);
        static_for<4>([&](auto Q) __attribute__((always_inline)) {
            constexpr int q = Q, c = q & 1, n = c ^ 1;
            if constexpr (q < 3) {
                // substep 2 also loads substep 3's B, so that every B load of
                // the stage is a substep old at the stage-end wait
                load_b(b_at, nxt, q);
                if constexpr (q == 2) load_b(b_at, nxt, 3);
                read_a(g, q + 1, fa[n]);
                mfma_rows(acc, fa[c], cur[q], 0, 8);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read (A)
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (u < (q == 2 ? 4 : 2)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load (B)
                }
                __builtin_amdgcn_sched_barrier(0);
                keep_operands(fa[c], cur[q]);
            } else {
                mfma_rows(acc, fa[c], cur[q], 0, 4);
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_barrier(0);
                pk_wait_lgkmcnt0();                              // this wave's reads of slot g are done
                // A(g+1) landed. Only the A(g+2) copies may still be in
                // flight: the count relies on the LDS copies completing in
                // order among themselves, never on their order relative to
                // the B loads into VGPRs or the epilogue's stores.
                pk_wait_vmcnt<A_LOADS>();
                __builtin_amdgcn_s_barrier();
                issue_a(g + SLOTS, ahead(here, next, has_next, SLOTS));
                read_a(g + 1, 0, fa[n]);
                mfma_rows(acc, fa[c], cur[q], 4, 8);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
                keep_operands(fa[c], cur[q]);
            }
        });
    };

    // Unit r of this workgroup (uniform: the divisions expand to VALU code,
    // so the results are read back as scalars).
    auto tile_pos = [&](int r) __attribute__((always_inline)) {
        const uint32_t U = blockIdx.x + (uint32_t)r * G;
        const uint32_t split = (uint32_t)__builtin_amdgcn_readfirstlane(U / total);
        uint32_t tm, tn;
        order.of(U - split * total, tm, tn);
        return Pos{(uint32_t)__builtin_amdgcn_readfirstlane(tm), (uint32_t)__builtin_amdgcn_readfirstlane(tn), 0,
                   (int)split * ktiles, split};
    };

    // Prologue. The issue order A(0), A(1), B(0), A(2) is the order the loop
    // keeps (A(g+1), B(g), A(g+2) are the youngest copies at the top of stage
    // g), so the compiler's waits for B registers come out the same on entry
    // and on the back edge.
    Pos here = tile_pos(0);
    issue_a(0, Pos{here.tm, here.tn, 0, here.kb, here.split});
    issue_a(1, Pos{here.tm, here.tn, 1, here.kb, here.split});
#pragma unroll
    for (int q = 0; q < 4; ++q) load_b(here, fb0, q);
    issue_a(2, Pos{here.tm, here.tn, 2, here.kb, here.split});
    pk_wait_vmcnt<(SLOTS - 1) * A_LOADS>();   // A(0) and B(0) landed; A(1), A(2) may not
    __builtin_amdgcn_s_barrier();
    read_a(0, 0, fa[0]);

    int g = 0;
    for (int r = 0; r < my_tiles; ++r) {
        here = tile_pos(r);
        const bool has_next = r + 1 < my_tiles;
        const Pos next = has_next ? tile_pos(r + 1) : here;
        if (S > 1) up.C = (float*)p.C + (size_t)here.split * M * p.N;
        float cb[2];
        pk_col_bias<GATED>(up, here.tn, wave, fr, cb);
        float16v acc[8][2];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = (float16v)0.f;
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
        pk_store<GATED>(up, acc, cb, here.tm, here.tn, wave, fr, fk);
    }
    pk_wait_vmcnt<0>();   // the clamped copies land before the workgroup retires
}

bool gemm_packed_ok(const GemmParams& p, bool gated)
{
    const uint32_t ncols = gated ? 2 * p.H : p.N;
    // K % 128: the stage loop runs two stages per trip; K >= 256: the copies
    // run at most one tile ahead
    // (split-K, not gated: K / splits obeys the same rules)
    const uint32_t S = p.splits ? p.splits : 1;
    if (S > 1 && (gated || p.K % (S * 128) != 0 || p.K / S < 256)) return false;
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % 128 == 0 && p.K >= 256 && p.batch == 1 &&
           (size_t)p.M * p.K * 2 < (1u << 31) && (size_t)((p.M + 255) / 256) * ((ncols + 255) / 256) * S >= 128;
}

hipError_t gemm_packed_launch(const GemmParams& p, const void* packed, bool gated, hipStream_t s)
{
    const uint32_t tiles_m = (p.M + pk::BM - 1) / pk::BM;
    const uint32_t tiles_n = gated ? (p.H + 127) / 128 : (p.N + pk::BN - 1) / pk::BN;
    auto kern = gated ? gemm_packed_kernel<true> : gemm_packed_kernel<false>;
    static PerDevice lds_once[2];
    hipError_t e = set_max_lds(lds_once[gated], (const void*)kern, (int)pk::LDS_BYTES);
    if (e != hipSuccess) return e;
    int cus = 0;
    if ((e = device_cus(&cus)) != hipSuccess) return e;
    const uint32_t units = tiles_m * tiles_n * (gated ? 1u : std::max<uint32_t>(p.splits, 1));
    const uint32_t grid = std::min<uint32_t>(units, (uint32_t)cus);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), pk::LDS_BYTES, s, p, (const half_t*)packed);
    return hipGetLastError();
}

}   // namespace vai_dev
