// scores.hip -- attention scores S = scale * Q K^T with the causal mask, fp16
// Q/K, fp32 S (the Q.K^T stage of /root/reference/vai/shaders/attention.comp:
// 155-182 and attention-fa.comp:581-591; mask rule of common/causal_mask.h).
//
// The work is bound by writing S (4 bytes per score against ~2 flop/byte of
// MFMA work per head-dim element), so the kernel is built around the store:
//  * one workgroup per 128x128 tile (64x64 when a mask applies) of one head,
//    each head's tiles on one XCD when the heads come in multiples of 8;
//    tiles the mask hides entirely are written as -inf and never touch Q, K
//    or the matrix cores; under a plain causal mask over a square S (a
//    multiple of 64) only the tiles on and below the diagonal are launched,
//    and each writes its mirror tile's -inf while its Q/K stages load
//    (config 4: 10.7-11.0 against 11.4-11.6 us with every tile launched);
//  * Q and K rows are copied global->LDS (buffer_load ... lds) in 64-wide
//    head-dim stages, double buffered; 4 waves x (T/2 x T/2 of 32x32x16
//    MFMAs); 64 KB (32 KB) of LDS, so two (four) workgroups share a CU and
//    one's stores overlap the others' loads (measured on MI355X: one
//    workgroup per CU with all of head_dim in flight is 40% slower, 32-wide
//    stages x 4 is 7% slower);
//  * the accumulators are written straight from registers (two 128-byte row
//    segments per non-temporal store instruction); tiles the mask cuts
//    through select -inf per output with 32-bit tile-relative compares, and
//    only tiles at the edges of S test bounds per output.
#include <algorithm>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

// cache policy bits of the buffer store builtins: 2 = non-temporal (S is
// written once and read by the next kernel, not by this one)
constexpr int kNonTemporal = 2;

namespace sc {
constexpr int BK = 64, CH = BK / 8, RPW = 16 / CH;             // stage depth, chunks per row
constexpr int NS = 2;                                          // double buffer
template <int T> struct Tile {
    static constexpr int WF = T / 64;                          // 32x32 fragments per wave, each way
    static constexpr int SLAB = T * BK * 2;                    // one operand, one stage
    static constexpr int STAGE = 2 * SLAB;                     // Q + K
    static constexpr int LOADS = STAGE / (4 * 1024);           // 1 KB copies per wave per stage
    static constexpr int LDS_BYTES = NS * STAGE;
};
__device__ __forceinline__ int slot(int row, int chunk) { return row * CH + (chunk ^ ((row / RPW) % CH)); }
}

template <int N>
__device__ __forceinline__ void sc_wait_vmcnt()
{
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// TRI (square causal scores, Tq == Tkv a multiple of T, no window or block
// list): the grid holds only the n (n + 1) / 2 tiles on and below the
// diagonal, and each tile below it first stores the -inf of its mirror tile
// above the diagonal, while its own Q/K stages are on their way.
template <int T, bool TRI = false>
__global__ __launch_bounds__(256, T == 128 ? 2 : (TRI ? 5 : 4)) void scores_kernel(GemmParams p)
{
    using namespace sc;
    constexpr int WF = Tile<T>::WF, STAGE = Tile<T>::STAGE, LOADS = Tile<T>::LOADS, HT = T / 2;
    extern __shared__ half8 lds[];
    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, fr = lane & 31, fk = lane >> 5;
    // Workgroup w runs on XCD w % 8. With a multiple of 8 batch entries
    // (heads), entry z's tiles go to XCD z % 8 only (w -> entry w % 8 of its
    // group of 8, tile w / 8), so one head's Q and K rows stay in one L2.
    uint32_t tx = blockIdx.x, ty = blockIdx.y, bz = blockIdx.z;
    if (gridDim.z % 8 == 0) {
        const uint32_t nt = gridDim.x * gridDim.y, w = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const uint32_t g = w / (8 * nt), r = w % (8 * nt), tile = r / 8;
        bz = g * 8 + r % 8;
        tx = tile % gridDim.x;
        ty = tile / gridDim.x;
    }
    if constexpr (TRI) {
        // lower-triangle tile k (row by row): row a holds a + 1 tiles
        const uint32_t k = ty * gridDim.x + tx;
        uint32_t a = (uint32_t)((__builtin_sqrtf(8.0f * (float)k + 1.0f) - 1.0f) * 0.5f);
        while (a * (a + 1) / 2 > k) --a;
        while ((a + 1) * (a + 2) / 2 <= k) ++a;
        ty = a;
        tx = k - a * (a + 1) / 2;
    }
    const uint32_t m0 = ty * T, n0 = tx * T;
    const uint32_t M = p.M, N = p.N, K = p.K;
    float* S = (float*)p.C + bz * p.c_batch_stride;

    if constexpr (TRI) {
        if (ty > tx) {
            // the mirror tile (tx, ty): rows above the diagonal block, all
            // hidden; issued before the Q/K copies, so that the waits below,
            // which count younger operations only, never pass on a store
            constexpr int LPR = HT / 4, RPI = 64 / LPR;
            const float4v ninf = (float4v)(-__builtin_inff());
            const uint32_t r0 = tx * T + wm * HT, c = ty * T + wn * HT + (lane % LPR) * 4;
#pragma unroll
            for (int it = 0; it < HT / RPI; ++it)
                __builtin_nontemporal_store(ninf, (float4v*)(S + (size_t)(r0 + it * RPI + lane / LPR) * N + c));
        }
    }

    // Tiles the mask hides entirely: -inf, 16 bytes per lane.
    if constexpr (!TRI) {
        // the tile's rows read at most keys [key_start(first row), key_end(last row))
        const uint32_t last = (m0 + T < M ? m0 + T : M) - 1;
        const bool hidden = (int64_t)n0 >= p.mask.key_end(last) || (int64_t)n0 + T <= p.mask.key_start(m0);
        if (hidden) {
            // each wave fills its (T/2)x(T/2) block, 16 bytes per lane and
            // 1 KB per store instruction; rows past M and columns past N are
            // skipped
            constexpr int LPR = HT / 4, RPI = 64 / LPR;   // lanes per row, rows per instruction
            const float4v ninf = (float4v)(-__builtin_inff());
            const uint32_t r0 = m0 + wm * HT, c = n0 + wn * HT + (lane % LPR) * 4;
            const bool vec = (N % 4) == 0 && c + 3 < N;
            for (int it = 0; it < HT / RPI; ++it) {
                const uint32_t r = r0 + it * RPI + lane / LPR;
                if (r >= M) break;
                if (vec) __builtin_nontemporal_store(ninf, (float4v*)(S + (size_t)r * N + c));
                else for (int e = 0; e < 4; ++e) if (c + e < N) S[(size_t)r * N + c + e] = -__builtin_inff();
            }
            return;
        }
    }

    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)uniform_ptr((const half_t*)p.A + bz * p.a_batch_stride), (short)0, (int)((size_t)M * K * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)uniform_ptr((const half_t*)p.B + (bz / p.b_group) * p.b_batch_stride), (short)0,
        (int)((size_t)N * K * 2), 0x00020000);
    // Copy i of wave w fills stage slots [(w*LOADS + i)*64, +64): Q rows first, then K rows.
    uint32_t off[LOADS];
    bool isk[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int s = (wave * LOADS + i) * 64 + lane;
        // (copies never straddle Q and K, T * CH being a multiple of 64: a
        // wave-uniform test keeps the descriptor choice scalar)
        isk[i] = (wave * LOADS + i) * 64 >= T * CH;
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
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(dst + i * 1024), 16, (int)off[i], kt * BK * 2, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (LDS_AS void*)(dst + i * 1024), 16, (int)off[i], kt * BK * 2, 0, 0);
        }
    };

    float16v acc[WF][WF];
#pragma unroll
    for (int i = 0; i < WF; ++i)
#pragma unroll
        for (int j = 0; j < WF; ++j) acc[i][j] = (float16v)0.f;

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
            half8 af[WF], bf[WF];
#pragma unroll
            for (int i = 0; i < WF; ++i) af[i] = q[slot(wm * HT + i * 32 + fr, ch)];
#pragma unroll
            for (int j = 0; j < WF; ++j) bf[j] = k[slot(wn * HT + j * 32 + fr, ch)];
#pragma unroll
            for (int i = 0; i < WF; ++i)
#pragma unroll
                for (int j = 0; j < WF; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + NS < ktiles) {
            // every wave is done reading this slot before it is refilled
            __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
            __builtin_amdgcn_s_barrier();
            issue(kt + NS);
        }
    }
    // Epilogue straight from the accumulators. D[i][j] of a fragment sits in
    // lane j + 32*((i/4)%2), register (i%4) + 4*(i/8): per register a
    // half-wave holds 32 consecutive columns of one row, so each store writes
    // two 128-byte row segments. Tiles the mask does not touch and that lie
    // inside S (almost all) store scale * acc through a buffer resource with
    // no per-output tests; the others apply the mask rule per output.
    const int64_t q0 = (int64_t)m0 + p.causal_offset;            // query position of the tile's row 0
    const bool any_mask = (p.causal && (int64_t)n0 + T - 1 > q0) ||
                          (p.span && (int64_t)n0 < q0 + T - (int64_t)p.span);
    const float scale = p.scalar_scale;
    const uint32_t rw0 = wm * HT + 4 * fk, cw0 = wn * HT + fr;     // this lane's row / column in the tile
    // A block list (more than one block) takes the checked path below, which
    // reads each row's key bounds from the rule.
    if (m0 + T <= M && n0 + T <= N && p.mask.blocks <= 1) {
        const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(S + (size_t)m0 * N + n0), (short)0, 0x7FFFFFFF, 0x00020000);
        const uint32_t lane_off = (rw0 * N + cw0) * 4;
        // mask rule in tile coordinates: with d = n0 - q0 and (rl, cl) the
        // output's row and column in the tile, causal hides cl - rl > -d;
        // span hides rl >= span - q0 and cl - rl < 1 - span - d
        const int d = (int)((int64_t)n0 - q0), lane_diff = (int)cw0 - (int)rw0;
        const bool causal = p.causal != 0, span = p.span != 0;
        const int span_row = (int)std::max<int64_t>(std::min<int64_t>((int64_t)p.span - q0, 1 << 30), -(1 << 30));
        const int span_lim = 1 - (int)p.span - d;
        static_for<WF>([&](auto I) __attribute__((always_inline)) {
            static_for<WF>([&](auto J) __attribute__((always_inline)) {
                static_for<16>([&](auto R) __attribute__((always_inline)) {
                    constexpr int i = I, j = J, r = R;
                    constexpr int rc = i * 32 + (r % 4) + 8 * (r / 4);   // row offset of this register
                    float v = acc[i][j][r] * scale;
                    if (any_mask) {
                        const int diff = lane_diff + j * 32 - rc;
                        const bool hide = (causal && diff > -d) ||
                                          (span && (int)rw0 + rc >= span_row && diff < span_lim);
                        v = hide ? -__builtin_inff() : v;
                    }
                    const uint32_t voff = lane_off + (uint32_t)rc * N * 4 + j * 128;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out, (int)voff, 0, kNonTemporal);
                });
            });
        });
        return;
    }
    static_for<WF>([&](auto I) __attribute__((always_inline)) {
        static_for<WF>([&](auto J) __attribute__((always_inline)) {
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int i = I, j = J, r = R;
                const uint32_t row = m0 + rw0 + i * 32 + (r % 4) + 8 * (r / 4), col = n0 + cw0 + j * 32;
                if (row < M && col < N) {
                    const bool hide = (int64_t)col >= p.mask.key_end(row) || (int64_t)col < p.mask.key_start(row);
                    S[(size_t)row * N + col] = hide ? -__builtin_inff() : acc[i][j][r] * scale;
                }
            });
        });
    });
}

bool scores_fast_ok(const GemmParams& p)
{
    return p.a_dtype == DT_F16 && p.b_dtype == DT_F16 && p.K % 64 == 0 &&
           (uint64_t)p.M * p.K * 2 < (1ull << 31) && (uint64_t)p.N * p.K * 2 < (1ull << 31) &&
           ((uintptr_t)p.A % 16) == 0 && ((uintptr_t)p.B % 16) == 0;
}

template <int T>
static hipError_t scores_launch_t(const GemmParams& p, hipStream_t s)
{
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)scores_kernel<T>, sc::Tile<T>::LDS_BYTES);
    if (e != hipSuccess) return e;
    dim3 grid((p.N + T - 1) / T, (p.M + T - 1) / T, p.batch);
    hipLaunchKernelGGL(scores_kernel<T>, grid, dim3(256), sc::Tile<T>::LDS_BYTES, s, p);
    return hipGetLastError();
}

static hipError_t scores_launch_tri(const GemmParams& p, hipStream_t s)
{
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)scores_kernel<64, true>, sc::Tile<64>::LDS_BYTES);
    if (e != hipSuccess) return e;
    const uint32_t n = p.M / 64;
    hipLaunchKernelGGL((scores_kernel<64, true>), dim3(n * (n + 1) / 2, 1, p.batch), dim3(256), sc::Tile<64>::LDS_BYTES,
                       s, p);
    return hipGetLastError();
}

// Masked scores use 64x64 tiles: hidden tiles are then finer, and four
// times as many workgroups spread the unevenly sized tiles over the CUs
// (config 4 on MI355X: 12.8 us against 14.1 us with 128x128 tiles); unmasked
// scores keep 128x128 tiles (fewer Q/K re-reads, 12.8 against 13.2 us).
hipError_t scores_launch(const GemmParams& p, hipStream_t s)
{
    if (p.causal && p.mask.blocks == 1 && p.mask.bits == 1 && p.span == 0 && p.mask.span == 0 && p.M == p.N &&
        p.causal_offset == 0 && p.M % 64 == 0)
        return scores_launch_tri(p, s);
    return (p.causal || p.span || p.mask.blocks > 1) ? scores_launch_t<64>(p, s) : scores_launch_t<128>(p, s);
}

}   // namespace vai_dev
