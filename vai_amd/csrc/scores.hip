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
//    multiple of 64) with head dim 64, 128 or 256, the strip form below
//    takes over; for other head dims only the tiles on and below the
//    diagonal are launched, and each writes its mirror tile's -inf while its
//    Q/K stages load (config 4 with Q and K resident, before the strip
//    form: 10.7-11.0 us against 11.4-11.6 with every tile launched);
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

// ---- strip form: plain causal scores over a square S (head dim 64-256) ----
// Workgroup (head, 64-row strip s, column class par of 4) owns the strip's
// 64x64 tiles j = par, par + 4, ..: those right of the diagonal (j > s) are
// hidden and only stored as -inf (first, while the operands load); the
// others are computed. Each wave keeps its 32 query rows of the strip in
// registers for the whole walk (the MFMA A operand, loaded once), so Q is
// read once per strip and class instead of once per tile, and the K tiles
// stream through two LDS slots by buffer_load ... lds (16-byte chunks
// XOR-swizzled by row), the next tile in flight while this one runs. Every
// workgroup stores the same n / 4 tiles whatever its share of the computed
// ones, and at most n / 4 are computed. Config 4 (512 workgroups, two per CU):
// 10.8-10.9 us against 11.2-11.3 for the 64x64-tile grid in the same runs;
// two classes (256 workgroups, up to 8 computed tiles each) 13.4, eight
// (1024, two rounds at two per CU) 14.6, the classes of a CU's two units
// balanced by reversing the second half of the units 11.1-11.2, stores
// without the non-temporal hint 15.7, a fifth wave per workgroup doing every
// load (Q and the K tiles through LDS, so that the four computing waves never
// wait on vmcnt, which on this architecture counts their stores too)
// 10.7-11.1 against 10.7-11.3. Writing S alone in this kernel's store
// patterns (no loads, no MFMAs; 512 workgroups x four 64x64 tiles) takes 6.8
// us with the hidden tiles' 16-byte stores and 7.0-7.2 us with the computed
// tiles' 4-byte stores, against 6.4 us for 32 MiB written in contiguous 16 KB
// runs per wave: the rest of this kernel's time is the longest strips' Q and K
// loads ahead of their stores. Units of at most 3 computed tiles with the
// hidden tiles in units of their own (no loads): 11.1-11.3 against 10.85-11.0
// us; at most 4 computed tiles so, 11.6: a hidden tile is cheapest as the
// store a computing unit issues while its first Q and K tiles load. The
// computed tiles stored 16 bytes per lane after a 4x4 transpose across each
// lane quad (two DPP exchange rounds per register group, 8 rows x 128 bytes
// per store instruction): 12.3-12.6 against 10.7-11.4 us.
template <int D>
__global__ __launch_bounds__(256, 2) void scores_strip_kernel(GemmParams p)
{
    constexpr int T = 64, ROWB = D * 2, CHR = D / 8, KS = D / 16;
    constexpr int TILE = T * ROWB, COPIES = TILE / 4096;   // 1 KB copies per wave per tile
    constexpr int SWZ = CHR >= 16 ? 15 : 7;                 // chunk bits XORed with the row
    extern __shared__ half8 lds[];
    LDS_AS char* lds_base = (LDS_AS char*)(LDS_AS void*)lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, fr = lane & 31, fk = lane >> 5;
    const uint32_t n = p.M / T, N = p.N;   // strips (= tiles per row); S row length
    // workgroup -> (head, unit); a head's units on one XCD when heads come in 8s
    uint32_t bz = blockIdx.z, u = blockIdx.x;
    if (gridDim.z % 8 == 0) {
        const uint32_t nt = gridDim.x, w = blockIdx.x + nt * blockIdx.z;
        const uint32_t g = w / (8 * nt), r = w % (8 * nt);
        bz = g * 8 + r % 8;
        u = r / 8;
    }
    constexpr uint32_t NC = 4;                          // column classes: tiles j = par, par + NC, ..
    const uint32_t s = n - 1 - u / NC, par = u % NC;
    const uint32_t m0 = s * T;
    float* S = (float*)p.C + bz * p.c_batch_stride;
    const half_t* Qh = (const half_t*)p.A + bz * p.a_batch_stride;
    const half_t* Kh = uniform_ptr((const half_t*)p.B + (bz / p.b_group) * p.b_batch_stride);

    // hidden tiles: the wave's 32x32 quadrant, 16 bytes per lane, 8 rows per store
    {
        const float4v ninf = (float4v)(-__builtin_inff());
        const uint32_t r0 = m0 + wm * 32, c = wn * 32 + (lane % 8) * 4;
        for (uint32_t j = par + ((s + NC - par) / NC) * NC; j < n; j += NC)
#pragma unroll
            for (int it = 0; it < 4; ++it)
                __builtin_nontemporal_store(ninf, (float4v*)(S + (size_t)(r0 + it * 8 + lane / 8) * N + j * T + c));
    }
    const uint32_t nc = s >= par ? (s - par) / NC + 1 : 0;   // computed tiles
    if (nc == 0) return;

    // K tile copies: copy i of wave w fills tile bytes [(w*COPIES + i) KB, +1 KB);
    // lane l's 16 bytes land at physical chunk pc of row r, from logical chunk pc ^ (r & SWZ)
    uint32_t coff[COPIES];
#pragma unroll
    for (int i = 0; i < COPIES; ++i) {
        const int byte = (wave * COPIES + i) * 1024 + lane * 16, r = byte / ROWB, pc = (byte % ROWB) / 16;
        coff[i] = (uint32_t)(r * ROWB + (pc ^ (r & SWZ)) * 16);
    }
    auto issue = [&](uint32_t c) __attribute__((always_inline)) {
        const uint32_t key0 = __builtin_amdgcn_readfirstlane((par + NC * c) * T);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(Kh + (size_t)key0 * D), (short)0, TILE, 0x00020000);
        LDS_AS char* dst = lds_base + (c & 1) * TILE + wave * COPIES * 1024;
#pragma unroll
        for (int i = 0; i < COPIES; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(dst + i * 1024), 16, (int)coff[i], 0, 0, 0);
    };

    // the wave's query rows m0 + 32 wm + fr, dims 16 ks + 8 fk (the A operand)
    half8 qf[KS];
    {
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform_ptr(Qh + (size_t)(m0 + wm * 32) * D), (short)0, 32 * ROWB, 0x00020000);
        const uint32_t qoff = (uint32_t)(fr * D + 8 * fk) * 2;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            qf[ks] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(qoff + 32 * ks), 0, 0));
    }
    issue(0);
    if (nc > 1) issue(1);

    // B fragments: key row wn*32 + fr of the tile, logical chunk 2 ks + fk
    const int brow = wn * 32 + fr;
    const float scale = p.scalar_scale;
    const uint32_t rw0 = wm * 32 + 4 * fk, cw0 = wn * 32 + fr;   // the lane's row / column in a tile
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
        (void*)uniform_ptr(S + (size_t)m0 * N), (short)0, 0x7FFFFFFF, 0x00020000);
    for (uint32_t c = 0; c < nc; ++c) {
        // tile c landed in every wave's share (tile c + 1's copies may be in flight)
        if (c + 1 < nc) sc_wait_vmcnt<COPIES>();
        else sc_wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        const LDS_AS char* kt = lds_base + (c & 1) * TILE + brow * ROWB;
        // all of the tile's B fragments read first, then the MFMAs (read one
        // at a time, each MFMA waited out its read's latency)
        half8 bf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) bf[ks] = *(const LDS_AS half8*)(kt + (((2 * ks + fk) ^ (brow & SWZ)) * 16));
        float16v acc = (float16v)0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qf[ks], bf[ks], acc, 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);   // the reads, in order, ...
        __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);   // ... then the MFMAs
        const uint32_t j = par + NC * c;
        if (c + 2 < nc) {
            // every wave is done reading this slot before it is refilled
            __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
            __builtin_amdgcn_s_barrier();
            issue(c + 2);
        }
        // D[i][j] of the 32x32 fragment: lane j + 32 ((i/4) % 2), register
        // (i % 4) + 4 (i / 8); the diagonal tile hides column > row
        const bool diag = j == s;
        const uint32_t lane_off = (rw0 * N + j * T + cw0) * 4;
        static_for<16>([&](auto R) __attribute__((always_inline)) {
            constexpr int r = R, rc = (r % 4) + 8 * (r / 4);
            float v = acc[r] * scale;
            if (diag) v = (int)cw0 > (int)rw0 + rc ? -__builtin_inff() : v;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out,
                                                  (int)(lane_off + (uint32_t)rc * N * 4), 0, kNonTemporal);
        });
    }
}

template <int D>
static hipError_t scores_launch_strip(const GemmParams& p, hipStream_t s)
{
    constexpr int LDS = 2 * 64 * D * 2;
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)scores_strip_kernel<D>, LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(scores_strip_kernel<D>, dim3(4 * (p.M / 64), 1, p.batch), dim3(256), LDS, s, p);
    return hipGetLastError();
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
        p.causal_offset == 0 && p.M % 64 == 0) {
        if (p.K == 256) return scores_launch_strip<256>(p, s);
        if (p.K == 128) return scores_launch_strip<128>(p, s);
        if (p.K == 64) return scores_launch_strip<64>(p, s);
        return scores_launch_tri(p, s);
    }
    return (p.causal || p.span || p.mask.blocks > 1) ? scores_launch_t<64>(p, s) : scores_launch_t<128>(p, s);
}

}   // namespace vai_dev
