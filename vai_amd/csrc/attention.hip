// attention.hip -- fused attention forward O = softmax(scale * Q K^T + mask) V
// for fp16 Q/K/V on gfx950 (the role of /root/reference/vai/shaders/
// attention-fa.comp: scores, online softmax and P.V in one pass; the mask
// rule of common/causal_mask.h:25-42; the node at nodes/attention.h:979-1304;
// the key-split merge of attention-fa-reduce.comp).
//
// One workgroup (4 waves) owns 128 query rows of one head, 32 per wave, and
// walks the 64-key tiles the mask leaves visible (or one chunk of them when
// the key range is split over workgroups). Everything runs on
// v_mfma_f32_32x32x16_f16 in transposed form, so that no value moves between
// lanes except for one exchange per row reduction:
//  * S^T = K Q^T: A = 32 keys x 16 head-dim values read from LDS, B = the
//    wave's 32 query rows, held in registers for the whole walk. Lane l gets
//    query l % 32 and 16 keys of each 32-key block (4 (l / 32) + {0-3, 8-11,
//    16-19, 24-27}); with its partner lane l ^ 32 it holds the query's whole
//    tile row, so the online softmax (running max m and sum l in fp32, exp2
//    with scale * log2(e) folded in) needs one exchange per reduction.
//  * O^T += V^T P^T: B = P^T, which is exactly the S^T accumulator layout
//    rounded to fp16 (the fp16 P operand of the reference's P.V stage),
//    taken 8 registers at a time; A = 32 head-dim values x 16 keys of V^T,
//    read from V's row-major LDS tile with ds_read_b64_tr_b16 (4 keys of one
//    column per lane per read) in the key order the P^T registers hold. O^T
//    gives lane l query l % 32 again, so the per-row rescale and the final
//    1/l use the lane's own m and l. O^T lives in accumulation registers,
//    D/32 fragments of 32x32.
//  * K and V tiles (row-major, 16-byte chunks XOR-swizzled by row) are copied
//    global -> LDS by buffer_load ... lds, double buffered: the copies of tile
//    t + 1 are issued during tile t's S^T MFMAs, a few per MFMA group (issued
//    as one burst, the wave stalled about 1,200 cycles on the vector memory
//    path before its next MFMA: 25.9 against 26.4 us per step at config
//    "attn").
// Rows with no visible key give 0.
#include <algorithm>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

namespace fa {
constexpr int NW = 4, QW = 32, BQ = NW * QW, BKV = 64;
template <int D> struct Lds {
    static constexpr int ROWB = D * 2;                  // bytes per K or V row
    static constexpr int CH = D / 8;                    // 16-byte chunks per row
    static constexpr int TILE = BKV * ROWB;             // one operand, one tile
    static constexpr int STAGE = 2 * TILE;              // K then V
    static constexpr int BYTES = 2 * STAGE;             // double buffered
    static constexpr int COPIES = TILE / 1024 / NW;     // 1 KB copies per wave and operand
};
// Physical 16-byte chunk of logical chunk c in row r. LDS serves a 16-byte
// read for 16 lanes per pass from 64 banks (256 bytes), and K / V rows of
// D >= 128 are 256 or 512 bytes long, so every row starts at bank 0. With
// 16 or more chunks per row the low four chunk bits XOR h(r % 16) = f(r % 8)
// + (r & 8), f = 0 2 4 6 1 3 5 7: the 16 rows one K fragment read touches
// per pass (lanes 0-15: rows 0-15 at one logical chunk) land on 16 distinct
// chunks of a 256-byte window, and the four rows each 16-lane group of a
// transposed V^T read touches (two chunks each) on eight distinct chunks.
// Rows of D = 64 (128 bytes, 8 chunks) XOR f(r % 8) in the low three bits.
// The swizzle is its own inverse.
__host__ __device__ constexpr int swz_f(int r) { return 2 * (r & 3) + ((r >> 2) & 1); }
template <int D> __host__ __device__ constexpr int swz(int r, int c)
{
    return D >= 128 ? (c & ~15) | ((c & 15) ^ (swz_f(r & 7) | (r & 8))) : (c & ~7) | ((c & 7) ^ swz_f(r & 7));
}
}

// LDS fragment reads of the main loop, as inline asm. The compiler's wait
// insertion makes its ds_read_b64_tr_b16 builtin wait for every LDS DMA in
// flight (vmcnt(0)), which would hold each tile's V^T reads until the next
// tile's copies have landed, and with no registers to spare at D = 256 it
// sinks prefetched reads down to their MFMAs. The reads below are invisible
// to that pass: fa_lgkm_wait<N> (N = LDS operations issued since the reads
// needed) waits for them, and fa_pin ties each fragment to the wait so that
// its MFMA cannot be scheduled above it. LDS operations complete in order;
// the loop issues no scalar memory loads (which share the counter out of
// order). The compiler's own waits only count more operations than it knows
// of, which makes them stricter.
template <int OFF>
__device__ __forceinline__ half8 lds_read128(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    half8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

// ds_read_b64_tr_b16 (gfx950): per 16-lane group, result lane j element k is
// element j % 4 of the 8 bytes that source lane 4 k + j / 4 points at.
template <int OFF>
__device__ __forceinline__ half4 lds_read_tr16(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    half4 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

// x * a for an accumulator element held in an accumulation register, in
// place: the compiler, given a plain multiply, keeps a VGPR copy of every
// accumulator live across the whole tile loop for the (rare) rescale and
// pays 128 register moves per tile at D = 256.
__device__ __forceinline__ float fa_scale_acc(float x, float a)
{
    float t;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(a));
    return x;
}

// Pairwise tree reductions of 32 values (depth 5 instead of a chain of 31).
__device__ __forceinline__ float fa_tree_max(float (&v)[32])
{
#pragma unroll
    for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) v[i] = fmaxf(v[i], v[i + w]);
    return v[0];
}
__device__ __forceinline__ float fa_tree_sum(float (&v)[32])
{
#pragma unroll
    for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) v[i] += v[i + w];
    return v[0];
}

template <int N>
__device__ __forceinline__ void fa_lgkm_wait()
{
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}

__device__ __forceinline__ void fa_pin(half8& v) { asm volatile("" : "+v"(v)); }

// K fragment of S^T step IDX (key block IDX % 2, head-dim step S = IDX / 2):
// lane (ql, hf) reads key row 32 (IDX % 2) + ql, head-dim values 16 S + 8 hf
// .. +7, i.e. logical chunk c = 2 S + hf. D >= 128: the physical chunk is
// 16 (S / 8) + (((2 (S % 4) + hf) ^ f(ql % 8)) | (8 ((S / 4) % 2) ^ (ql & 8))),
// so the lane part is kaddr[S % 8] = stage + ql ROWB + that chunk without its
// first term, times 16, and the immediate adds 32 (IDX % 2) ROWB + 256 (S / 8).
// D = 64 (S < 4): kaddr[S] with the three-bit swizzle.
template <int D>
constexpr int fa_nk = D >= 128 ? 8 : 4;
template <int D, int IDX>
__device__ __forceinline__ half8 fa_kfrag(const uint32_t (&kaddr)[fa_nk<D>])
{
    constexpr int S = IDX >> 1;
    return lds_read128<32 * (IDX & 1) * fa::Lds<D>::ROWB + (S >> 3) * 256>(kaddr[S & (fa_nk<D> - 1)]);
}

// V^T fragment of key step KK, head-dim block DD: two transposed 8-byte reads
// of keys 16 KK + 8 part + lr (lr = vkey + vrow < 8), head-dim values 32 DD +
// vcol .. +3 (logical chunk c = 4 DD + vcol / 8). The row's swizzle is f(lr)
// plus 8 part, so the physical chunk is 16 (DD / 4) + ((4 (DD % 2) + vcol / 8)
// ^ f(lr)) + 8 ((DD / 2) % 2 ^ part) (D = 64: DD < 2, no bit 3). The lane part
// is vaddr[DD % 2] = stage + lr ROWB + ((4 (DD % 2) + vcol / 8) ^ f(lr)) 16 +
// (vcol % 8) 2; the immediate adds the V tile, (16 KK + 8 part) ROWB and the
// rest of the chunk.
template <int D, int KK, int DD, int PART>
constexpr int fa_voff()
{
    using L = fa::Lds<D>;
    return L::TILE + (16 * KK + 8 * PART) * L::ROWB + (DD >> 2) * 256 +
           (D >= 128 ? (((DD >> 1) & 1) ^ PART) * 128 : (DD >> 1) * 128);
}
template <int D, int KK, int DD>
__device__ __forceinline__ half8 fa_vfrag(const uint32_t (&vaddr)[2])
{
    const half4 h0 = lds_read_tr16<fa_voff<D, KK, DD, 0>()>(vaddr[DD & 1]);
    const half4 h1 = lds_read_tr16<fa_voff<D, KK, DD, 1>()>(vaddr[DD & 1]);
    return __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
}

// The dispatcher deals workgroups out to the 8 XCDs round-robin (linear
// workgroup w runs on XCD w % 8). Logical block of w: XCD x takes the
// contiguous range [x q + min(x, r), ..) of the n blocks (q = n / 8,
// r = n % 8), so that consecutive units -- one head's query tiles and key
// chunks, which read the same K, V and Q -- share one XCD's L2.
__host__ __device__ inline uint32_t fa_xcd_block(uint32_t w, uint32_t n)
{
    const uint32_t q = n / 8, r = n % 8, x = w % 8;
    return x * q + (x < r ? x : r) + w / 8;
}

// The 64-key tiles query tile qt can see: [tb, te), in global key positions
// (a KV cache holding `cached` positions ahead of the new keys).
__host__ __device__ inline void fa_tile_range(const AttnParams& p, uint32_t qt, uint32_t cached, int64_t& tb,
                                              int64_t& te)
{
    const uint32_t q0 = qt * fa::BQ, q1 = std::min<uint32_t>(q0 + fa::BQ, p.tq) - 1;
    const int64_t kend = p.mask.key_end_cached(q1, cached), kbeg = p.mask.key_start_cached(q0, cached);
    tb = kbeg / fa::BKV;
    te = kend <= kbeg ? tb : (kend + fa::BKV - 1) / fa::BKV;
}

// Chunks of query tile qt (at least one, so that every tile writes output).
__host__ __device__ inline uint32_t fa_chunks(const AttnParams& p, uint32_t qt, uint32_t cached)
{
    int64_t tb, te;
    fa_tile_range(p, qt, cached, tb, te);
    const int64_t n = te - tb;   // at most Tkv / 64: a 32-bit division suffices
    return n <= 0 ? 1u : ((uint32_t)n + p.chunk_tiles - 1) / p.chunk_tiles;
}

// K / V tile copies into stage t % 2, through resources that start at the
// tile's first key row and end at the head's last: copy j of this wave fills
// tile bytes [(wave*COPIES + j) KB, +1 KB); rows past Tkv and the padding past
// the head dim read as zero (the range check, which sees the per-lane offset).
template <int D>
__device__ __forceinline__ void fa_issue(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, LDS_AS char* lds,
                                         const uint32_t* coff, int t, int wave)
{
    using L = fa::Lds<D>;
    LDS_AS char* st = lds + (t & 1) * L::STAGE + wave * L::COPIES * 1024;
#pragma unroll
    for (int j = 0; j < L::COPIES; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(st + j * 1024), 16, (int)coff[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < L::COPIES; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (LDS_AS void*)(st + L::TILE + j * 1024), 16, (int)coff[j], 0, 0,
                                                 0);
}

template <int N>
__device__ __forceinline__ void fa_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// D is the padded head dim the LDS tiles and MFMA steps use (64, 128 or
// 256); HD = p.head_dim <= D is the operands' own, a multiple of 8. The
// padding reads as zero (out of the buffers' range), so it adds nothing to
// any score or output; output columns past HD are not stored.
template <int D>
__global__ __launch_bounds__(256, 1) void attention_fwd_kernel(AttnParams p)
{
    using namespace fa;
    using L = Lds<D>;
    const uint32_t HD = p.head_dim, ROWG = HD * 2;   // head dim and K / V row bytes in HBM
    constexpr int KS = D / 16, DF = D / 32;   // 16-wide head-dim steps; 32-wide output fragments
    extern __shared__ half8 fa_lds[];
    LDS_AS char* lds = (LDS_AS char*)(LDS_AS void*)fa_lds;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ql = lane & 31, hf = lane >> 5;   // lane's query (of the wave's 32) and lane half
    const uint32_t Tq = p.tq;
    // keys: positions [0, live); with a cache, its count is read here, at run time
    const uint32_t cached = p.cache_count ? __builtin_amdgcn_readfirstlane(*p.cache_count) : 0u;
    // (a cache without a ring holds kv_rows positions; the caller keeps the
    // count within it, and the clamp keeps a violation inside the buffers)
    const uint32_t KR = p.kv_rows, live = p.ring ? cached + p.tkv : std::min(cached + p.tkv, KR);
    const uint32_t nqt = (Tq + BQ - 1) / BQ;
    // (every argument the set-up needs, fetched in one batch with the
    // workgroup's table entry; left alone, the compiler fetches each behind
    // the branch that first uses it)
    asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.v), "s"(p.tq), "s"(p.tkv), "s"(p.head_dim), "s"(p.hq),
                 "s"(p.hkv), "s"(p.units), "s"(p.q_dtype), "s"(p.chunk_tiles));
    uint32_t unit, h, b, qt, chunk = 0;
    if (p.units != 0) {
        // the plan's table: one entry per workgroup of the 1-D grid
        const uint32_t e0 = p.wg_tab[2 * blockIdx.x], e1 = p.wg_tab[2 * blockIdx.x + 1];
        qt = e0 & 0xFFFF;
        chunk = (e0 >> 16) & 0xFF;
        unit = e1 & 0x3FF;
        h = (e1 >> 10) & 0x3FF;
        b = e1 >> 20;
    } else {
        // Workgroup -> (query tile, head, batch) with one head's query
        // tiles on one XCD (fa_xcd_block), the longest causal walks first.
        const uint32_t X = gridDim.x, HX = X * gridDim.y;
        const uint32_t lb = fa_xcd_block(blockIdx.x + X * (blockIdx.y + gridDim.y * blockIdx.z), HX * gridDim.z);
        unit = lb % X;
        h = (lb / X) % gridDim.y;
        b = lb / HX;
        qt = nqt - 1 - unit;
    }
    qt = __builtin_amdgcn_readfirstlane(qt);
    chunk = __builtin_amdgcn_readfirstlane(chunk);
    const uint32_t q0 = qt * BQ;
    const uint32_t hk = h / (p.hq / p.hkv);
    const uint32_t qsz = p.q_dtype == DT_F32 ? 4 : 2;
    const char* Q = uniform_ptr((const char*)p.q + ((size_t)b * p.hq + h) * Tq * HD * qsz);

    const uint32_t qrow = q0 + wave * QW + ql;

    // The wave's 32 query rows go straight into VGPRs as the B operand of
    // S^T = K Q^T (lane l: query l % 32, head-dim values 16 s + 8 (l / 32)
    // .. +7 of step s; rows past Tq read as zero through the resource's
    // range), issued first; then tile 0's copies. Both are waited for in
    // full (vmcnt(0)) at the top of tile 0; tile 1's copies go out during
    // tile 0's S^T MFMAs.
    // fp32 Q is rounded to fp16 here (the reference's f16 staging of Q,
    // attention-fa.comp:335-342 with stagingF16, as its AMD tiles take).
    half8 qf[KS];
    {
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            (void*)uniform_ptr(Q + (size_t)q0 * HD * qsz), (short)0,
            (int)__builtin_amdgcn_readfirstlane((Tq - q0) * HD * qsz), 0x00020000);
        const uint32_t qel = (wave * QW + ql) * HD + 8 * hf;   // first element of step 0
        if (p.q_dtype == DT_F32) {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint32_t off = 16 * s + 8 * hf < HD ? (qel + 16 * s) * 4 : 0x80000000u;
                const float4v lo = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)off, 0, 0));
                const float4v hi =
                    __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)off, 16, 0));
                const half4 l4 = __builtin_convertvector(lo, half4), h4 = __builtin_convertvector(hi, half4);
                qf[s] = __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        } else {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint32_t off = 16 * s + 8 * hf < HD ? (qel + 16 * s) * 2 : 0x80000000u;
                qf[s] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)off, 0, 0));
            }
        }
    }

    // visible key tiles of the query tile, then this unit's chunk of them
    int64_t tb, te;
    fa_tile_range(p, qt, cached, tb, te);
    if (p.units != 0) {
        const int64_t c0 = tb + (int64_t)chunk * p.chunk_tiles;
        te = std::min<int64_t>(te, c0 + p.chunk_tiles);
        tb = c0;
    }
    const int ntiles = (int)__builtin_amdgcn_readfirstlane((int)std::max<int64_t>(te - tb, 0));

    // K / V tile copies: copy j of this wave fills tile bytes [(wave*COPIES + j) KB, +1 KB);
    // lane l's 16 bytes land at physical chunk pc of row r and come from
    // logical chunk swz<D>(r, pc) of that row (the swizzle is its own inverse).
    // (a chunk past the head dim points at byte 2^31, beyond any range)
    const char* kh0 = uniform_ptr((const char*)((const half_t*)p.k + ((size_t)b * p.hkv + hk) * KR * HD));
    const char* vh0 = uniform_ptr((const char*)((const half_t*)p.v + ((size_t)b * p.hkv + hk) * KR * HD));
    uint32_t coff[L::COPIES];
#pragma unroll
    for (int j = 0; j < L::COPIES; ++j) {
        const int byte = (wave * L::COPIES + j) * 1024 + lane * 16;
        const int r = byte / L::ROWB, pc = (byte % L::ROWB) / 16, lc = swz<D>(r, pc);
        coff[j] = 8u * lc < HD ? (uint32_t)(r * ROWG + lc * 16) : 0x80000000u;
    }
    // Tile t's resources: they start at the tile's first key row and end at
    // the last live key (rows past it read as zero, not as stale cache rows)
    // or the plane's end. A ring holds position j at row j % KR, and KR is a
    // multiple of 64, so no tile wraps. A tile past the unit's last (never
    // copied) gets an empty range.
    const auto rsrc = [&](int t, const char* h) __attribute__((always_inline)) {
        const uint32_t j0 = __builtin_amdgcn_readfirstlane((uint32_t)(tb + t) * BKV);
        const uint32_t row0 = j0 < live ? (p.ring ? j0 % KR : j0) : 0u;
        const uint32_t rows = j0 < live ? std::min(live - j0, KR - row0) : 0u;
        return __builtin_amdgcn_make_buffer_rsrc((void*)(h + (size_t)row0 * ROWG), (short)0, (int)(rows * ROWG),
                                                 0x00020000);
    };
    if (ntiles > 0) fa_issue<D>(rsrc(0, kh0), rsrc(0, vh0), lds, coff, 0, wave);

    // (the rest of the set-up runs while Q and the first tiles load)
    const float sl2 = p.scale * 1.4426950408889634f;   // scores in log2 units
    const uint32_t qclip = qrow < Tq ? qrow : Tq - 1;
    const int64_t row_kend = std::min<int64_t>(p.mask.key_end_cached(qclip, cached), live);
    const int64_t row_kbeg = p.mask.key_start_cached(qclip, cached);
    float m = -__builtin_inff(), l = 0.f;
    float16v o[DF];
#pragma unroll
    for (int d = 0; d < DF; ++d) o[d] = (float16v)0.f;

    // V^T fragment reads: in each 16-lane group g the transposed read gives
    // lane j head-dim value dg + j and 4 consecutive keys; source lane s of
    // the group points at key (base + s / 4), values dg + 4 (s % 4) .. +3.
    const int g = lane >> 4, s16 = lane & 15;
    const int vrow = s16 >> 2, vcol = 16 * (g & 1) + 4 * (s16 & 3);   // + 32 d; key + 16 kk + 8 part
    const int vkey = 4 * (g >> 1);
    // lane parts of the fragment addresses (fa_kfrag, fa_vfrag), stage 0
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(lds);
    constexpr int NK = fa_nk<D>;
    uint32_t kofs[NK], vofs[2];
#pragma unroll
    for (int j = 0; j < NK; ++j)
        kofs[j] = lds0 + ql * L::ROWB +
                  (((2 * (j & 3) + hf) ^ swz_f(ql & 7)) + (D >= 128 ? (8 * (j >> 2)) ^ (ql & 8) : 0)) * 16;
#pragma unroll
    for (int j = 0; j < 2; ++j)
        vofs[j] = lds0 + (vkey + vrow) * L::ROWB + ((4 * j + (vcol >> 3)) ^ swz_f((vkey + vrow) & 7)) * 16 +
                  (vcol & 7) * 2;

    for (int t = 0; t < ntiles; ++t) {
        // Tile t landed in every wave's share: nothing younger is in flight
        // (tile t + 1's copies are issued during tile t's S^T MFMAs, a few
        // per group, so that the wave does not stall on a burst of them).
        fa_wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        const uint32_t sb = (t & 1) * L::STAGE;
        uint32_t kaddr[NK], vaddr[2];
#pragma unroll
        for (int j = 0; j < NK; ++j) kaddr[j] = kofs[j] + sb;
#pragma unroll
        for (int j = 0; j < 2; ++j) vaddr[j] = vofs[j] + sb;
        const int64_t j0 = (tb + t) * BKV;

        // S^T for the tile's two 32-key blocks. Step i of the 2 KS MFMAs is
        // key block i % 2, head-dim step i / 2 (two independent accumulation
        // chains); K fragments are read in groups of G, the next group's
        // reads in flight behind the current group's MFMAs.
        constexpr int NS = 2 * KS, G = NS < 8 ? NS : (D == 256 ? 4 : 8);
        constexpr int OPG = 2 * L::COPIES / (NS / G);   // tile t + 1 copies per MFMA group
        static_assert(OPG * (NS / G) == 2 * L::COPIES, "copies spread evenly over the groups");
        const bool next = t + 1 < ntiles;
        const __amdgpu_buffer_rsrc_t rkn = rsrc(t + 1, kh0), rvn = rsrc(t + 1, vh0);
        LDS_AS char* nst = lds + ((t + 1) & 1) * L::STAGE + wave * L::COPIES * 1024;
        float16v sacc[2] = {(float16v)0.f, (float16v)0.f};
        half8 ka[2][G];
        static_for<G>([&](auto I) __attribute__((always_inline)) { ka[0][I] = fa_kfrag<D, I>(kaddr); });
        static_for<NS / G>([&](auto GI) __attribute__((always_inline)) {
            constexpr int gi = GI, cur = gi & 1;
            if constexpr (gi + 1 < NS / G) {
                static_for<G>([&](auto I) __attribute__((always_inline)) {
                    ka[cur ^ 1][I] = fa_kfrag<D, (gi + 1) * G + I>(kaddr);
                });
                fa_lgkm_wait<G>();
            } else {
                fa_lgkm_wait<0>();
            }
#pragma unroll
            for (int i = 0; i < G; ++i) fa_pin(ka[cur][i]);
#pragma unroll
            for (int i = 0; i < G; ++i) {
                const int idx = gi * G + i;
                sacc[idx & 1] =
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[cur][i], qf[idx >> 1], sacc[idx & 1], 0, 0, 0);
            }
            if (next) {
                static_for<OPG>([&](auto I) __attribute__((always_inline)) {
                    constexpr int op = gi * OPG + I;   // K copies, then V copies
                    constexpr int j = op % L::COPIES;
                    if constexpr (op < L::COPIES)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rkn, (LDS_AS void*)(nst + j * 1024), 16, (int)coff[j],
                                                                 0, 0, 0);
                    else
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rvn, (LDS_AS void*)(nst + L::TILE + j * 1024), 16,
                                                                 (int)coff[j], 0, 0, 0);
                });
            }
        });
        // first key step's V^T fragments, read while the softmax runs (after
        // it at D = 256, where the registers would not hold them)
        constexpr bool VPRE = D < 256;
        half8 vb[2][DF];
        if constexpr (VPRE)
            static_for<DF>([&](auto DD) __attribute__((always_inline)) { vb[0][DD] = fa_vfrag<D, 0, DD>(vaddr); });

        // Online softmax in log2 units (scores x scale x log2 e). Keys of the
        // tile: kb*32 + 8 (rr / 4) + 4 hf + rr % 4. Tiles wholly visible to
        // every row of the wave (the mask's interior) with a non-negative
        // scale take the short path: the max over the raw scores, then
        // 2^(fma(s, scale', -m)). Others scale and mask first.
        const bool fast = __all(j0 >= row_kbeg && j0 + BKV <= row_kend) && sl2 >= 0.f;
        // (reductions as trees: with one wave per SIMD a chain of dependent
        // steps costs its whole latency)
        float tv[32];
        float tmax;
        if (fast) {
#pragma unroll
            for (int i = 0; i < 32; ++i) tv[i] = sacc[i >> 4][i & 15];
            tmax = fa_tree_max(tv) * sl2;
        } else {
            // visible local keys [lo, hi) of the tile, clamped into [-1, 65]
            const int lo = (int)std::min<int64_t>(std::max<int64_t>(row_kbeg - j0, -1), 65);
            const int hi = (int)std::min<int64_t>(std::max<int64_t>(row_kend - j0, -1), 65);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    const int kl = kb * 32 + 8 * (rr >> 2) + 4 * hf + (rr & 3);
                    const float v = (kl >= hi || kl < lo) ? -__builtin_inff() : sacc[kb][rr] * sl2;
                    sacc[kb][rr] = v;
                    tv[kb * 16 + rr] = v;
                }
            tmax = fa_tree_max(tv);
        }
        tmax = swap_max32(tmax);
        // Lazy rescaling: the reference m of a row (the exponent offset of
        // its O and l) moves only when the row max exceeds it by more than
        // 8, and then for the whole wave at once (a uniform branch), so that
        // most tiles skip rescaling O. P = 2^(s - m) then stays below 2^8;
        // fp16 keeps the same relative precision there, and O / l does not
        // depend on m. A row with no visible key yet has m = -inf: its first
        // key moves m; until then 2^(-inf - 0) = 0 keeps P, O and l zero.
        if (__builtin_expect(__any(tmax > m + 8.f), 0)) {
            const float mnew = fmaxf(m, tmax);
            const float alpha = __builtin_amdgcn_exp2f(m - (mnew == -__builtin_inff() ? 0.f : mnew));
            l *= alpha;
            m = mnew;
            // before the unit's first P.V, O is zero in every row: nothing to
            // rescale (every unit's first tile moves m from -inf)
            if (t > 0) {
#pragma unroll
                for (int d = 0; d < DF; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[d][r] = fa_scale_acc(o[d][r], alpha);
            }
        }
        const float mref = m == -__builtin_inff() ? 0.f : m;
        half8 pb[4];   // P^T operand of key step kk: registers 8 (kk % 2) .. +7 of block kk / 2
        if (fast) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][rr], sl2, -mref));
                    tv[kb * 16 + rr] = e;
                    pb[2 * kb + (rr >> 3)][rr & 7] = (half_t)e;
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    const float e = __builtin_amdgcn_exp2f(sacc[kb][rr] - mref);
                    tv[kb * 16 + rr] = e;
                    pb[2 * kb + (rr >> 3)][rr & 7] = (half_t)e;
                }
        }
        {
            const float ps = fa_tree_sum(tv);
            l += swap_sum<32>(ps, ps);
        }

        // O^T += V^T P^T over the tile's four 16-key steps, the next step's
        // V^T fragments in flight behind the current step's MFMAs
        if constexpr (!VPRE)
            static_for<DF>([&](auto DD) __attribute__((always_inline)) { vb[0][DD] = fa_vfrag<D, 0, DD>(vaddr); });
        static_for<4>([&](auto KK) __attribute__((always_inline)) {
            constexpr int kk = KK, cur = kk & 1;
            if constexpr (kk + 1 < 4) {
                static_for<DF>([&](auto DD) __attribute__((always_inline)) {
                    vb[cur ^ 1][DD] = fa_vfrag<D, kk + 1, DD>(vaddr);
                });
                fa_lgkm_wait<(2 * DF < 15 ? 2 * DF : 15)>();
            } else {
                fa_lgkm_wait<0>();
            }
#pragma unroll
            for (int d = 0; d < DF; ++d) fa_pin(vb[cur][d]);
#pragma unroll
            for (int d = 0; d < DF; ++d)
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb[cur][d], pb[kk], o[d], 0, 0, 0);
        });
        // every wave is done reading stage t & 1 before tile t + 2 overwrites it
        __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
    }

    // Output: a partial when the key range is split, else O / l. A partial
    // is (m, l) per row and O: unnormalised in fp32 for fp32 output (as
    // attention-fa-reduce.comp keeps it), O / l in fp16 for fp16 output (a
    // convex combination of V rows, rounded once more before the final fp16
    // rounding; half the bytes through HBM, which bound the split). O^T fragment d gives lane (ql, hf) query ql,
    // head-dim values 32 d + 8 q4 + 4 hf .. +3 of register group q4. The
    // wave's 32 rows are contiguous in either destination, so they go out
    // through LDS: written as fp32 rows (16-byte chunk c of row r at slot
    // c ^ (r % 16), conflict-free both ways), read back as whole rows, stored
    // 64 lanes x 16 contiguous bytes at a time. The last tile's barrier
    // already saw every wave's reads of the K / V stages; each wave then
    // uses its own 32 QW D bytes (the four regions are exactly the stages).
    constexpr int CR = D / 4;    // 16-byte fp32 chunks per row
    constexpr int CH16 = D / 8;  // 16-byte fp16 chunks per row
    const bool partial = p.units != 0, part16 = partial && p.o_dtype == DT_F16;
    const float inv = (partial && !part16) ? 1.0f : (l > 0.f ? 1.0f / l : 0.f);
    const size_t gid = ((size_t)b * p.hq + h) * p.units + unit;
    if (partial && hf == 0) {
        float* wml = p.ws_ml + (gid * BQ + wave * QW + ql) * 2;
        wml[0] = m;
        wml[1] = l;
    }
    // Partials keep the padded rows (D wide, the wave's 32 rows contiguous);
    // the output is token-major [batch, Tq, Hq, HD]: query row r of head h at
    // row (b Tq + r) Hq + h. One loop per destination, so that no branch sits
    // between the LDS reads and the stores.
    const uint32_t wrow0 = q0 + wave * QW;   // the wave's first query row
    if (part16) {
        // fp16 partials go through LDS as fp16 (half the LDS traffic of the
        // fp32 rows): 8-byte pieces, 16-byte chunk 4 d + q4 of the row at
        // slot chunk ^ (r % 16) (r % 8 at D = 64), read back as whole chunks
        LDS_AS half4* obh = (LDS_AS half4*)(lds + wave * QW * D * 4);
        constexpr int SW16 = CH16 >= 16 ? 15 : CH16 - 1;
#pragma unroll
        for (int d = 0; d < DF; ++d)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int c = 4 * d + q4;
                const float4v v = {o[d][4 * q4] * inv, o[d][4 * q4 + 1] * inv, o[d][4 * q4 + 2] * inv,
                                   o[d][4 * q4 + 3] * inv};
                obh[(ql * CH16 + (c ^ (ql & SW16))) * 2 + hf] = __builtin_convertvector(v, half4);
            }
        constexpr int NJ16 = QW * CH16 / 64;   // 16-byte chunks per lane
        const LDS_AS half8* rb = (const LDS_AS half8*)(lds + wave * QW * D * 4);
        half_t* dst = uniform_ptr((half_t*)p.ws_o + (gid * BQ + wave * QW) * D);
#pragma unroll
        for (int j = 0; j < NJ16; ++j) {
            const int e = j * 64 + lane, r = e / CH16, c = e % CH16;
            *(half8*)(dst + r * D + 8 * c) = rb[r * CH16 + (c ^ (r & SW16))];
        }
        return;
    }
    LDS_AS float4v* ob = (LDS_AS float4v*)(lds + wave * QW * D * 4);
#pragma unroll
    for (int d = 0; d < DF; ++d)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int c = 8 * d + 2 * q4 + hf;
            const float4v v = {o[d][4 * q4] * inv, o[d][4 * q4 + 1] * inv, o[d][4 * q4 + 2] * inv,
                               o[d][4 * q4 + 3] * inv};
            ob[ql * CR + (c ^ (ql & 15))] = v;
        }
    constexpr int NJ = QW * CR / 64;         // 16-byte chunks per lane
    if (partial) {
        float* dst = uniform_ptr(p.ws_o + (gid * BQ + wave * QW) * D);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int e = j * 64 + lane, r = e / CR, c = e % CR;
            *(float4v*)(dst + r * D + 4 * c) = ob[r * CR + (c ^ (r & 15))];
        }
    } else {
        const bool o16 = p.o_dtype == DT_F16;
        const size_t rstride = (size_t)p.hq * HD;   // elements from one query row to the next
        const size_t base = (((size_t)b * Tq + wrow0) * p.hq + h) * HD;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int e = j * 64 + lane, r = e / CR, c = e % CR;
            const float4v v = ob[r * CR + (c ^ (r & 15))];
            if (wrow0 + r < Tq && 4u * c < HD) {
                const size_t o0 = base + r * rstride + 4 * c;
                if (o16) *(half4*)((half_t*)p.out + o0) = __builtin_convertvector(v, half4);
                else *(float4v*)((float*)p.out + o0) = v;
            }
        }
    }
}

// Merge of the key chunks of one query tile: O = sum_c 2^(m_c - M) O_c /
// sum_c 2^(m_c - M) l_c, M = max_c m_c (m in log2 units); 0 without keys.
// With fp16 partials O_c holds O_c / l_c, weighed by 2^(m_c - M) l_c.
template <int D>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p)
{
    using namespace fa;
    constexpr int MAXC = 64, RG = 8;   // chunks per query tile; rows per workgroup
    static_assert(RG * 32 == 256, "one 32-lane group per row");
    __shared__ float wgt[RG][MAXC];
    const uint32_t qt = blockIdx.x / (BQ / RG), r0 = (blockIdx.x % (BQ / RG)) * RG;
    const uint32_t h = blockIdx.y, b = blockIdx.z;
    const uint32_t tab = p.qt_tab[qt], u0 = tab & 0xFFFF, nc = tab >> 16;   // a scalar load of the arguments
    const size_t g0 = ((size_t)b * p.hq + h) * p.units + u0;
    const bool part16 = p.o_dtype == DT_F16;
    // per-row chunk weights 2^(m_c - M) (l_c) / sum_c 2^(m_c - M) l_c: thread t
    // takes row t / 32 and chunks t % 32, t % 32 + 32; max and sum reduce
    // over the row's 32 lanes
    {
        const uint32_t rl = threadIdx.x / 32, c0 = threadIdx.x % 32, row = r0 + rl;
        float mc[2], lc[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {   // both loads in flight (chunks past nc read nc - 1, then dropped)
            const uint32_t c = min(c0 + 32 * k, nc - 1);
            const float2 ml = *(const float2*)(p.ws_ml + ((g0 + c) * BQ + row) * 2);
            const bool in = c0 + 32 * k < nc;
            mc[k] = in ? ml.x : -__builtin_inff();
            lc[k] = in ? ml.y : 0.f;
        }
        float M = fmaxf(mc[0], mc[1]);
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) M = fmaxf(M, __shfl_xor(M, s, 32));
        float w[2], den = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            w[k] = (M == -__builtin_inff() || mc[k] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(mc[k] - M);
            den += w[k] * lc[k];
            if (part16) w[k] *= lc[k];
        }
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) den += __shfl_xor(den, s, 32);
        const float inv = den > 0.f ? 1.0f / den : 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) wgt[rl][c0 + 32 * k] = w[k] * inv;   // 0 past nc
    }
    __syncthreads();
    // thread t: rows r0 + (t*4 / D) .., 4 consecutive columns. Chunks 8 at a
    // time with all eight loads in flight (chunks past nc read chunk nc - 1
    // and weigh 0; one loop per partial type, so no branch sits between the
    // loads and their waits).
    const uint32_t ncr = (nc + 7) & ~7u;
    for (uint32_t e = threadIdx.x * 4; e < RG * D; e += 256 * 4) {
        const uint32_t rl = e / D, col = e % D, qrow = qt * BQ + r0 + rl;
        if (qrow >= p.tq || col >= p.head_dim) continue;   // (whole 4-column groups: head_dim % 8 == 0)
        const size_t base = (g0 * BQ + r0 + rl) * D + col, cstride = (size_t)BQ * D;
        float4v acc = (float4v)0.f;
        if (part16) {
            const half_t* src = (const half_t*)p.ws_o + base;
            for (uint32_t c0 = 0; c0 < ncr; c0 += 8) {
                half4 v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = *(const half4*)(src + min(c0 + i, nc - 1) * cstride);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += wgt[rl][c0 + i] * __builtin_convertvector(v[i], float4v);
            }
        } else {
            const float* src = p.ws_o + base;
            for (uint32_t c0 = 0; c0 < ncr; c0 += 8) {
                float4v v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = *(const float4v*)(src + min(c0 + i, nc - 1) * cstride);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += wgt[rl][c0 + i] * v[i];
            }
        }
        const size_t o = (((size_t)b * p.tq + qrow) * p.hq + h) * p.head_dim + col;
        if (p.o_dtype == DT_F16) *(half4*)((half_t*)p.out + o) = __builtin_convertvector(acc, half4);
        else *(float4v*)((float*)p.out + o) = acc;
    }
}

// The cache count a plan is sized for: the most a launch can see (a full
// cache; a ring's visible keys span no more than that either), 0 without one.
// A launch with fewer cached keys runs the same units, some of them empty.
static uint32_t plan_cached(const AttnParams& p)
{
    return p.cache_count && p.kv_rows > p.tkv ? p.kv_rows - p.tkv : 0u;
}

uint32_t attention_units(const AttnParams& p, uint32_t chunk_tiles)
{
    AttnParams q = p;
    q.chunk_tiles = chunk_tiles;
    const uint32_t nqt = (p.tq + fa::BQ - 1) / fa::BQ, cached = plan_cached(p);
    uint32_t units = 0;
    for (uint32_t qt = 0; qt < nqt; ++qt) units += fa_chunks(q, qt, cached);
    return units == nqt ? 0u : units;
}

// The plain path: one workgroup per (query row, head, sequence) walks the
// row's visible keys 256 at a time in fp32 -- thread t scores key j0 + t,
// the block takes the tile's max and sum (online softmax in natural-log
// units, as attention.comp's fp32 naive kernel), then every thread adds the
// tile's P V into the head-dim columns it owns (t, t + 256, ..). Any head dim
// up to 256 * NAIVE_COLS, any mix of fp32 / fp16 operands; no workspace.
constexpr int NAIVE_COLS = 8;

__device__ __forceinline__ float naive_block_reduce(float v, bool is_max, float* red)
{
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const float o = __shfl_xor(v, s, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    __syncthreads();   // red's previous readers are done
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) v = is_max ? fmaxf(v, red[w]) : v + red[w];
    return v;
}

__global__ __launch_bounds__(256) void attention_naive_kernel(AttnParams p)
{
    __shared__ float qs[256 * NAIVE_COLS];
    __shared__ float ps[256];
    __shared__ float red[4];
    const uint32_t i = blockIdx.x, h = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
    const uint32_t HD = p.head_dim, hk = h / (p.hq / p.hkv);
    const size_t qbase = (((size_t)b * p.hq + h) * p.tq + i) * HD;
    const size_t kvbase = ((size_t)b * p.hkv + hk) * p.kv_rows * HD;
    for (uint32_t d = t; d < HD; d += 256) qs[d] = ld(p.q, p.q_dtype, qbase + d);
    const uint32_t cached = p.cache_count ? *p.cache_count : 0u;
    const int64_t live = p.ring ? (int64_t)cached + p.tkv : std::min<int64_t>((int64_t)cached + p.tkv, p.kv_rows);
    const int64_t kbeg = p.mask.key_start_cached(i, cached);
    const int64_t kend = std::min<int64_t>(p.mask.key_end_cached(i, cached), live);
    const auto krow = [&](int64_t j) -> size_t { return p.ring ? (size_t)(j % p.kv_rows) : (size_t)j; };
    float o[NAIVE_COLS];
#pragma unroll
    for (int r = 0; r < NAIVE_COLS; ++r) o[r] = 0.f;
    float m = -__builtin_inff(), l = 0.f;
    __syncthreads();
    for (int64_t j0 = kbeg; j0 < kend; j0 += 256) {
        const int64_t j = j0 + t;
        float sc = -__builtin_inff();
        if (j < kend) {
            float acc = 0.f;
            const size_t kr = kvbase + krow(j) * HD;
            for (uint32_t d = 0; d < HD; ++d) acc = fmaf(qs[d], ld(p.k, p.kv_dtype, kr + d), acc);
            sc = acc * p.scale;
        }
        const float mnew = fmaxf(m, naive_block_reduce(sc, true, red));   // finite: the tile has a key
        const float alpha = m == -__builtin_inff() ? 0.f : expf(m - mnew);
        const float e = sc == -__builtin_inff() ? 0.f : expf(sc - mnew);
        ps[t] = e;
        l = l * alpha + naive_block_reduce(e, false, red);   // (its barriers publish ps)
        m = mnew;
        const int64_t n = kend - j0 < 256 ? kend - j0 : 256;
#pragma unroll
        for (int r = 0; r < NAIVE_COLS; ++r) {
            const uint32_t d = t + 256 * r;
            if (d >= HD) break;
            float acc = o[r] * alpha;
            for (int64_t jj = 0; jj < n; ++jj)
                acc = fmaf(ps[jj], ld(p.v, p.kv_dtype, kvbase + krow(j0 + jj) * HD + d), acc);
            o[r] = acc;
        }
        __syncthreads();   // ps is rewritten by the next tile
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const size_t obase = (((size_t)b * p.tq + i) * p.hq + h) * HD;
#pragma unroll
    for (int r = 0; r < NAIVE_COLS; ++r) {
        const uint32_t d = t + 256 * r;
        if (d < HD) st(p.out, p.o_dtype, obase + d, o[r] * inv);
    }
}

// The KV cache append (the reference's fused append, attention-fa.comp:
// 344-400): the tkv new K / V rows of KV head blockIdx.y go to positions
// cached .. cached + tkv - 1 of the cache (row p, or p % kv_rows for a ring),
// converted to the cache dtype. A cache without a ring drops rows past its
// size (the caller keeps the count within it).
__global__ __launch_bounds__(256) void attention_append_kernel(AttnParams p)
{
    const uint32_t HD = p.head_dim, hk = blockIdx.y, cached = *p.cache_count;
    const size_t n = (size_t)p.tkv * HD;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) {
        const uint32_t tok = (uint32_t)(e / HD), d = (uint32_t)(e % HD), pos = cached + tok;
        if (!p.ring && pos >= p.kv_rows) continue;
        // a ring keeps the call's last kv_rows tokens: an earlier token that a
        // later one of the same call lands on is not written (no write race)
        if (p.ring && tok + p.kv_rows < p.tkv) continue;
        const size_t row = p.ring ? pos % p.kv_rows : pos;
        const size_t src = ((size_t)hk * p.tkv + tok) * HD + d, dst = ((size_t)hk * p.kv_rows + row) * HD + d;
        st((void*)p.k, p.kv_dtype, dst, ld(p.k_new, p.new_dtype, src));
        st((void*)p.v, p.kv_dtype, dst, ld(p.v_new, p.new_dtype, src));
    }
}

// fp32 K and V rounded to fp16 (round to nearest even) for the flash kernel,
// n4 groups of 4 values each.
__global__ __launch_bounds__(256) void attention_kv_f16_kernel(const float4v* k, const float4v* v, half4* ko,
                                                               half4* vo, size_t n4)
{
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n4; e += (size_t)gridDim.x * 256) {
        ko[e] = __builtin_convertvector(k[e], half4);
        vo[e] = __builtin_convertvector(v[e], half4);
    }
}

// Split the key ranges only when the query tiles alone leave CUs idle, in the
// shortest chunks whose work units still fit one round of workgroups (the
// merge pass reads every unit's partial O back). At most 64 chunks per query
// tile (the merge keeps their weights in LDS).
void attention_plan(AttnParams& p, uint32_t cus)
{
    p.units = 0;
    p.chunk_tiles = 0;
    const uint32_t HD = p.head_dim;
    const uint32_t qsz = p.q_dtype == DT_F32 ? 4 : 2;
    // The flash kernel's operand rules (the reference's FA gate, attention.h:
    // 916-945: Dh % 8 == 0, 16 <= Dh <= 256), plus 16-byte aligned operands
    // and buffer ranges under 2^31 bytes; anything else takes the plain path.
    const bool flash = HD % 8 == 0 && HD >= 16 && HD <= 256 && ((uintptr_t)p.q % 16) == 0 &&
                       ((uintptr_t)p.k % 16) == 0 && ((uintptr_t)p.v % 16) == 0 &&
                       (size_t)p.kv_rows * HD * 2 < (1ull << 31) && (size_t)p.tq * HD * qsz < (1ull << 31);
    p.dp = !flash ? 0 : HD <= 64 ? 64 : HD <= 128 ? 128 : 256;
    if (!p.dp) return;
    const uint32_t nqt = (p.tq + fa::BQ - 1) / fa::BQ, tiles = p.batch * p.hq * nqt;
    const uint32_t key_tiles = (plan_cached(p) + p.tkv + fa::BKV - 1) / fa::BKV;
    const uint32_t min_chunk = std::max<uint32_t>(2, (key_tiles + 63) / 64);
    p.chunk_tiles = std::max<uint32_t>(min_chunk, key_tiles);
    if (tiles >= cus) return;
    for (uint32_t c = min_chunk; c <= key_tiles; ++c) {
        const uint32_t u = attention_units(p, c);
        if (u == 0) return;   // chunks as long as the whole walks: no split
        const uint64_t wgs = (uint64_t)u * p.batch * p.hq;
        if (wgs <= cus && wgs <= AttnParams::FA_WG_TAB && nqt <= 0x10000) {
            p.chunk_tiles = c;
            p.units = u;
            // the units of a head, from the last query tile (the longest
            // causal walks start first), chunk by chunk
            uint32_t uq[AttnParams::FA_WG_TAB], uc[AttnParams::FA_WG_TAB], un[AttnParams::FA_WG_TAB], n = 0;
            for (uint32_t qt = nqt; qt-- > 0;) {
                const uint32_t nc = fa_chunks(p, qt, plan_cached(p));
                p.qt_tab[qt] = n | nc << 16;
                for (uint32_t ch = 0; ch < nc; ++ch, ++n) {
                    uq[n] = qt;
                    uc[n] = ch;
                    un[n] = nc;
                }
            }
            // workgroup w -> unit of head and batch, a head's units on one XCD
            for (uint32_t w = 0; w < wgs; ++w) {
                const uint32_t lb = fa_xcd_block(w, (uint32_t)wgs), unit = lb % u, h = (lb / u) % p.hq,
                               b = lb / (u * p.hq);
                p.wg_tab[2 * w] = uq[unit] | uc[unit] << 16 | un[unit] << 24;
                p.wg_tab[2 * w + 1] = unit | h << 10 | b << 20;
            }
            return;
        }
    }
}

static size_t attention_kv_bytes(const AttnParams& p)
{
    if (!p.dp || p.kv_dtype != DT_F32) return 0;
    const size_t n = (size_t)p.batch * p.hkv * p.kv_rows * p.head_dim;
    return (2 * n * sizeof(half_t) + 255) & ~(size_t)255;
}

size_t attention_workspace_bytes(const AttnParams& p)
{
    size_t bytes = attention_kv_bytes(p);
    if (p.units) bytes += (size_t)p.batch * p.hq * p.units * fa::BQ * (p.dp + 2) * sizeof(float);
    return bytes;
}

void attention_set_workspace(AttnParams& p, void* ws)
{
    const size_t kvb = attention_kv_bytes(p);
    p.ws_kv = kvb ? ws : nullptr;
    p.ws_o = (float*)((char*)ws + kvb);
    p.ws_ml = p.ws_o + (size_t)p.batch * p.hq * p.units * fa::BQ * p.dp;
}

bool attention_ok(const AttnParams& p)
{
    const auto dt_ok = [](int d) { return d == DT_F32 || d == DT_F16; };
    return p.hq > 0 && p.hkv > 0 && p.hq % p.hkv == 0 && p.head_dim > 0 && p.head_dim <= 256 * NAIVE_COLS &&
           dt_ok(p.q_dtype) && dt_ok(p.kv_dtype) && dt_ok(p.o_dtype);
}

template <int D>
static hipError_t attention_launch_d(const AttnParams& p, hipStream_t s)
{
    static PerDevice lds_once;
    {
        hipError_t e = set_max_lds(lds_once, (const void*)attention_fwd_kernel<D>, fa::Lds<D>::BYTES);
        if (e != hipSuccess) return e;
    }
    const uint32_t nqt = (p.tq + fa::BQ - 1) / fa::BQ;
    const dim3 grid = p.units ? dim3(p.units * p.hq * p.batch) : dim3(nqt, p.hq, p.batch);
    hipLaunchKernelGGL(attention_fwd_kernel<D>, grid, dim3(256), fa::Lds<D>::BYTES, s, p);
    if (p.units == 0) return hipGetLastError();
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge_kernel<D>, dim3(nqt * (fa::BQ / 8), p.hq, p.batch), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t attention_launch(const AttnParams& p0, hipStream_t s)
{
    if (p0.cache_count && p0.tkv > 0) {
        const size_t n = (size_t)p0.tkv * p0.head_dim;
        const uint32_t blocks = (uint32_t)std::min<size_t>((n + 255) / 256, 1024);
        hipLaunchKernelGGL(attention_append_kernel, dim3(blocks, p0.hkv), dim3(256), 0, s, p0);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (!p0.dp) {
        hipLaunchKernelGGL(attention_naive_kernel, dim3(p0.tq, p0.hq, p0.batch), dim3(256), 0, s, p0);
        return hipGetLastError();
    }
    AttnParams p = p0;
    if (p.kv_dtype == DT_F32) {
        if (!p.ws_kv) return hipErrorInvalidValue;
        const size_t n = (size_t)p.batch * p.hkv * p.kv_rows * p.head_dim;
        half_t* k16 = (half_t*)p.ws_kv;
        half_t* v16 = k16 + n;
        const size_t n4 = n / 4;
        const uint32_t blocks = (uint32_t)std::min<size_t>((n4 + 255) / 256, 4096);
        hipLaunchKernelGGL(attention_kv_f16_kernel, dim3(blocks), dim3(256), 0, s, (const float4v*)p.k,
                           (const float4v*)p.v, (half4*)k16, (half4*)v16, n4);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        p.k = k16;
        p.v = v16;
        p.kv_dtype = DT_F16;
    }
    switch (p.dp) {
    case 64: return attention_launch_d<64>(p, s);
    case 128: return attention_launch_d<128>(p, s);
    case 256: return attention_launch_d<256>(p, s);
    default: return hipErrorInvalidValue;
    }
}

}   // namespace vai_dev
