// attention.hip -- fused attention forward O = softmax(scale * Q K^T + mask) V
// for fp16 Q/K/V on gfx950 (the role of /root/reference/vai/shaders/
// attention-fa.comp: scores, online softmax and P.V in one pass; the mask
// rule of common/causal_mask.h:25-42; the node at nodes/attention.h:979-1304).
//
// One workgroup (4 waves) owns 64 query rows of one head, 16 per wave, and
// walks the key tiles (64 keys) the mask leaves visible. Per key tile:
//  * K [64 x D] and V^T [D x 64] are staged in LDS (V transposed on the way,
//    so a lane reads its P.V operand as two 8-byte runs);
//  * S^T = K Q^T on v_mfma_f32_16x16x32_f16 (A = K rows from LDS, B = the
//    wave's Q rows, held in registers for the whole walk). S^T rather than S:
//    the output then gives lane l query row l % 16 and 16 of the tile's keys
//    (16f + 4*(l/16) + r), which is exactly the A operand of the P.V MFMA
//    with the keys of a 32-wide step in the order 4g + r, 16 + 4g + r; V is
//    read in the same key order, so each product is still summed once;
//  * online softmax per query row (running max m and sum l in fp32; row
//    reductions are two cross-lane exchanges), exp2 with scale * log2(e)
//    folded in;
//  * O += P V with P rounded to fp16 (the fp16 operand of the reference's
//    P.V stage), O in fp32 registers: D/16 fragments of 16x16.
// The rows a lane holds in O (4*(l/16) + r) differ from its softmax row
// (l % 16): the per-row rescale and the final 1/l move across lanes by
// shuffle. Rows with no visible key give 0. The next key tile's global loads
// are issued into registers before the current tile is computed.
#include <algorithm>

#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

namespace vai_dev {

namespace fa {
constexpr int BQ = 64, BKV = 64;
template <int D> struct Lds {
    static constexpr int KP = D + 8;              // K row pitch (halves): rows 16 B apart in banks
    static constexpr int VP = BKV + 8;            // V^T row pitch (halves)
    static constexpr int K_BYTES = BKV * KP * 2;
    static constexpr int BYTES = K_BYTES + D * VP * 2;
};
}

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// The 64-key tiles query tile qt can see: [tb, te).
__host__ __device__ inline void fa_tile_range(const AttnParams& p, uint32_t qt, int64_t& tb, int64_t& te)
{
    const uint32_t q0 = qt * fa::BQ, q1 = std::min<uint32_t>(q0 + fa::BQ, p.tq) - 1;
    const int64_t kend = p.mask.key_end(q1), kbeg = p.mask.key_start(q0);
    tb = kbeg / fa::BKV;
    te = kend <= kbeg ? tb : (kend + fa::BKV - 1) / fa::BKV;
}

// Chunks of query tile qt (at least one, so that every tile writes output).
__host__ __device__ inline uint32_t fa_chunks(const AttnParams& p, uint32_t qt)
{
    int64_t tb, te;
    fa_tile_range(p, qt, tb, te);
    const int64_t n = te - tb;   // at most Tkv / 64: a 32-bit division suffices
    return n <= 0 ? 1u : ((uint32_t)n + p.chunk_tiles - 1) / p.chunk_tiles;
}

template <int D>
__global__ __launch_bounds__(256) void attention_fwd_kernel(AttnParams p)
{
    using namespace fa;
    constexpr int KP = Lds<D>::KP, VP = Lds<D>::VP, KS = D / 32, DB = D / 16;
    extern __shared__ half8 fa_lds[];
    half_t* ks = (half_t*)fa_lds;                              // [BKV][KP]
    half_t* vt = ks + BKV * KP;                                // [D][VP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const uint32_t Tq = p.tq, Tkv = p.tkv;
    const uint32_t h = blockIdx.y, b = blockIdx.z, nqt = (Tq + BQ - 1) / BQ;
    // Work unit -> (query tile, key chunk). Units enumerate the query tiles
    // from the last (the longest causal walks start first), chunk by chunk.
    uint32_t qt, chunk = 0;
    if (p.units == 0) {
        qt = nqt - 1 - blockIdx.x;
    } else {
        uint32_t u = blockIdx.x;
        qt = nqt - 1;
        for (;;) {
            const uint32_t nc = fa_chunks(p, qt);
            if (u < nc || qt == 0) break;
            u -= nc;
            --qt;
        }
        chunk = u;
        qt = __builtin_amdgcn_readfirstlane(qt);
        chunk = __builtin_amdgcn_readfirstlane(chunk);
    }
    const uint32_t q0 = qt * BQ;
    const uint32_t hk = h / (p.hq / p.hkv);
    const half_t* Q = (const half_t*)p.q + ((size_t)b * p.hq + h) * Tq * D;
    const half_t* K = (const half_t*)p.k + ((size_t)b * p.hkv + hk) * Tkv * D;
    const half_t* V = (const half_t*)p.v + ((size_t)b * p.hkv + hk) * Tkv * D;

    // this wave's 16 query rows as the B operand of S^T = K Q^T
    const uint32_t qrow = q0 + wave * 16 + lr;
    half8 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
        qf[s] = qrow < Tq ? *(const half8*)(Q + (size_t)qrow * D + s * 32 + lg * 8) : (half8)0;

    // visible key tiles of the query tile, then this unit's chunk of them
    int64_t tb, te;
    fa_tile_range(p, qt, tb, te);
    if (p.units != 0) {
        const int64_t c0 = tb + (int64_t)chunk * p.chunk_tiles;
        te = std::min<int64_t>(te, c0 + p.chunk_tiles);
        tb = c0;
    }
    const int64_t kbeg = tb * BKV, kend = std::min<int64_t>(te * BKV, (int64_t)Tkv);

    const float sl2 = p.scale * 1.4426950408889634f;   // scores in log2 units
    // this lane's query row reads keys [row_kbeg, row_kend)
    const uint32_t qclip = qrow < Tq ? qrow : Tq - 1;
    const int64_t row_kend = p.mask.key_end(qclip), row_kbeg = p.mask.key_start(qclip);
    float m = -__builtin_inff(), l = 0.f;
    float4v o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = (float4v)0.f;

    // Key tile j0 is loaded into registers one tile ahead (its global loads
    // fly while the tile before it is computed), then written to LDS: K
    // rows as 16-byte chunks, V transposed. K chunk c of a thread is row
    // c / NC, chunk c % NC (coalesced rows, conflict-free 16-byte writes). V
    // chunks go 8 keys x 8 chunks per 64 lanes: each load instruction reads
    // eight 128-byte row pieces, and the transposed 2-byte writes of one
    // instruction land on consecutive keys of 8 V^T rows (one chunk per row
    // across the lanes would put 64 lanes on two bank positions).
    constexpr int NC = D / 8;                  // 16-byte chunks per row
    constexpr int CPT = BKV * NC / 256;        // chunks per thread and operand
    half8 kreg[CPT], vreg[CPT];
    auto vmap = [&](int i, int& r, int& ch) __attribute__((always_inline)) {
        const int slot = (tid >> 6) + 4 * i, l = tid & 63;   // slot: 64-lane group, 0 .. NC-1
        r = (slot % 8) * 8 + l / 8;
        ch = (slot / 8) * 8 + l % 8;
    };
    auto load_tile = [&](int64_t j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 256, r = c / NC, ch = c % NC;
            int vr, vc;
            vmap(i, vr, vc);
            kreg[i] = j0 + r < (int64_t)Tkv ? *(const half8*)(K + (size_t)(j0 + r) * D + ch * 8) : (half8)0;
            vreg[i] = j0 + vr < (int64_t)Tkv ? *(const half8*)(V + (size_t)(j0 + vr) * D + vc * 8) : (half8)0;
        }
    };
    if (kbeg < kend) load_tile(kbeg);
    for (int64_t j0 = kbeg; j0 < kend; j0 += BKV) {
        __syncthreads();   // the previous tile's reads are done
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * 256, r = c / NC, ch = c % NC;
            *(half8*)(ks + r * KP + ch * 8) = kreg[i];
            int vr, vc;
            vmap(i, vr, vc);
#pragma unroll
            for (int e = 0; e < 8; ++e) vt[(vc * 8 + e) * VP + vr] = vreg[i][e];
        }
        __syncthreads();
        if (j0 + BKV < kend) load_tile(j0 + BKV);

        // S^T for the 4 key blocks of 16: lane holds query row lr, keys 16f + 4lg + r
        float4v st[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            st[f] = (float4v)0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const half8 ka = *(const half8*)(ks + (16 * f + lr) * KP + s * 32 + lg * 8);
                st[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[s], st[f], 0, 0, 0);
            }
        }
        // mask, scale, running max
        float tmax = -__builtin_inff();
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t kpos = j0 + 16 * f + 4 * lg + r;
                const bool hide = kpos >= row_kend || kpos < row_kbeg;
                const float v = hide ? -__builtin_inff() : st[f][r] * sl2;
                st[f][r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(m, tmax);
        const float alpha = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
        float psum = 0.f;
        half8 pa[2];
#pragma unroll
        for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = st[f][r] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(st[f][r] - mnew);
                psum += e;
                pa[f / 2][(f % 2) * 4 + r] = (half_t)e;
            }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l = alpha * l + psum;
        m = mnew;

        // O rows 4lg + r take the rescale of their softmax row (held by lane 4lg + r)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * lg + r, 64);
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d][r] *= ar;
        }
        // O += P V: k-step s2 covers keys 32 s2 + {4lg + r, 16 + 4lg + r}
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const half_t* vr = vt + (d * 16 + lr) * VP + 32 * s2 + 4 * lg;
                const half4v lo = *(const half4v*)vr, hi = *(const half4v*)(vr + 16);
                const half8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[s2], vb, o[d], 0, 0, 0);
            }
    }

    if (p.units != 0) {
        // partial result: O unnormalised, (m, l) per row
        const size_t gid = ((size_t)b * p.hq + h) * p.units + blockIdx.x;
        float* wo = p.ws_o + gid * BQ * D;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int d = 0; d < DB; ++d) wo[(size_t)(wave * 16 + 4 * lg + r) * D + d * 16 + lr] = o[d][r];
        if (lg == 0) {
            float* wml = p.ws_ml + (gid * BQ + wave * 16 + lr) * 2;
            wml[0] = m;
            wml[1] = l;
        }
        return;
    }
    // O / l per row, then the store: lane holds rows 4lg + r, column d*16 + lr
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float ir = __shfl(inv, 4 * lg + r, 64);
        const uint32_t row = q0 + wave * 16 + 4 * lg + r;
        if (row >= Tq) continue;
        const size_t base = (((size_t)b * p.hq + h) * Tq + row) * D + lr;
#pragma unroll
        for (int d = 0; d < DB; ++d) st(p.out, p.o_dtype, base + d * 16, o[d][r] * ir);
    }
}

// Merge of the key chunks of one query tile: O = sum_c 2^(m_c - M) O_c /
// sum_c 2^(m_c - M) l_c, M = max_c m_c (m in log2 units); 0 without keys.
template <int D>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnParams p)
{
    using namespace fa;
    constexpr int MAXC = 64, RG = 8;   // chunks per query tile; rows per workgroup
    static_assert(RG * 32 == 256, "one 32-lane group per row");
    __shared__ float wgt[RG][MAXC];
    const uint32_t nqt = (p.tq + BQ - 1) / BQ, qt = blockIdx.x / (BQ / RG), r0 = (blockIdx.x % (BQ / RG)) * RG;
    const uint32_t h = blockIdx.y, b = blockIdx.z;
    // first unit of query tile qt: the chunks of the later tiles (units run
    // from the last query tile down), summed across a 64-lane group
    __shared__ uint32_t first_unit;
    if (threadIdx.x < 64) {
        uint32_t n = 0;
        for (uint32_t q = qt + 1 + threadIdx.x; q < nqt; q += 64) n += fa_chunks(p, q);
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) n += __shfl_xor(n, s, 64);
        if (threadIdx.x == 0) first_unit = n;
    }
    __syncthreads();
    const uint32_t u0 = first_unit;
    const uint32_t nc = fa_chunks(p, qt);
    const size_t g0 = ((size_t)b * p.hq + h) * p.units + u0;
    // per-row chunk weights 2^(m_c - M) / sum_c 2^(m_c - M) l_c: thread t
    // takes row t / 32 and chunks t % 32, t % 32 + 32; max and sum reduce
    // over the row's 32 lanes
    {
        const uint32_t rl = threadIdx.x / 32, c0 = threadIdx.x % 32, row = r0 + rl;
        float mc[2], lc[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t c = c0 + 32 * k;
            mc[k] = -__builtin_inff();
            lc[k] = 0.f;
            if (c < nc) {
                const float2 ml = *(const float2*)(p.ws_ml + ((g0 + c) * BQ + row) * 2);
                mc[k] = ml.x;
                lc[k] = ml.y;
            }
        }
        float M = fmaxf(mc[0], mc[1]);
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) M = fmaxf(M, __shfl_xor(M, s, 32));
        float w[2], den = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            w[k] = (M == -__builtin_inff() || mc[k] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(mc[k] - M);
            den += w[k] * lc[k];
        }
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) den += __shfl_xor(den, s, 32);
        const float inv = den > 0.f ? 1.0f / den : 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k)
            if (c0 + 32 * k < nc) wgt[rl][c0 + 32 * k] = w[k] * inv;
    }
    __syncthreads();
    // thread t: rows r0 + (t*4 / D) .., 4 consecutive columns (16-byte loads)
    for (uint32_t e = threadIdx.x * 4; e < RG * D; e += 256 * 4) {
        const uint32_t rl = e / D, col = e % D, qrow = qt * BQ + r0 + rl;
        if (qrow >= p.tq) continue;
        float4v acc = (float4v)0.f;
        for (uint32_t c = 0; c < nc; ++c)
            acc += wgt[rl][c] * *(const float4v*)(p.ws_o + ((g0 + c) * BQ + r0 + rl) * D + col);
        const size_t o = (((size_t)b * p.hq + h) * p.tq + qrow) * D + col;
#pragma unroll
        for (int k = 0; k < 4; ++k) st(p.out, p.o_dtype, o + k, acc[k]);
    }
}

uint32_t attention_units(const AttnParams& p, uint32_t chunk_tiles)
{
    AttnParams q = p;
    q.chunk_tiles = chunk_tiles;
    const uint32_t nqt = (p.tq + fa::BQ - 1) / fa::BQ;
    uint32_t units = 0;
    for (uint32_t qt = 0; qt < nqt; ++qt) units += fa_chunks(q, qt);
    return units == nqt ? 0u : units;
}

size_t attention_workspace_bytes(const AttnParams& p, uint32_t units)
{
    return (size_t)p.batch * p.hq * units * fa::BQ * (p.head_dim + 2) * sizeof(float);
}

bool attention_ok(const AttnParams& p)
{
    return (p.head_dim == 64 || p.head_dim == 128 || p.head_dim == 256) && p.hq > 0 && p.hkv > 0 &&
           p.hq % p.hkv == 0 && ((uintptr_t)p.q % 16) == 0 && ((uintptr_t)p.k % 16) == 0 &&
           ((uintptr_t)p.v % 16) == 0;
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
    const dim3 grid(p.units ? p.units : nqt, p.hq, p.batch);
    hipLaunchKernelGGL(attention_fwd_kernel<D>, grid, dim3(256), fa::Lds<D>::BYTES, s, p);
    if (p.units == 0) return hipGetLastError();
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge_kernel<D>, dim3(nqt * (fa::BQ / 8), p.hq, p.batch), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t attention_launch(const AttnParams& p, hipStream_t s)
{
    switch (p.head_dim) {
    case 64: return attention_launch_d<64>(p, s);
    case 128: return attention_launch_d<128>(p, s);
    case 256: return attention_launch_d<256>(p, s);
    default: return hipErrorInvalidValue;
    }
}

}   // namespace vai_dev
