// slab.hip -- Linear for M <= 8: the HBM-streaming GEMV (the role of
// /root/reference/vai/shaders/linear-slab.comp).
//
// O[m,n] = s * epi(sum_k I[m,k] W[n,k] + B) (+R), fp32 accumulation on the
// operands as stored (fp16 is exact in fp32), as linear-slab.comp:5-15 states.
//
// Design (gfx950): W dominates the traffic (N*K elements, read once), so the
// kernel is shaped for HBM: each wave owns R whole rows of W and issues all
// of its 16-byte non-temporal loads for a K block before touching them, so a
// CU keeps ~100 KB of loads in flight. The M <= 8 input rows are staged once
// per workgroup in LDS and broadcast to the four waves. Each lane ends with
// M*R partial dot products; a butterfly over the wave halves the number of
// values per lane at each exchange (M*R + 6 - log2(M*R) shuffles instead of
// 6*M*R), leaving lane groups that each own one output for the epilogue.
#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

#include <algorithm>
#include <type_traits>

#define LDS_AS __attribute__((address_space(3)))

namespace vai_dev {

__device__ __forceinline__ OutputSpec slab_output(const SlabParams& a)
{
    return OutputSpec{a.out, a.bias, a.residual, a.o_dtype, a.b_dtype, a.bias_repeat, a.residual_repeat,
                      a.epilogue, a.residual_order, a.scalar_scale};
}

template <typename T> struct Vec16;
template <> struct Vec16<half_t> { typedef half8 type; static constexpr int n = 8; };
template <> struct Vec16<float> { typedef float4v type; static constexpr int n = 4; };

// x + (x of the lane the DPP control names); all 64 lanes take part.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x)
{
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true);
    return x + __builtin_bit_cast(float, moved);
}

// Sum over the lane bits below LIMIT, lowest first: bits 0-3 stay inside a
// row of 16 lanes and go through DPP (quad_perm 1032, quad_perm 2301,
// row_half_mirror, row_mirror: after the lower bits are summed, each of
// these pairs lanes that differ in the next bit); bits 4 and 5 use the
// permlane swaps.
template <int LIMIT>
__device__ __forceinline__ float lane_sum_low(float x)
{
    if constexpr (LIMIT > 1) x = dpp_add<0xB1>(x);
    if constexpr (LIMIT > 2) x = dpp_add<0x4E>(x);
    if constexpr (LIMIT > 4) x = dpp_add<0x141>(x);
    if constexpr (LIMIT > 8) x = dpp_add<0x140>(x);
    if constexpr (LIMIT > 16) x = swap_sum<16>(x, x);
    if constexpr (LIMIT > 32) x = swap_sum<32>(x, x);
    return x;
}

// Butterfly over a wave of CNT values per lane: at offset O a lane keeps the
// half selected by (lane & O) and adds its partner's copy of that half, so
// each exchange halves the values per lane; once one is left, the lane bits
// below O are summed by lane_sum_low.
template <int CNT, int O>
__device__ __forceinline__ void butterfly(float* acc, int lane)
{
    if constexpr (CNT > 1) {
        constexpr int H = CNT / 2;
        if constexpr (O >= 16) {
#pragma unroll
            for (int i = 0; i < H; ++i) acc[i] = swap_sum<O>(acc[i], acc[i + H]);
        } else {
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float send = upper ? acc[i] : acc[i + H];
                const float keep = upper ? acc[i + H] : acc[i];
                acc[i] = keep + __shfl_xor(send, O, 64);
            }
        }
        butterfly<H, O / 2>(acc, lane);
    } else {
        acc[0] = lane_sum_low<O * 2>(acc[0]);
    }
}

// The value index a lane holds after butterfly<V, 32>.
template <int V>
__device__ __forceinline__ int butterfly_index(int lane)
{
    int idx = 0, h = V;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        if (h > 1) {
            h >>= 1;
            if (lane & o) idx += h;
        }
    }
    return idx;
}

// Lanes that agree on their value form groups of this size; the group's
// lowest lane writes.
template <int V>
constexpr int butterfly_low()
{
    int h = V, low = 64;
    for (int o = 32; o >= 1 && h > 1; o >>= 1) { h >>= 1; low = o; }
    return low;
}

// The dot products of one 16-byte W chunk against one X chunk: v_dot2_f32_f16
// for fp16 x fp16 (two exact products into the fp32 sum per instruction, half
// the VALU work of widening each operand), fp32 FMAs otherwise.
template <typename TI, typename TW, typename WV, typename XV>
__device__ __forceinline__ float chunk_dot(const WV& w, const XV& x, float s)
{
    constexpr int EPC = Vec16<TW>::n;
    if constexpr (std::is_same_v<TI, half_t> && std::is_same_v<TW, half_t>) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int e = 0; e < EPC; e += 2) s = __builtin_amdgcn_fdot2(h2{w[e], w[e + 1]}, h2{x[e], x[e + 1]}, s, false);
    } else {
#pragma unroll
        for (int e = 0; e < EPC; ++e) s = fmaf((float)w[e], (float)x[e], s);
    }
    return s;
}

// Few input rows (MP <= 2, or <= 4 when fp16): each lane keeps its X chunks in
// registers. Per K block the wave issues every W load of its R rows, then the
// X loads (L2-resident; issued before W, every wave's X fetch delayed the
// whole W stream), then computes as the loads land. A wave whose rows and
// block lie inside W runs a straight-line block with no per-load guards
// (exec-mask branches around each load spread the issue over hundreds of
// cycles and made the compiler wait for every load before the first product).
// ALL_FULL (N a multiple of 4R, K of the block): no guards anywhere, so the
// compiler interleaves each chunk's W and X loads and starts each chunk's
// products as it lands (config 2 at M = 1: 6.4 us against 6.8 us with the
// guarded block merged in).
// W, X, K, N and M also come as leading scalar arguments, which the launch
// preloads into SGPRs (this file is built with kernarg preloading): the
// first loads need nothing from the argument struct.
template <int MP, int R, int KCH, typename TI, typename TW, bool ALL_FULL>
__global__ __launch_bounds__(256) void slab_reg_kernel(const TW* __restrict__ Wp, const TI* __restrict__ Xp, uint32_t Kp,
                                                       uint32_t Np, uint32_t Mp, SlabParams a)
{
    typedef typename Vec16<TW>::type wvec;
    constexpr int EPC = Vec16<TW>::n;      // W elements per 16-byte chunk
    constexpr int KB = 64 * KCH * EPC;     // K elements per block iteration
    constexpr int V = MP * R;              // dot products per lane
    static_assert(V <= 64 && (V & (V - 1)) == 0, "butterfly needs a power of two <= 64");
    typedef TI xvec __attribute__((ext_vector_type(EPC)));

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = (blockIdx.x * 4u + wave) * R;
    const uint32_t K = Kp, N = Np, M = Mp;
    const TW* __restrict__ W = Wp;
    const TI* __restrict__ X = Xp;

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;

    auto block = [&](uint32_t kb, auto full_c) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full_c)::value;
        wvec wv[R][KCH];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < KCH; ++c) {
                const uint32_t k = kb + (uint32_t)(c * 64 + lane) * EPC;
                if (FULL || (n0 + r < N && k < K))
                    wv[r][c] = __builtin_nontemporal_load((const wvec*)(W + (size_t)(n0 + r) * K + k));
                else
                    wv[r][c] = (wvec)0;
            }
        // rows past M read row 0 (a valid address); their sums are never stored
        xvec xr[KCH][MP];
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
            const uint32_t k = kb + (uint32_t)(c * 64 + lane) * EPC;
#pragma unroll
            for (int m = 0; m < MP; ++m) {
                const uint32_t mr = (uint32_t)m < M ? (uint32_t)m : 0u;
                xr[c][m] = (FULL || k < K) ? *(const xvec*)(X + (size_t)mr * K + k) : (xvec)0;
            }
        }
#pragma unroll
        for (int c = 0; c < KCH; ++c)
#pragma unroll
            for (int m = 0; m < MP; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m * R + r] = chunk_dot<TI, TW>(wv[r][c], xr[c][m], acc[m * R + r]);
    };
    // K > 0 (the C ABI checks it): a loop that runs at least once lets the
    // compiler fetch every kernel argument in one batch at entry (a `K > 0`
    // test first had it fetch the weight pointer in a second, dependent round).
    uint32_t kb = 0;
    do {
        if constexpr (ALL_FULL) block(kb, std::true_type{});
        else if (n0 + R <= N && kb + KB <= K) block(kb, std::true_type{});
        else block(kb, std::false_type{});
        kb += KB;
    } while (kb < K);

    // Butterfly over the wave; afterwards lane `lane` holds value idx.
    butterfly<V, 32>(acc, lane);
    const int idx = butterfly_index<V>(lane);
    if ((lane & (butterfly_low<V>() - 1)) != 0) return;
    const uint32_t m = idx / R, r = idx % R;
    if (m >= M || n0 + r >= N) return;
    store_output(slab_output(a), (size_t)m * N + n0 + r, acc[0]);
}


// More input rows (5-8, or 3-8 with fp32 input): the M rows of each K block
// are staged once per workgroup in LDS and broadcast to the four waves.
template <int MP, int R, int KCH, typename TI, typename TW>
__global__ __launch_bounds__(256) void slab_vec_kernel(SlabParams a)
{
    typedef typename Vec16<TW>::type wvec;
    constexpr int EPC = Vec16<TW>::n;      // W elements per 16-byte chunk
    constexpr int KB = 64 * KCH * EPC;     // K elements per block iteration
    constexpr int V = MP * R;              // dot products per lane
    static_assert(V <= 64 && (V & (V - 1)) == 0, "butterfly needs a power of two <= 64");
    __shared__ TI xs[MP * KB];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = (blockIdx.x * 4u + wave) * R;
    const uint32_t K = a.K, N = a.N, M = a.M;
    const TW* __restrict__ W = (const TW*)a.weight;
    const TI* __restrict__ X = (const TI*)a.in;

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;

    for (uint32_t kb = 0; kb < K; kb += KB) {
        // 1. Every W load of this block for this wave's R rows, issued up front.
        wvec wv[R][KCH];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < KCH; ++c) {
                const uint32_t k = kb + (uint32_t)(c * 64 + lane) * EPC;
                if (n0 + r < N && k < K)
                    wv[r][c] = __builtin_nontemporal_load((const wvec*)(W + (size_t)(n0 + r) * K + k));
                else
                    wv[r][c] = (wvec)0;
            }
        // 2. The M input rows of this block into LDS (zero past K and past M).
        __syncthreads();
        for (uint32_t i = threadIdx.x * EPC; i < (uint32_t)(MP * KB); i += 256 * EPC) {
            const uint32_t m = i / KB, kk = kb + (i % KB);
            // EPC elements of X per thread: K % EPC == 0 keeps them in one row.
            typedef TI xvec __attribute__((ext_vector_type(EPC)));
            xvec v = (m < M && kk < K) ? *(const xvec*)(X + (size_t)m * K + kk) : (xvec)0;
            *(xvec*)(xs + i) = v;
        }
        __syncthreads();
        // 3. Dot products.
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
#pragma unroll
            for (int m = 0; m < MP; ++m) {
                float xf[EPC];
                const TI* xp = xs + m * KB + (c * 64 + lane) * EPC;
#pragma unroll
                for (int e = 0; e < EPC; ++e) xf[e] = (float)xp[e];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float s = acc[m * R + r];
#pragma unroll
                    for (int e = 0; e < EPC; ++e) s = fmaf((float)wv[r][c][e], xf[e], s);
                    acc[m * R + r] = s;
                }
            }
        }
    }

    // Butterfly over the wave; afterwards lane `lane` holds value idx.
    butterfly<V, 32>(acc, lane);
    const int idx = butterfly_index<V>(lane);
    if ((lane & (butterfly_low<V>() - 1)) != 0) return;
    const uint32_t m = idx / R, r = idx % R;
    if (m >= M || n0 + r >= N) return;
    store_output(slab_output(a), (size_t)m * N + n0 + r, acc[0]);
}

// Any K, any alignment: one wave per output column, scalar loads.
template <int MP>
__global__ __launch_bounds__(256) void slab_scalar_kernel(SlabParams a)
{
    const int lane = threadIdx.x & 63;
    const uint32_t n = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (n >= a.N) return;
    float acc[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) acc[m] = 0.f;
    for (uint32_t k = lane; k < a.K; k += 64) {
        const float w = ld(a.weight, a.w_dtype, (size_t)n * a.K + k);
#pragma unroll
        for (int m = 0; m < MP; ++m)
            if ((uint32_t)m < a.M) acc[m] = fmaf(ld(a.in, a.i_dtype, (size_t)m * a.K + k), w, acc[m]);
    }
#pragma unroll
    for (int m = 0; m < MP; ++m) {
        const float v = wave_sum(acc[m]);
        if (lane == 0 && (uint32_t)m < a.M) {
            const size_t o = (size_t)m * a.N + n;
            const float b = a.bias ? ld(a.bias, a.b_dtype, a.bias_repeat ? o % a.bias_repeat : o) : 0.f;
            const float rr = a.residual ? ld(a.residual, a.o_dtype, a.residual_repeat ? o % a.residual_repeat : o) : 0.f;
            st(a.out, a.o_dtype, o, finish(v + b, rr, a.epilogue, a.residual_order, a.scalar_scale));
        }
    }
}

// fp16 I and W, 2 <= M <= 16: the GEMV on v_mfma_f32_16x16x32_f16. A = I
// padded to 16 rows (rows >= M read as zero), B = 16 rows of W. fp16 products
// are exact in fp32 and accumulate in fp32, the slab contract, while the
// matrix core keeps the arithmetic off the VALU (at M = 8 the FMA path costs
// more than the 32 MB HBM stream it overlaps). A workgroup owns 16 W rows;
// wave w takes the K quarter [w*K/4, (w+1)*K/4) through a private 16 KB LDS
// region, 512 k per pass, and the four 16x16 partials meet in LDS at the end.
// W goes global -> LDS by buffer_load ... lds, 1 KB of one row per copy
// instruction, and the fragments are read back from LDS; the 16-byte chunks
// of row r sit at chunk ^ r, so a fragment read (16 rows, one chunk) hits
// distinct banks. (Loading fragments straight from W, 16 rows x 64 bytes per
// load instruction, measured 2-3% slower.)
__global__ __launch_bounds__(256) void gemv_lds_kernel(SlabParams a)
{
    extern __shared__ half8 gl_lds[];
    __shared__ float part[4][16][17];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = blockIdx.x * 16, K = a.K, N = a.N, M = a.M;
    const int fr = lane & 15, fg = lane >> 4;
    const uint32_t kq = K / 4, kbeg = wave * kq;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const half_t*)a.weight + (size_t)n0 * K), (short)0,
        (int)std::min<size_t>((size_t)(N - n0) * K * 2, 0x7FFFFFFF), 0x00020000);
    LDS_AS char* region = (LDS_AS char*)(LDS_AS void*)gl_lds + wave * 16384;
    const bool xrow_ok = (uint32_t)fr < M;
    const half_t* xp = (const half_t*)a.in + (size_t)(xrow_ok ? fr : 0) * K + kbeg + fg * 8;
    float4v acc = (float4v)0.f;
    for (uint32_t k = 0; k < kq; k += 512) {
        // row r: lane l copies logical chunk l ^ r of the row's 1 KB
#pragma unroll
        for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LDS_AS void*)(region + r * 1024), 16,
                                                     (int)((r * K + kbeg + k) * 2 + (lane ^ r) * 16), 0, 0, 0);
        half8 xv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            xv[i] = (xrow_ok && k + i * 32 < kq) ? *(const half8*)(xp + k + i * 32) : (half8)0;
        __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));   // vmcnt(0)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = 4 * i + fg;   // logical chunk of k = k + 32 i + 8 fg
            half8 wv = *(LDS_AS const half8*)(region + fr * 1024 + ((c ^ fr) * 16));
            if (k + i * 32 >= kq) wv = (half8)0;
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv[i], wv, acc, 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0): region free
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][fg * 4 + r][fr] = acc[r];
    __syncthreads();
    const int m = threadIdx.x / 16, j = threadIdx.x % 16;
    if ((uint32_t)m < M && n0 + j < N) {
        const float v = part[0][m][j] + part[1][m][j] + part[2][m][j] + part[3][m][j];
        const size_t o = (size_t)m * N + n0 + j;
        const float b = a.bias ? ld(a.bias, a.b_dtype, a.bias_repeat ? o % a.bias_repeat : o) : 0.f;
        const float rr = a.residual ? ld(a.residual, a.o_dtype, a.residual_repeat ? o % a.residual_repeat : o) : 0.f;
        st(a.out, a.o_dtype, o, finish(v + b, rr, a.epilogue, a.residual_order, a.scalar_scale));
    }
}

bool gemv_mfma_ok(const SlabParams& a)
{
    return a.i_dtype == DT_F16 && a.w_dtype == DT_F16 && a.M <= 16 && a.K % 128 == 0 &&
           ((uintptr_t)a.weight % 16) == 0 && ((uintptr_t)a.in % 16) == 0;
}

template <int MP, typename TI, typename TW>
static hipError_t launch_vec(const SlabParams& a, hipStream_t s)
{
    // R rows per wave x KCH chunks per lane: 2 x 4 (8 loads of 16 B in flight
    // per lane, 4096 waves at the config-2 shape) measured fastest on MI355X
    // among 1..8 x 2..8.
    constexpr int R = 2, KCH = 4;
    const uint32_t blocks = (a.N + 4 * R - 1) / (4 * R);
    constexpr uint32_t KB = 64 * KCH * Vec16<TW>::n;
    if constexpr (MP <= 2 || (MP <= 4 && sizeof(TI) == 2)) {
        if (a.N % (4 * R) == 0 && a.K % KB == 0)
            hipLaunchKernelGGL((slab_reg_kernel<MP, R, KCH, TI, TW, true>), dim3(blocks), dim3(256), 0, s,
                               (const TW*)a.weight, (const TI*)a.in, a.K, a.N, a.M, a);
        else
            hipLaunchKernelGGL((slab_reg_kernel<MP, R, KCH, TI, TW, false>), dim3(blocks), dim3(256), 0, s,
                               (const TW*)a.weight, (const TI*)a.in, a.K, a.N, a.M, a);
    } else
        hipLaunchKernelGGL((slab_vec_kernel<MP, R, KCH, TI, TW>), dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int MP>
static hipError_t launch_m(const SlabParams& a, hipStream_t s)
{
    if (a.i_dtype == DT_F16 && a.w_dtype == DT_F16) return launch_vec<MP, half_t, half_t>(a, s);
    if (a.i_dtype == DT_F32 && a.w_dtype == DT_F16) return launch_vec<MP, float, half_t>(a, s);
    if (a.i_dtype == DT_F16 && a.w_dtype == DT_F32) return launch_vec<MP, half_t, float>(a, s);
    return launch_vec<MP, float, float>(a, s);
}

bool slab_vec_ok(const SlabParams& a)
{
    const uint32_t epc = a.w_dtype == DT_F16 ? 8 : 4;
    const size_t ib = a.i_dtype == DT_F16 ? 2 : 4;
    return a.K % epc == 0 && ((uintptr_t)a.weight % 16) == 0 && ((uintptr_t)a.in % (epc * ib)) == 0;
}

hipError_t slab_launch(const SlabParams& a, hipStream_t s)
{
    // fp16 M 3-4: the vector kernel, dot products on v_dot2 (7.7 us on config
    // 2 at M = 4 against 8.8 us for the MFMA kernel); M >= 5: the MFMA kernel.
    if (a.M >= 5 && gemv_mfma_ok(a)) {
        static PerDevice lds_once;   // 64 KB dynamic + the static partial-sum array
        hipError_t e = set_max_lds(lds_once, (const void*)gemv_lds_kernel, 65536);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(gemv_lds_kernel, dim3((a.N + 15) / 16), dim3(256), 65536, s, a);
        return hipGetLastError();
    }
    if (slab_vec_ok(a)) {
        switch (a.M) {
        case 1: return launch_m<1>(a, s);
        case 2: return launch_m<2>(a, s);
        case 3: case 4: return launch_m<4>(a, s);
        default: return launch_m<8>(a, s);
        }
    }
    const uint32_t blocks = (a.N + 3) / 4;
    switch (a.M) {
    case 1: hipLaunchKernelGGL((slab_scalar_kernel<1>), dim3(blocks), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((slab_scalar_kernel<2>), dim3(blocks), dim3(256), 0, s, a); break;
    case 3: case 4: hipLaunchKernelGGL((slab_scalar_kernel<4>), dim3(blocks), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((slab_scalar_kernel<8>), dim3(blocks), dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

}   // namespace vai_dev
