// conv.hip -- implicit-GEMM convolution for fp16 weights on gfx950 (the role
// of /root/reference/vai/shaders/conv-k3s1-implicit-gemm.comp and
// conv-implicit-gemm.comp; plan choice in convolution.h:5408-5443).
//
//   out[b,co,ho,wo] = epi(scale[co] * sum_{c,kh,kw} W[co,c,kh,kw] X[b,c,ho*s+kh-p,wo*s+kw-p]
//                         + bias[co] (+R)) (+R)
//
// The reduction index is (tap, channel) here instead of the reference's
// c*k*k + tap: the order of an fp32 sum is free, and this one makes 8
// consecutive k values 8 consecutive channels, which is what one MFMA lane
// consumes. Weights are packed once to that order, in MFMA fragment order
// with channels zero-padded to a multiple of 32 (the reference transforms
// conv weights once too, convolution.h:6224-6235).
//
// Forward kernel: one workgroup of 8 waves per (32 output channels, one
// output row, image), or of 16 waves per 64 output channels when 32-channel
// workgroups would outnumber the CUs (fp16 input). It stages the k input rows it needs from NCHW into LDS
// transposed to [row][column][channel] (8 channels x 8 columns per work item:
// eight 16-byte loads, a register transpose, eight 16-byte LDS writes), so 8
// channels are one 16-byte LDS read; weight fragments come straight from the
// packed buffer (L2-resident) into VGPRs, 1 KB of contiguous memory per
// tap and wave (packing [tap][co][c] instead, a fragment load reads 16 rows x
// 64 bytes and the loads cost 25% of the kernel time). Waves = 4 channel blocks x 2
// (or 4) groups of 16 output channels; each runs v_mfma_f32_16x16x32_f16 over
// every tap, their partial sums meet in LDS, and scale, bias, residual and
// the activation are applied once per output with coalesced stores. A wave
// stays within 128 VGPRs and only the input band occupies LDS, so two
// workgroups (16 waves) share a CU and hide each other's latencies.
// Measured on MI355X (config 5): splitting a row over two workgroups (640
// of them, three per CU) is 16% slower, and giving each wave every channel
// block of its own outputs (no LDS sum) is 50% slower -- the weight loads
// then serialize.
#include "device_common.h"
#include "kernels.h"
#include "launch_once.h"

namespace vai_dev {

namespace cv {
constexpr int CO_TILE = 32;
constexpr int MAX_WO_FRAGS = 8;          // output row <= 128 positions
inline __host__ __device__ uint32_t ci32(uint32_t ci) { return (ci + 31) / 32 * 32; }
inline __host__ __device__ uint32_t cip(uint32_t ci) { return ci32(ci) + 8; }   // LDS row stride (halves)
}

// LDS of the input band, later reused by the cross-wave sum (the larger of
// the two); the epilogue's bias and scale follow it.
// (ct output channels per workgroup, nf 16-wide fragments of an output row)
__host__ __device__ inline size_t conv_main_lds_bytes(uint32_t ci, uint32_t wi, uint32_t ks, uint32_t ct = cv::CO_TILE,
                                                      uint32_t nf = cv::MAX_WO_FRAGS)
{
    const size_t WiP = wi + 2 * (ks / 2), CIP = cv::cip(ci);
    const size_t stage = (size_t)ks * WiP * CIP * 2;
    const size_t red = 4ull * ct * 16 * nf * 4;
    return stage > red ? stage : red;
}

// W [Co, C, k, k] (fp16) -> the fragment-major packed weight: for tap t,
// 16-channel output block o, 32-channel input block cb and MFMA lane l
// (output channel o*16 + l%16, input channels cb*32 + 8*(l/16) .. +7):
//   Wp[((t*CO16 + o)*NB + cb)*64 + l][0..7],  CO16 = ceil(Co/16), NB = C32/32
// so a wave's A fragment of one tap is 1 KB of contiguous memory. Padding
// output channels and input channels past C are zero. One workgroup per
// (padded) output channel: its C*k*k weights are read contiguously into LDS
// and written out in 16-byte chunks.
__global__ __launch_bounds__(256) void pack_weight_kernel(half_t* __restrict__ dst, const half_t* __restrict__ w,
                                                          uint32_t Co, uint32_t C, uint32_t C32, uint32_t kk)
{
    extern __shared__ half_t row[];
    const uint32_t co = blockIdx.x, CO16 = gridDim.x / 16, NB = C32 / 32;
    const size_t n = (size_t)C * kk;
    if (co < Co)
        for (size_t i = threadIdx.x; i < n; i += 256) row[i] = w[(size_t)co * n + i];
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kk * (C32 / 8); i += 256) {
        const uint32_t chunk = i % (C32 / 8), tap = i / (C32 / 8), cb = chunk / 4, fg = chunk % 4;
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t c = chunk * 8 + e;
            v[e] = (co < Co && c < C) ? row[(size_t)c * kk + tap] : (half_t)0;
        }
        const size_t lane = co % 16 + 16 * fg;
        *(half8*)(dst + ((((size_t)tap * CO16 + co / 16) * NB + cb) * 64 + lane) * 8) = v;
    }
}

// The activation of epilogue kind EPI (the same formulas as epilogue()).
template <int EPI>
__device__ __forceinline__ float cv_act(float x)
{
    if constexpr (EPI == 1) return x > 0.f ? x : 0.f;
    else if constexpr (EPI == 2) return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
    else if constexpr (EPI == 3) return 0.5f * x * (1.0f + fast_tanh(0.79788456080286535f * (x + 0.044715f * x * x * x)));
    else if constexpr (EPI == 4) return x * fast_rcp(1.0f + fast_exp(-x));
    else if constexpr (EPI == 5) return fast_rcp(1.0f + fast_exp(-x));
    else return x;
}

// conv_store's 16-byte form: 4 consecutive positions of one output channel
// per work item, four 16-byte partial-sum reads and one 16-byte (fp32) or
// 8-byte (fp16) store. A row of Wo outputs stays 16-byte aligned (Ho Wo and
// Wo are multiples of 4). The activation, the residual and the output dtype
// are template parameters: chosen per element at run time they left a
// branch in every output.
template <int CT, int EPI, bool RES, bool O16>
__device__ __forceinline__ void conv_store_vec4(const ConvParams& p, const float* red, uint32_t rw, const float* epi_bs,
                                                uint32_t co0, uint32_t ho, uint32_t b)
{
    constexpr int NT = CT / 4 * 64;
    const size_t HoWo = (size_t)p.ho * p.wo;
    const bool before = p.residual_order == 1;
    const uint32_t q4 = p.wo / 4, items = CT * q4;
    for (uint32_t it = threadIdx.x; it < items; it += NT) {
        const uint32_t col = it / q4, wo = (it % q4) * 4, co = co0 + col;
        if (co >= p.co) continue;
        float4v v = *(const float4v*)(red + (size_t)col * rw + wo);
#pragma unroll
        for (int w = 1; w < 4; ++w) v += *(const float4v*)(red + ((size_t)w * CT + col) * rw + wo);
        const float bias = p.bias ? epi_bs[col] : 0.f, sc = p.scale ? epi_bs[CT + col] : 1.f;
        const size_t o = ((size_t)b * p.co + co) * HoWo + (size_t)ho * p.wo + wo;
        float4v rr = (float4v)0.f;
        if constexpr (RES) {
            if (p.residual_dtype == DT_F16) rr = __builtin_convertvector(*(const half4*)((const half_t*)p.residual + o), float4v);
            else rr = *(const float4v*)((const float*)p.residual + o);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // (sc is 1 without a scale: fma(a, 1, b) is exactly a + b)
            float x = fmaf(v[e], sc, bias);
            if constexpr (RES) x += before ? rr[e] : 0.f;
            x = cv_act<EPI>(x);
            if constexpr (RES) x += before ? 0.f : rr[e];
            v[e] = x;
        }
        if constexpr (O16) *(half4*)((half_t*)p.out + o) = __builtin_convertvector(v, half4);
        else *(float4v*)((float*)p.out + o) = v;
    }
}

// Scale, bias, residual and activation of a workgroup's CT output channels
// x one output row, from the partial sums of its four channel-block waves in
// LDS (red[w][CT][rw], positions along a row), with stores per output row.
// CT * 16 threads (NW = CT / 4 waves).
template <int CT>
__device__ __forceinline__ void conv_store(const ConvParams& p, const float* red, uint32_t rw, const float* epi_bs,
                                           uint32_t co0, uint32_t ho, uint32_t b)
{
    using namespace cv;
    constexpr int NW = CT / 4, NT = NW * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int EPI_COLS = CT / NW;   // output channels per wave in the scalar path
    const size_t HoWo = (size_t)p.ho * p.wo;
    const bool vec4 = p.wo % 4 == 0 && (uintptr_t)p.out % 16 == 0 && (uintptr_t)p.residual % 16 == 0;
    if (vec4) {
        const bool res = p.residual != nullptr, o16 = p.o_dtype == DT_F16;
        auto go = [&](auto E) __attribute__((always_inline)) {
            if (res) {
                if (o16) conv_store_vec4<CT, E, true, true>(p, red, rw, epi_bs, co0, ho, b);
                else conv_store_vec4<CT, E, true, false>(p, red, rw, epi_bs, co0, ho, b);
            } else {
                if (o16) conv_store_vec4<CT, E, false, true>(p, red, rw, epi_bs, co0, ho, b);
                else conv_store_vec4<CT, E, false, false>(p, red, rw, epi_bs, co0, ho, b);
            }
        };
        switch (p.epilogue) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 5: go(std::integral_constant<int, 5>{}); break;
        default: go(std::integral_constant<int, 0>{}); break;
        }
        return;
    }
    // Outputs (co0 + wave + NW i, wo = lane + 64 k); residuals first, all
    // loads in flight together (indices clamped, unused values discarded).
    constexpr int EPI_W = MAX_WO_FRAGS * 16 / 64;
    float rv[EPI_COLS][EPI_W] = {};
    if (p.residual) {
        const bool r16 = p.residual_dtype == DT_F16;
#pragma unroll
        for (int i = 0; i < EPI_COLS; ++i)
#pragma unroll
            for (int k = 0; k < EPI_W; ++k) {
                const uint32_t co = min(co0 + wave + NW * i, p.co - 1), wo = min(lane + 64 * k, p.wo - 1);
                const size_t o = ((size_t)b * p.co + co) * HoWo + (size_t)ho * p.wo + wo;
                rv[i][k] = r16 ? (float)((const half_t*)p.residual)[o] : 0.f;
            }
        if (!r16) {
#pragma unroll
            for (int i = 0; i < EPI_COLS; ++i)
#pragma unroll
                for (int k = 0; k < EPI_W; ++k) {
                    const uint32_t co = min(co0 + wave + NW * i, p.co - 1), wo = min(lane + 64 * k, p.wo - 1);
                    rv[i][k] = ((const float*)p.residual)[((size_t)b * p.co + co) * HoWo + (size_t)ho * p.wo + wo];
                }
        }
    }
#pragma unroll
    for (int i = 0; i < EPI_COLS; ++i) {
        const uint32_t col = wave + NW * i, co = co0 + col;
        if (co >= p.co) break;
        const float bias = p.bias ? epi_bs[col] : 0.f, sc = p.scale ? epi_bs[CT + col] : 1.f;
        const size_t obase = ((size_t)b * p.co + co) * HoWo + (size_t)ho * p.wo;
#pragma unroll
        for (int k = 0; k < EPI_W; ++k) {
            const uint32_t wo = lane + 64 * k;
            if (wo >= p.wo) break;
            float v = red[(size_t)col * rw + wo] + red[((size_t)CT + col) * rw + wo] +
                      red[((size_t)2 * CT + col) * rw + wo] + red[((size_t)3 * CT + col) * rw + wo];
            v = p.scale ? fmaf(v, sc, bias) : v + bias;
            const float rr = rv[i][k];
            if (p.residual && p.residual_order == 1) v += rr;
            v = epilogue(v, p.epilogue);
            if (p.residual && p.residual_order == 0) v += rr;
            st(p.out, p.o_dtype, obase + wo, v);
        }
    }
}

template <int KS, int NF, typename TI, int CT>
__global__ __launch_bounds__(CT * 16) __attribute__((amdgpu_waves_per_eu(4))) void conv_kernel(ConvParams p)
{
    using namespace cv;
    constexpr int NT = CT * 16;   // threads: 4 channel blocks x CT / 16 output-channel groups, one wave each
    extern __shared__ half8 smem[];
    const uint32_t C32 = ci32(p.ci), CIP = cip(p.ci);
    constexpr int PAD = KS / 2;
    const uint32_t WiP = p.wi + 2 * PAD;
    half_t* xs = (half_t*)smem;                              // [KS][WiP][CIP]
    float* epi_bs = (float*)((char*)smem + conv_main_lds_bytes(p.ci, p.wi, KS, CT, NF));   // [bias x CT, scale x CT]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cw = wave & 3, half = wave >> 2;               // channel-block lane, output-channel half
    const uint32_t co0 = blockIdx.x * CT, ho = blockIdx.y, b = blockIdx.z;
    const int fr = lane & 15, fg = lane >> 4;
    const uint32_t nblk = C32 / 32;

    // A fragments straight from the packed weight (L2-resident, shared by all
    // blocks): issued first so their latency hides behind the input staging.
    half8 wa[KS * KS];
    const uint32_t CO16 = (p.co + 15) / 16, oblk = min(blockIdx.x * (CT / 16) + half, CO16 - 1);   // past Co: discarded
    auto load_w = [&](uint32_t cb) {
#pragma unroll
        for (int tap = 0; tap < KS * KS; ++tap)
            wa[tap] = *(const half8*)(p.wp + ((((size_t)tap * CO16 + oblk) * nblk + cb) * 64 + lane) * 8);
    };
    if ((uint32_t)cw < nblk) load_w(cw);

    // ---- input rows: NCHW -> LDS [row][pad + w][c] ----
    // Work item = 8 channels x 8 columns of one input row: eight 16-byte
    // (fp16) row loads, a transpose in registers, eight 16-byte LDS writes
    // (one per column, 8 consecutive channels = one MFMA operand chunk).
    // Items are ordered channel group fastest: the 16 lanes of a column
    // group write one contiguous 256-byte channel run (all 64 banks), and a
    // load instruction reads 64-byte runs of 16 channel rows.
    {
        const uint32_t ngc = C32 / 8, ngw = (p.wi + 7) / 8, items = KS * ngc * ngw;
        const size_t plane = (size_t)p.hi * p.wi;
        // (channel offsets up to C32 planes, plus 2^31 for a row outside the
        // image, must stay 32-bit and past the resource's end)
        const bool vec = p.wi % 8 == 0 && ((uintptr_t)p.x % (8 * sizeof(TI))) == 0 &&
                         (size_t)C32 * plane * sizeof(TI) < (1ull << 31);
        const uint32_t plane_bytes = (uint32_t)(plane * sizeof(TI));
        const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const TI*)p.x + (size_t)b * p.ci * plane), (short)0,
            (int)std::min<size_t>((size_t)p.ci * plane * sizeof(TI), 0x7FFFFFFF), 0x00020000);
        for (uint32_t it = tid; it < items; it += NT) {
            const uint32_t cg = it % ngc, rest = it / ngc, wg = rest % ngw, r = rest / ngw;
            const int hi = (int)(ho * p.stride) + (int)r - PAD;
            const bool row_ok = hi >= 0 && hi < (int)p.hi;
            const uint32_t c0 = cg * 8, w0 = wg * 8;
            half8 col[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) col[j] = (half8)(half_t)0;
            if (vec && sizeof(TI) == 2) {
                // eight 16-byte loads issued together through a resource over
                // the image: channels past Ci fall outside it, and so does a
                // row outside the image, whose offset is 2^31 plus the channel's
                // (the image is under 2^31 bytes), so the hardware bounds check
                // returns their zeros. (Guarded loads would each wait out a
                // full memory latency.)
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const uint32_t rowoff = row_ok ? (uint32_t)(hi * (int)p.wi + (int)w0) * 2u : 0x80000000u;
                u32x4 t[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    t[e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         xrsrc, (int)(rowoff + (c0 + e) * plane_bytes), 0, 0));
                __builtin_amdgcn_sched_barrier(0);   // all eight issued before the first use
                // transpose: column j's channel pair (2k, 2k + 1) is one dword,
                // the j-th halves of channel 2k's and 2k + 1's column runs
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    u32x4 v;
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        v[k] = __builtin_amdgcn_perm(t[2 * k + 1][j / 2], t[2 * k][j / 2],
                                                     (j & 1) ? 0x07060302u : 0x05040100u);
                    col[j] = __builtin_bit_cast(half8, v);
                }
            } else if (row_ok) {
                // (fp32 input: eight 32-byte rows at once would not fit the
                // register budget; one channel at a time)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (c0 + e >= p.ci) continue;
                    const TI* src = (const TI*)p.x + ((size_t)b * p.ci + c0 + e) * plane + (size_t)hi * p.wi + w0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) col[j][e] = w0 + j < p.wi ? (half_t)src[j] : (half_t)0;
                }
            }
            half_t* dst = xs + ((size_t)r * WiP + PAD + w0) * CIP + c0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (w0 + j < p.wi) *(half8*)(dst + (size_t)j * CIP) = col[j];
        }
        // the zero padding columns
        for (uint32_t i = tid; i < (uint32_t)(KS * 2 * PAD) * (C32 / 8); i += NT) {
            const uint32_t cg = i % (C32 / 8), rc = i / (C32 / 8), r = rc / (2 * PAD), e = rc % (2 * PAD);
            const uint32_t w = e < PAD ? e : PAD + p.wi + (e - PAD);
            *(half8*)(xs + ((size_t)r * WiP + w) * CIP + cg * 8) = (half8)(half_t)0;
        }
        // bias and scale of the tile's output channels, for the epilogue
        // (unconditional loads: a missing one reads the packed weight, at
        // least Co values long, and the epilogue ignores it)
        if (tid < 2 * CT) {
            const half_t* src = tid < CT ? (p.bias ? (const half_t*)p.bias : p.wp)
                                         : (p.scale ? (const half_t*)p.scale : p.wp);
            epi_bs[tid] = (float)src[min(co0 + (tid % CT), p.co - 1)];
        }
    }
    __syncthreads();

    // ---- MFMAs: 16 output channels x the row, this wave's channel blocks ----
    constexpr int nf = NF;                                   // output-position fragments (compile time:
                                                             // a runtime count makes the loop nest spill)
    float4v acc[MAX_WO_FRAGS];
#pragma unroll
    for (int f = 0; f < MAX_WO_FRAGS; ++f) acc[f] = (float4v)0.f;
    uint32_t wo_s[MAX_WO_FRAGS];
#pragma unroll
    for (int f = 0; f < MAX_WO_FRAGS; ++f) wo_s[f] = min((uint32_t)(f * 16 + fr), p.wo - 1) * p.stride;
    for (uint32_t cb = cw; cb < nblk; cb += 4) {
        if (cb != (uint32_t)cw) load_w(cb);
        const uint32_t cofs = cb * 32 + fg * 8;
#pragma unroll
        for (int kh = 0; kh < KS; ++kh)
#pragma unroll
            for (int kw = 0; kw < KS; ++kw) {
                const half_t* xrow = xs + ((size_t)kh * WiP + kw) * CIP + cofs;
#pragma unroll
                for (int f = 0; f < MAX_WO_FRAGS; ++f) {
                    if (f < nf) {
                        const half8 bv = *(const half8*)(xrow + (size_t)wo_s[f] * CIP);
                        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[kh * KS + kw], bv, acc[f], 0, 0, 0);
                    }
                }
            }
    }
    __syncthreads();

    // ---- cross-wave sum in LDS, then the epilogue ----
    // D[i][j] of a 16x16 fragment sits in lane j + 16*(i/4), register i%4.
    float* red = (float*)smem;                               // [4 channel lanes][CT co][16*nf positions]
    const uint32_t rw = (uint32_t)nf * 16;
#pragma unroll
    for (int f = 0; f < MAX_WO_FRAGS; ++f)
        if (f < nf)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[((size_t)cw * CT + half * 16 + fg * 4 + r) * rw + f * 16 + fr] = acc[f][r];
    __syncthreads();
    conv_store<CT>(p, red, rw, epi_bs, co0, ho, b);
}

// ---- 3x3, stride 1, fp16 NCHW input, row width 16 NF (config 5's shape) ----
// The input rows go global -> LDS unchanged, by buffer_load ... lds (each
// channel's rows are contiguous halves in NCHW as in LDS), and the transpose
// to channel-major MFMA operands happens in the LDS read: ds_read_b64_tr_b16
// gives lane j of a 16-lane group 4 consecutive channels of column j, where
// source lane 4 k + q points at channel k, columns 4 q .. +3 (two reads: the
// lane's 8 channels). A B fragment (32 channels x 16 columns, unshifted)
// serves all three kw taps: tap kw accumulates into its own P_kw, and the
// taps meet at the end shifted by one column,
//   out(x) = P_0(x - 1) + P_1(x) + P_2(x + 1),
// the shift a DPP row rotation (a fragment's 16 columns are the 16 lanes of
// a row) with the edge column taken from the neighbouring fragment, zero at
// the image border (the padding). This replaces the VALU transpose of the
// general kernel's staging.
//
// A workgroup covers CT = 32 or 64 output channels x one output row with
// CT / 4 waves (channel block lane, 16-channel output group), as the general
// kernel at CT = 32. (Two rows per workgroup, with the weight fragments
// copied into LDS once for both, halve the bytes per row but leave 96 of the
// 256 CUs idle at config 5: 9.1 against 8.3 us.)
__host__ __device__ constexpr uint32_t conv3_stage_bytes(uint32_t c32, uint32_t nf) { return c32 * 96 * nf; }
template <int CT>
__host__ __device__ inline size_t conv3_main_lds_bytes(uint32_t c32, uint32_t nf)
{
    const size_t red = 4ull * CT * 16 * nf * 4;
    return conv3_stage_bytes(c32, nf) > red ? conv3_stage_bytes(c32, nf) : red;
}
template <int CT>
__host__ __device__ inline size_t conv3_lds_bytes(uint32_t c32, uint32_t nf)
{
    return conv3_main_lds_bytes<CT>(c32, nf) + 2 * CT * sizeof(float);
}

// The C32 channels x 3 rows x WI columns of image b around output row ho
// into LDS, in 1 KB copies per wave instruction: byte pos of the stage is
// channel pos / CHB, row (pos % CHB) / ROWB, column bytes the rest. Rows
// outside the image and channels past Ci read as zero (offset 2^31, or past
// the resource's end; C32 planes stay under 2^31 bytes, so no offset wraps).
template <int NF, int NW>
__device__ __forceinline__ void conv3_stage(const ConvParams& p, __attribute__((address_space(3))) char* xs,
                                            uint32_t c32, uint32_t ho, uint32_t b, int wave, int lane)
{
    constexpr uint32_t ROWB = 32 * NF, CHB = 3 * ROWB;
    const uint32_t plane_bytes = p.hi * ROWB;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const half_t*)p.x + (size_t)b * p.ci * p.hi * (16 * NF)), (short)0, (int)(p.ci * plane_bytes),
        0x00020000);
    const uint32_t n = c32 * CHB;
    for (uint32_t i0 = (uint32_t)wave * 1024; i0 < n; i0 += NW * 1024) {
        const uint32_t pos = i0 + (uint32_t)lane * 16, c = pos / CHB, w = pos % CHB, r = w / ROWB;
        const int hi = (int)ho + (int)r - 1;
        const uint32_t off = (hi >= 0 && hi < (int)p.hi) ? c * plane_bytes + (uint32_t)hi * ROWB + w % ROWB
                                                          : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(xs + i0), 16, (int)off,
                                                 0, 0, 0);
    }
}

typedef __fp16 cv_fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));

__device__ __forceinline__ half4 cv_read_tr16(const __attribute__((address_space(3))) char* a)
{
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         (__attribute__((address_space(3))) cv_fp16x4*)a));
}

// x of lane (j - 1) of its 16-lane row (k = 1), or of lane (j + 1) (k = 15).
template <int K>
__device__ __forceinline__ float cv_row_ror(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + K, 0xF, 0xF,
                                                                 false));
}

// The epilogue: 8 consecutive positions of one output channel per thread
// (32 x 2 NF items, one pass): the residual loads first, then the four
// partial sums from LDS, scale and bias, the activation chosen once per
// thread (EPI), and one 32-byte (fp32) or 16-byte (fp16) store.
template <int EPI>
__device__ __forceinline__ void cv_finish8(float8v& v, const float8v& rr, bool res, uint32_t order, float sc, float bias,
                                           bool scaled)
{
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float x = scaled ? fmaf(v[e], sc, bias) : v[e] + bias;
        if (res && order == 1) x += rr[e];
        x = cv_act<EPI>(x);
        if (res && order == 0) x += rr[e];
        v[e] = x;
    }
}

template <int NF, int CT>
__device__ __forceinline__ void conv3_store(const ConvParams& p, const float* red, const float* epi_bs, uint32_t co0,
                                            uint32_t ho, uint32_t b)
{
    constexpr uint32_t RW = NF * 16, Q8 = 2 * NF;
    const uint32_t it = threadIdx.x;
    if (it >= CT * Q8) return;
    const uint32_t col = it / Q8, wo = (it % Q8) * 8, co = co0 + col;
    if (co >= p.co) return;
    const size_t o = ((size_t)b * p.co + co) * ((size_t)p.ho * RW) + (size_t)ho * RW + wo;
    const bool res = p.residual != nullptr;
    float8v rr = (float8v)0.f;
    if (res) {
        if (p.residual_dtype == DT_F16) rr = __builtin_convertvector(*(const half8*)((const half_t*)p.residual + o), float8v);
        else rr = *(const float8v*)((const float*)p.residual + o);
    }
    const float* rp = red + (size_t)col * RW + wo;
    float8v v = *(const float8v*)rp;
#pragma unroll
    for (int w = 1; w < 4; ++w) v += *(const float8v*)(rp + (size_t)w * CT * RW);
    const float bias = p.bias ? epi_bs[col] : 0.f, sc = epi_bs[CT + col];
    const bool scaled = p.scale != nullptr;
    switch (p.epilogue) {
    case 1: cv_finish8<1>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    case 2: cv_finish8<2>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    case 3: cv_finish8<3>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    case 4: cv_finish8<4>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    case 5: cv_finish8<5>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    default: cv_finish8<0>(v, rr, res, p.residual_order, sc, bias, scaled); break;
    }
    if (p.o_dtype == DT_F16) *(half8*)((half_t*)p.out + o) = __builtin_convertvector(v, half8);
    else *(float8v*)((float*)p.out + o) = v;
}

template <int NF, int CT>
__global__ __launch_bounds__(CT * 16) __attribute__((amdgpu_waves_per_eu(4))) void conv3_tr_kernel(ConvParams p)
{
    constexpr int NW = CT / 4;   // waves: 4 channel blocks x CT / 16 output-channel groups
    using namespace cv;
    constexpr uint32_t ROWB = 32 * NF, CHB = 3 * ROWB;
    extern __shared__ half8 smem[];
    __attribute__((address_space(3))) char* xs = (__attribute__((address_space(3))) char*)(
        __attribute__((address_space(3))) void*)smem;
    const uint32_t C32 = ci32(p.ci), nblk = C32 / 32;
    float* epi_bs = (float*)((char*)smem + conv3_main_lds_bytes<CT>(C32, NF));   // [bias x 32, scale x 32]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cw = wave & 3, half = wave >> 2;   // channel-block lane, output-channel half
    const uint32_t co0 = blockIdx.x * CT, ho = blockIdx.y, b = blockIdx.z;
    const int fr = lane & 15, fg = lane >> 4;

    // the nine taps' A fragments of channel block cb (issued before the staging)
    half8 wa[9];
    const uint32_t CO16 = (p.co + 15) / 16, oblk = min(blockIdx.x * (CT / 16) + half, CO16 - 1);   // past Co: discarded
    auto load_w = [&](uint32_t cb) {
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
            wa[tap] = *(const half8*)(p.wp + ((((size_t)tap * CO16 + oblk) * nblk + cb) * 64 + lane) * 8);
    };
    if ((uint32_t)cw < nblk) load_w(cw);
    conv3_stage<NF, NW>(p, xs, C32, ho, b, wave, lane);
    if (tid < 2 * CT) {   // bias and scale (a missing one reads the packed weight; ignored)
        const half_t* src = tid < CT ? (p.bias ? (const half_t*)p.bias : p.wp)
                                     : (p.scale ? (const half_t*)p.scale : p.wp);
        epi_bs[tid] = (float)src[min(co0 + (tid % CT), p.co - 1)];
    }
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));   // vmcnt(0): copies landed
    __syncthreads();

    float4v P[3][NF];
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int f = 0; f < NF; ++f) P[k][f] = (float4v)0.f;
    for (uint32_t cb = cw; cb < nblk; cb += 4) {
        if (cb != (uint32_t)cw) load_w(cb);
        // source lane (k, q) = (fr / 4, fr % 4) of group fg: channel cb 32 + 8 fg + k, columns 4 q ..
        const __attribute__((address_space(3))) char* base = xs + (cb * 32 + 8 * fg + (fr >> 2)) * CHB + (fr & 3) * 8;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const half4 lo = cv_read_tr16(base + kh * ROWB + f * 32);
                const half4 hi = cv_read_tr16(base + 4 * CHB + kh * ROWB + f * 32);
                const half8 bv = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int kw = 0; kw < 3; ++kw)
                    P[kw][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[kh * 3 + kw], bv, P[kw][f], 0, 0, 0);
            }
    }
    // the taps combined: column j of fragment f is lane fr = j of each row
    float4v acc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float a0 = cv_row_ror<1>(P[0][f][r]);
            const float e0 = f > 0 ? cv_row_ror<1>(P[0][f > 0 ? f - 1 : 0][r]) : 0.f;
            const float a2 = cv_row_ror<15>(P[2][f][r]);
            const float e2 = f + 1 < NF ? cv_row_ror<15>(P[2][f + 1 < NF ? f + 1 : f][r]) : 0.f;
            acc[f][r] = P[1][f][r] + (fr == 0 ? e0 : a0) + (fr == 15 ? e2 : a2);
        }
    __syncthreads();   // every wave done reading the stage before the sums overwrite it
    float* red = (float*)smem;   // [4 channel lanes][32 co][16 NF positions]
    constexpr uint32_t rw = NF * 16;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((size_t)cw * CT + half * 16 + fg * 4 + r) * rw + f * 16 + fr] = acc[f][r];
    __syncthreads();
    conv3_store<NF, CT>(p, red, epi_bs, co0, ho, b);
}

// ---- the pipelined form, for up to four 32-channel input blocks ----
// The same LDS transpose and tap shift, but each wave owns 16 output
// channels x the whole row over every input-channel block, so no partial sums
// meet in LDS and the epilogue runs from the accumulators. A workgroup (4
// waves, 64 output channels x one output row) reads, per block j, the wave's
// nine weight fragments and its share of the block's input rows (CPW 1 KB
// copies, the block padded to 4 KB per wave so that every wave issues the
// same count): 9 + CPW operations. Blocks 0 and 1 are issued at entry; the
// operations of block j + 2 are spread over block j's MFMA steps, one per
// step, so that they queue behind MFMAs instead of holding the wave at entry
// (a CU's vector memory path takes a wave about 100 cycles per 1 KB
// operation here, and a block's MFMAs about 1,100 cycles). Block j starts
// when the wave's own operations of block j have landed (a counted vmcnt:
// only block j + 1's 9 + CPW, issued during block j - 1, may still be in
// flight) and every wave has passed that point (s_barrier). Blocks occupy
// LDS regions of their own, so no copy waits for a reader. The B fragments
// are read by inline asm, which the compiler's wait insertion does not see
// (its own ds_read_b64_tr_b16 would wait for every LDS copy in flight); a
// ring of DPF steps is in flight ahead of the MFMAs, lgkmcnt counting the
// reads issued since. The loop issues no scalar loads (they share lgkmcnt)
// and the issue points are scheduling barriers, so the counts hold as
// written. The MFMA takes the input fragment as A and the weight as B, so a
// lane's accumulator registers hold four consecutive output columns of one
// channel (a 16-byte store each).
// Measured at config 5 (MI355X, 100-launch graph): 6.08-6.15 us; all of
// every block issued at entry 6.45-6.54 (same runs), the four-channel-block-
// waves form above 7.35. Per-wave timestamps (cycles, median): entry to the
// first two blocks issued 2,300, block compute 1,090 (1,400-1,700 with the
// next block's operations interleaved), the last block plus the tap shift
// and the epilogue 3,300. Variants that measured no better: 8 waves splitting
// the blocks in two with an LDS sum (6.97), 32 output channels per workgroup
// so that 320 of them cover every CU (7.09), the epilogue through an LDS tile
// (7.46), deeper read rings (DPF 5, 7: 7.06, 7.09), copy offsets computed
// once for all blocks (6.94), and four more waves that only load, with the
// weight fragments through a three-slot LDS ring (6.55: the weights' LDS
// writes and reads, 72 KB per block, made each block about 1,300 cycles,
// and a loading wave cannot release a landed block while it is held
// issuing the next).
namespace cvp {
template <int NF> struct Geo {
    static constexpr uint32_t ROWB = 32 * NF;              // bytes per staged row (16 NF fp16 columns)
    static constexpr uint32_t CHB = 3 * ROWB;              // bytes per channel (3 rows)
    static constexpr uint32_t BLK = 32 * CHB;              // bytes of one 32-channel block
    static constexpr uint32_t CPW = (BLK + 4095) / 4096;   // 1 KB copies per wave (4 waves) and block
    static constexpr uint32_t CBB = CPW * 4096;            // LDS bytes per block
};
constexpr int DPF = 3;   // B steps in flight ahead of the MFMAs (6 reads)
}

template <int OFF>
__device__ __forceinline__ half4 cv_tr16_asm(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    half4 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}
__device__ __forceinline__ void cv_pin(half4& v) { asm volatile("" : "+v"(v)); }
template <int N>
__device__ __forceinline__ void cv_lgkm_wait()
{
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}
template <int N>
__device__ __forceinline__ void cv_vm_wait()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// The epilogue from the accumulators: lane (cl, g) holds output channel co
// (cl = lane % 16 of the wave's 16) at positions 16 f + 4 g .. +3 of each
// fragment f, so one 16-byte (fp32) or 8-byte (fp16) store writes four
// consecutive outputs, and each store instruction 16 channels x 64 bytes.
// Residual loads go first (all in flight), then the values and the stores;
// RES and O16 are template flags, so the straight-line code carries no
// per-element branches. (With the channels across the accumulator's
// registers instead, the same outputs took four 4-byte stores each: 20
// store instructions per wave, and the epilogue about 2,200 of a wave's
// 10,500 cycles at config 5.)
template <int EPI, bool RES, bool O16, int NF>
__device__ __forceinline__ void conv3_pipe_store(const ConvParams& p, float4v (&acc)[NF], float bias, float sc,
                                                 uint32_t co, uint32_t ho, uint32_t b, int g)
{
    if (co >= p.co) return;
    const bool before = p.residual_order == 1;
    const size_t o0 = (((size_t)b * p.co + co) * p.ho + ho) * p.wo + 4 * g;
    float4v rr[NF];
    if constexpr (RES) {
#pragma unroll
        for (int f = 0; f < NF; ++f)
            rr[f] = p.residual_dtype == DT_F16
                        ? __builtin_convertvector(*(const half4*)((const half_t*)p.residual + o0 + 16 * f), float4v)
                        : *(const float4v*)((const float*)p.residual + o0 + 16 * f);
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        float4v v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // (sc is 1 without a scale: fma(a, 1, b) is exactly a + b)
            float x = fmaf(acc[f][r], sc, bias);
            if constexpr (RES) x += before ? rr[f][r] : 0.f;
            x = cv_act<EPI>(x);
            if constexpr (RES) x += before ? 0.f : rr[f][r];
            v[r] = x;
        }
        if constexpr (O16) *(half4*)((half_t*)p.out + o0 + 16 * f) = __builtin_convertvector(v, half4);
        else *(float4v*)((float*)p.out + o0 + 16 * f) = v;
    }
}

template <int EPI, int NF>
__device__ __forceinline__ void conv3_pipe_store_sel(const ConvParams& p, float4v (&acc)[NF], float bias, float sc,
                                                     uint32_t co, uint32_t ho, uint32_t b, int g)
{
    const bool res = p.residual != nullptr, o16 = p.o_dtype == DT_F16;
    if (res) {
        if (o16) conv3_pipe_store<EPI, true, true>(p, acc, bias, sc, co, ho, b, g);
        else conv3_pipe_store<EPI, true, false>(p, acc, bias, sc, co, ho, b, g);
    } else {
        if (o16) conv3_pipe_store<EPI, false, true>(p, acc, bias, sc, co, ho, b, g);
        else conv3_pipe_store<EPI, false, false>(p, acc, bias, sc, co, ho, b, g);
    }
}

// The taps combined: output column x = 16 f + 4 fg + r takes P[1] at x,
// P[0] at x - 1 and P[2] at x + 1. Inside a lane's four registers that is a
// register index; the first P[0] and the last P[2] term come from the
// neighbouring position group (lane -16, resp. +16, mod 64), which for the
// fragment's first (last) group is the previous (next) fragment's last
// (first) group; past the row's ends they are the zero padding. Each lane
// offers the value its neighbour needs, one bpermute each way. Then the
// epilogue.
template <int NF>
__device__ __forceinline__ void conv3_taps_store(const ConvParams& p, float4v (&P)[3][NF], float bias, float sc,
                                                 uint32_t co, uint32_t ho, uint32_t b, int fg, int lane)
{
    const int src_lo = ((lane + 48) & 63) * 4, src_hi = ((lane + 16) & 63) * 4;
    float4v acc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const float off0 = fg == 3 ? (f > 0 ? P[0][f > 0 ? f - 1 : 0][3] : 0.f) : P[0][f][3];
        const float off2 = fg == 0 ? (f + 1 < NF ? P[2][f + 1 < NF ? f + 1 : f][0] : 0.f) : P[2][f][0];
        const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lo, __builtin_bit_cast(int, off0)));
        const float x2 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_hi, __builtin_bit_cast(int, off2)));
        acc[f][0] = P[1][f][0] + x0 + P[2][f][1];
        acc[f][1] = P[1][f][1] + P[0][f][0] + P[2][f][2];
        acc[f][2] = P[1][f][2] + P[0][f][1] + P[2][f][3];
        acc[f][3] = P[1][f][3] + P[0][f][2] + x2;
    }
    switch (p.epilogue) {
    case 1: conv3_pipe_store_sel<1, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    case 2: conv3_pipe_store_sel<2, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    case 3: conv3_pipe_store_sel<3, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    case 4: conv3_pipe_store_sel<4, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    case 5: conv3_pipe_store_sel<5, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    default: conv3_pipe_store_sel<0, NF>(p, acc, bias, sc, co, ho, b, fg); break;
    }
}

// The common epilogues (none, SiLU; no residual) as a kernel parameter and
// without a branch: the output dtype picks one of two buffer resources, the
// other holding no bytes (its store is dropped by the range check), as is a
// lane past Co. With no branch in it, one fragment's output can be stored in
// the middle of the last block's MFMA steps without the control flow that
// would make the compiler's waits conservative around it. (A runtime choice
// of the activation, as a select or as bit masks, cost 0.2-1 us at config 5.)
typedef uint32_t cv_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t cv_u32x2 __attribute__((ext_vector_type(2)));
struct Conv3CheapOut {
    __amdgpu_buffer_rsrc_t o32, o16;
    // element index of the lane's first output of fragment 0, 2^28 for a
    // lane past Co: its byte offsets (2^30 fp32, 2^29 fp16) then lie past
    // either resource's range, which the plan keeps under 2^30 bytes
    uint32_t o;
    float bias, sc;
};

template <int NF, int F, int EPI>
__device__ __forceinline__ void conv3_tap_frag_cheap(const Conv3CheapOut& c, float4v (&P)[3][NF], int fg, int lane)
{
    constexpr int f = F;
    const int src_lo = ((lane + 48) & 63) * 4, src_hi = ((lane + 16) & 63) * 4;
    const float off0 = fg == 3 ? (f > 0 ? P[0][f > 0 ? f - 1 : 0][3] : 0.f) : P[0][f][3];
    const float off2 = fg == 0 ? (f + 1 < NF ? P[2][f + 1 < NF ? f + 1 : f][0] : 0.f) : P[2][f][0];
    const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lo, __builtin_bit_cast(int, off0)));
    const float x2 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_hi, __builtin_bit_cast(int, off2)));
    float4v acc;
    acc[0] = P[1][f][0] + x0 + P[2][f][1];
    acc[1] = P[1][f][1] + P[0][f][0] + P[2][f][2];
    acc[2] = P[1][f][2] + P[0][f][1] + P[2][f][3];
    acc[3] = P[1][f][3] + P[0][f][2] + x2;
    float4v v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = cv_act<EPI>(fmaf(acc[r], c.sc, c.bias));
    const uint32_t e = c.o + 16 * f;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(cv_u32x4, v), c.o32, (int)(e * 4), 0, 0);
    const half4 h = __builtin_convertvector(v, half4);
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(cv_u32x2, h), c.o16, (int)(e * 2), 0, 0);
}

// The epilogue kind of the cheap form (-1: the general epilogue): its
// 16-byte (8-byte fp16) stores need a 16-byte aligned output, and the
// output's byte offsets must fit the buffer resources' 31 bits.
static int conv_cheap_kind(const ConvParams& p)
{
    const int k = p.epilogue;
    const bool fits = (size_t)p.batch * p.co * p.ho * p.wo * 4 < (1ull << 30);
    return !p.residual && fits && (uintptr_t)p.out % 16 == 0 && (k == 0 || k == 4) ? k : -1;
}

template <int NF, int NB, int EK>
__global__ __launch_bounds__(256) void conv3_pipe_kernel(const half_t* wp, const void* x, const void* bias_p,
                                                         const void* scale_p, uint32_t co_n, uint32_t ci_n,
                                                         uint32_t hi_n, ConvParams pk)
{
    // what the entry's loads need, as leading scalar arguments (preloaded
    // into SGPRs at launch); the rest of the parameters from the struct
    ConvParams p = pk;
    p.wp = wp; p.x = x; p.bias = bias_p; p.scale = scale_p; p.co = co_n; p.ci = ci_n; p.hi = hi_n;
    using G = cvp::Geo<NF>;
    using cvp::DPF;
    constexpr uint32_t ROWB = G::ROWB, CHB = G::CHB, CPW = G::CPW, CBB = G::CBB;
    constexpr int S = 3 * NF;        // B steps per block: (kh, fragment)
    constexpr int NW = 4;            // waves
    extern __shared__ half8 smem[];
    __attribute__((address_space(3))) char* xs = (__attribute__((address_space(3))) char*)(
        __attribute__((address_space(3))) void*)smem;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = wave;   // output-channel group
    const uint32_t co0 = blockIdx.x * 64, ho = blockIdx.y, b = blockIdx.z;
    const int fr = lane & 15, fg = lane >> 4;
    const uint32_t CO16 = (p.co + 15) / 16, oblk = min(blockIdx.x * 4 + g, CO16 - 1);   // past Co: discarded
    // accumulator layout (the MFMA takes the input as A and the weight as
    // B): lane (fr, fg) holds output channel co at positions 4 fg .. +3 of
    // each 16-wide fragment, one per register
    const uint32_t co = co0 + g * 16 + fr;

    // bias and scale of the lane's channel (a missing one reads the packed
    // weight, at least Co values long, and is ignored)
    float bias, sc;
    {
        const half_t* bsrc = p.bias ? (const half_t*)p.bias : p.wp;
        const half_t* ssrc = p.scale ? (const half_t*)p.scale : p.wp;
        const uint32_t cc = min(co, p.co - 1);
        const float bv = (float)bsrc[cc], sv = (float)ssrc[cc];   // unconditional: no branch, no early wait
        bias = p.bias ? bv : 0.f;
        sc = p.scale ? sv : 1.f;
    }

    // Block j: this wave's weight fragments, then its share of the block's
    // copies (9 + CPW operations).
    const uint32_t plane_bytes = p.hi * ROWB;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const half_t*)p.x + (size_t)b * p.ci * p.hi * (16 * NF)), (short)0, (int)(p.ci * plane_bytes),
        0x00020000);
    half8 wa[NB][9];
    // operation i of block j (9 + CPW per block): weight fragment i, then copy i - 9
    auto issue_op = [&](auto J, auto I) __attribute__((always_inline)) {
        constexpr int j = J, i = I;
        if constexpr (i < 9) {
            wa[j][i] = *(const half8*)(p.wp + ((((size_t)i * CO16 + oblk) * NB + j) * 64 + lane) * 8);
        } else {
            constexpr uint32_t k = i - 9;
            const uint32_t i0 = (k * NW + (uint32_t)wave) * 1024, pos = i0 + (uint32_t)lane * 16;
            const uint32_t c = j * 32 + pos / CHB, w = pos % CHB, r = w / ROWB;
            const int hi = (int)ho + (int)r - 1;
            const uint32_t off = (pos < G::BLK && hi >= 0 && hi < (int)p.hi)
                                     ? c * plane_bytes + (uint32_t)hi * ROWB + w % ROWB
                                     : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(xs + j * CBB + i0),
                                                     16, (int)off, 0, 0, 0);
        }
    };
    constexpr int OPS = 9 + (int)CPW;
    // blocks 0 and 1 up front; block j + 2 is issued during block j's MFMAs
    static_for<(NB < 2 ? NB : 2)>([&](auto J) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        static_for<OPS>([&](auto I) __attribute__((always_inline)) { issue_op(J, I); });
        __builtin_amdgcn_sched_barrier(0);
    });

    float4v P[3][NF];
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int f = 0; f < NF; ++f) P[k][f] = (float4v)0.f;
    constexpr bool CHEAP = EK >= 0;   // the cheap epilogue, activation EK
    Conv3CheapOut cheap;
    if constexpr (CHEAP) {
        const uint32_t bytes = p.batch * p.co * p.ho * p.wo * 4;
        const bool o16 = p.o_dtype == DT_F16;
        cheap.o32 = __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, o16 ? 0 : (int)bytes, 0x00020000);
        cheap.o16 = __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, o16 ? (int)(bytes / 2) : 0, 0x00020000);
        cheap.o = co < p.co ? ((b * p.co + co) * p.ho + ho) * p.wo + 4 * fg : 0x10000000u;
        cheap.bias = bias;
        cheap.sc = sc;
    }
    // B source lane (k, q) = (fr / 4, fr % 4) of group fg: channel 8 fg + k of
    // the block, columns 4 q ..; the high half 4 channels on
    const uint32_t lbase =
        (uint32_t)reinterpret_cast<uintptr_t>(xs) + (8 * fg + (fr >> 2)) * CHB + (fr & 3) * 8;
    static_for<NB>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = J;
        // this wave's operations of block j have landed (only block j + 1's,
        // issued during block j - 1, may be outstanding) ...
        cv_vm_wait<(j + 1 < NB ? OPS : 0)>();
        __builtin_amdgcn_s_barrier();               // ... and every other wave's
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t base = lbase + j * CBB;
        half4 lo[S], hi[S];
        auto rd = [&](auto SS) __attribute__((always_inline)) {
            constexpr int s = SS, kh = s / NF, f = s % NF;
            lo[s] = cv_tr16_asm<kh * ROWB + f * 32>(base);
            hi[s] = cv_tr16_asm<4 * CHB + kh * ROWB + f * 32>(base);
        };
        static_for<DPF>([&](auto SS) __attribute__((always_inline)) { rd(SS); });
        static_for<S>([&](auto SS) __attribute__((always_inline)) {
            constexpr int s = SS, kh = s / NF, f = s % NF;
            if constexpr (s + DPF < S) rd(std::integral_constant<int, s + DPF>{});
            constexpr int later = (S - 1 - s) < DPF ? (S - 1 - s) : DPF;   // steps read after this one
            cv_lgkm_wait<2 * later>();
            cv_pin(lo[s]);
            cv_pin(hi[s]);
            const half8 bv = __builtin_shufflevector(lo[s], hi[s], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int kw = 0; kw < 3; ++kw)
                P[kw][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bv, wa[j][kh * 3 + kw], P[kw][f], 0, 0, 0);
            // one operation of block j + 2 per step, so that its loads queue
            // behind the MFMAs instead of ahead of them
            if constexpr (j + 2 < NB) {
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (s < OPS) issue_op(std::integral_constant<int, j + 2>{}, SS);
                if constexpr (s == S - 1 && S < OPS)
                    static_for<OPS - S>([&](auto I) __attribute__((always_inline)) {
                        issue_op(std::integral_constant<int, j + 2>{}, std::integral_constant<int, S + I>{});
                    });
                __builtin_amdgcn_sched_barrier(0);
            }
            // cheap epilogue: in the last block, fragment f's taps are all
            // issued at step 2 NF + f, and fragment f - 1 then has every
            // value it needs; its stores leave while the MFMAs go on
            if constexpr (CHEAP && j + 1 == NB && kh == 2 && f > 0) {
                __builtin_amdgcn_sched_barrier(0);
                conv3_tap_frag_cheap<NF, (f > 0 ? f - 1 : 0), (EK >= 0 ? EK : 0)>(cheap, P, fg, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
        __builtin_amdgcn_sched_barrier(0);
    });

    if constexpr (CHEAP) conv3_tap_frag_cheap<NF, NF - 1, (EK >= 0 ? EK : 0)>(cheap, P, fg, lane);
    else conv3_taps_store<NF>(p, P, bias, sc, co, ho, b, fg, lane);
}

template <int NF, int NB, int EK>
static hipError_t launch_pipe_form(const ConvParams& p, hipStream_t s)
{
    constexpr uint32_t lds = NB * cvp::Geo<NF>::CBB;
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)conv3_pipe_kernel<NF, NB, EK>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((conv3_pipe_kernel<NF, NB, EK>), dim3((p.co + 63) / 64, p.ho, p.batch), dim3(256), lds, s,
                       p.wp, p.x, p.bias, p.scale, p.co, p.ci, p.hi, p);
    return hipGetLastError();
}

template <int NF, int NB>
static hipError_t launch_pipe(const ConvParams& p, hipStream_t s)
{
    switch (conv_cheap_kind(p)) {
    case 0: return launch_pipe_form<NF, NB, 0>(p, s);
    case 4: return launch_pipe_form<NF, NB, 4>(p, s);
    default: return launch_pipe_form<NF, NB, -1>(p, s);
    }
}

template <int NF>
static hipError_t launch_pipe_nb(const ConvParams& p, hipStream_t s)
{
    switch (cv::ci32(p.ci) / 32) {
    case 1: return launch_pipe<NF, 1>(p, s);
    case 2: return launch_pipe<NF, 2>(p, s);
    case 3: return launch_pipe<NF, 3>(p, s);
    default: return launch_pipe<NF, 4>(p, s);
    }
}

// ---- pointwise (1x1, stride 1) form, fp16 input with C <= 256 ----
// A 1x1 convolution is a plain GEMM over the image's H W positions taken as
// one flat row, so a workgroup (4 waves, 64 output channels) takes 16
// consecutive positions: the C32 channels x 16 positions of input (32 bytes
// per channel, one 1 KB copy per 32-channel block) reach LDS by
// buffer_load ... lds, the transposed read makes the B fragments as in the
// 3x3 kernels, and each wave runs one 16x16x32 MFMA per block for its 16
// output channels and stores its 16 x 16 outputs from the accumulators.
// Everything a workgroup reads is issued at entry and waited for once: the
// work per workgroup is a few MFMAs, so the time is the load latency. YOLOX's
// CSP pointwise conv ([1,256,40,40] -> 128, 200 workgroups): 3.15-3.26 us
// against 4.46 with the general kernel; 32 positions per workgroup 4.43, 32
// output channels per workgroup 3.33-3.34, 16 channels 3.71. With the cheap
// epilogue (no residual, none / SiLU) 2.45 us: one 16-byte store per lane
// and no branch instead of four 4-byte stores behind per-channel checks.
template <int EPI, bool O16>
__device__ __forceinline__ void conv1_store(const ConvParams& p, const float4v& acc, uint32_t co_lane, uint32_t pos,
                                            uint32_t b)
{
    const size_t HW = (size_t)p.ho * p.wo;
    if (pos >= HW) return;
    const bool scaled = p.scale != nullptr, res = p.residual != nullptr, before = p.residual_order == 1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t co = co_lane + r;
        if (co >= p.co) break;
        const size_t o = ((size_t)b * p.co + co) * HW + pos;
        const float bias = p.bias ? (float)((const half_t*)p.bias)[co] : 0.f;
        float x = scaled ? fmaf(acc[r], (float)((const half_t*)p.scale)[co], bias) : acc[r] + bias;
        const float rr = !res ? 0.f
                              : p.residual_dtype == DT_F16 ? (float)((const half_t*)p.residual)[o]
                                                           : ((const float*)p.residual)[o];
        x += before ? rr : 0.f;
        x = cv_act<EPI>(x);
        x += before ? 0.f : rr;
        if constexpr (O16) ((half_t*)p.out)[o] = (half_t)x;
        else ((float*)p.out)[o] = x;
    }
}

// EK >= 0: the cheap epilogue with activation EK (see Conv3CheapOut). The
// MFMA then takes the input as A and the weight as B, so that a lane holds
// one output channel at four consecutive positions: one 16-byte store.
template <int NB, int EK>
__global__ __launch_bounds__(256) void conv1_pipe_kernel(const half_t* wp, const void* x, const void* bias_p,
                                                         const void* scale_p, uint32_t co_n, uint32_t ci_n,
                                                         uint32_t hw_n, ConvParams pk)
{
    // what the entry's loads need, as leading scalar arguments (preloaded
    // into SGPRs at launch); the rest of the parameters from the struct
    ConvParams p = pk;
    p.wp = wp; p.x = x; p.bias = bias_p; p.scale = scale_p; p.co = co_n; p.ci = ci_n;
    extern __shared__ half8 smem[];
    __attribute__((address_space(3))) char* xs = (__attribute__((address_space(3))) char*)(
        __attribute__((address_space(3))) void*)smem;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t p0 = blockIdx.x * 16, co0 = blockIdx.y * 64, b = blockIdx.z;
    const uint32_t HW = hw_n;
    const int fr = lane & 15, fg = lane >> 4;
    const uint32_t CO16 = (p.co + 15) / 16, oblk = min(blockIdx.y * 4 + wave, CO16 - 1);   // past Co: discarded

    // the wave's weight fragments, then its share of the input copies (block
    // j by wave j % 4): lane l copies channel 32 j + l / 2, positions p0 +
    // 8 (l % 2) .. +7; channels past C and positions past H W read as zero
    half8 wa[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) wa[j] = *(const half8*)(p.wp + (((size_t)oblk * NB + j) * 64 + lane) * 8);
    // the cheap epilogue's bias and scale of the lane's channel, loaded with
    // the rest (a missing one reads the packed weight and is ignored)
    float bias = 0.f, sc = 1.f;
    if constexpr (EK >= 0) {
        const uint32_t cc = min(co0 + wave * 16 + fr, p.co - 1);
        const float bv = (float)(p.bias ? (const half_t*)p.bias : p.wp)[cc];
        const float sv = (float)(p.scale ? (const half_t*)p.scale : p.wp)[cc];
        bias = p.bias ? bv : 0.f;
        sc = p.scale ? sv : 1.f;
    }
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)uniform_ptr((const half_t*)p.x + (size_t)b * p.ci * HW), (short)0, (int)(p.ci * HW * 2), 0x00020000);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if ((j & 3) != wave) continue;
        const uint32_t c = j * 32 + lane / 2, q = p0 + 8 * (lane & 1);
        const uint32_t off = (c < p.ci && q < HW) ? (c * HW + q) * 2 : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(xs + j * 1024), 16,
                                                 (int)off, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));   // vmcnt(0): copies landed
    __syncthreads();

    // B source lane (k, q) = (fr / 4, fr % 4) of group fg: channel 8 fg + k of
    // the block, positions 4 q ..; the high half 4 channels on
    const __attribute__((address_space(3))) char* base = xs + (8 * fg + (fr >> 2)) * 32 + (fr & 3) * 8;
    float4v acc = (float4v)0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const half4 lo = cv_read_tr16(base + j * 1024);
        const half4 hi = cv_read_tr16(base + j * 1024 + 4 * 32);
        const half8 xv = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        if constexpr (EK >= 0) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wa[j], acc, 0, 0, 0);
        else acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[j], xv, acc, 0, 0, 0);
    }
    if constexpr (EK >= 0) {
        // D[pos][co]: lane (fr, fg) holds channel co0 + 16 wave + fr at
        // positions p0 + 4 fg .. +3 (H W % 8 == 0: all four or none inside)
        const uint32_t co = co0 + wave * 16 + fr, q = p0 + 4 * fg;
        const uint32_t bytes = p.batch * p.co * HW * 4;
        const bool o16 = p.o_dtype == DT_F16;
        const uint32_t e = co < p.co && q < HW ? (b * p.co + co) * HW + q : 0x10000000u;
        float4v v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = cv_act<(EK >= 0 ? EK : 0)>(fmaf(acc[r], sc, bias));
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(cv_u32x4, v),
            __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, o16 ? 0 : (int)bytes, 0x00020000), (int)(e * 4), 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(
            __builtin_bit_cast(cv_u32x2, __builtin_convertvector(v, half4)),
            __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, o16 ? (int)(bytes / 2) : 0, 0x00020000), (int)(e * 2), 0,
            0);
        return;
    }
    // D[i][j] of the 16x16 fragment: lane j + 16 (i / 4), register i % 4
    const uint32_t co_lane = co0 + wave * 16 + fg * 4, pos = p0 + fr;
    const bool o16 = p.o_dtype == DT_F16;
    switch (p.epilogue) {
    case 1: o16 ? conv1_store<1, true>(p, acc, co_lane, pos, b) : conv1_store<1, false>(p, acc, co_lane, pos, b); break;
    case 2: o16 ? conv1_store<2, true>(p, acc, co_lane, pos, b) : conv1_store<2, false>(p, acc, co_lane, pos, b); break;
    case 3: o16 ? conv1_store<3, true>(p, acc, co_lane, pos, b) : conv1_store<3, false>(p, acc, co_lane, pos, b); break;
    case 4: o16 ? conv1_store<4, true>(p, acc, co_lane, pos, b) : conv1_store<4, false>(p, acc, co_lane, pos, b); break;
    case 5: o16 ? conv1_store<5, true>(p, acc, co_lane, pos, b) : conv1_store<5, false>(p, acc, co_lane, pos, b); break;
    default: o16 ? conv1_store<0, true>(p, acc, co_lane, pos, b) : conv1_store<0, false>(p, acc, co_lane, pos, b); break;
    }
}

// fp16 input, 1x1 stride 1, C <= 256, positions in whole 16-byte chunks
// (H W % 8 == 0) from a 16-byte aligned image, under 2^31 bytes
static bool conv1_pipe_ok(const ConvParams& p, int x_dt)
{
    const size_t HW = (size_t)p.hi * p.wi;
    return p.ks == 1 && p.stride == 1 && x_dt == DT_F16 && p.ci <= 256 && HW % 8 == 0 && ((uintptr_t)p.x % 16) == 0 &&
           (size_t)p.ci * HW * 2 < (1ull << 31);
}

template <int NB, int EK>
static hipError_t launch_conv1_form(const ConvParams& p, hipStream_t s)
{
    const uint32_t HW = p.ho * p.wo;
    hipLaunchKernelGGL((conv1_pipe_kernel<NB, EK>), dim3((HW + 15) / 16, (p.co + 63) / 64, p.batch), dim3(256),
                       NB * 1024, s, p.wp, p.x, p.bias, p.scale, p.co, p.ci, HW, p);
    return hipGetLastError();
}

template <int NB>
static hipError_t launch_conv1(const ConvParams& p, hipStream_t s)
{
    switch (conv_cheap_kind(p)) {
    case 0: return launch_conv1_form<NB, 0>(p, s);
    case 4: return launch_conv1_form<NB, 4>(p, s);
    default: return launch_conv1_form<NB, -1>(p, s);
    }
}

static hipError_t launch_conv1_nb(const ConvParams& p, hipStream_t s)
{
    switch (cv::ci32(p.ci) / 32) {
    case 1: return launch_conv1<1>(p, s);
    case 2: return launch_conv1<2>(p, s);
    case 3: return launch_conv1<3>(p, s);
    case 4: return launch_conv1<4>(p, s);
    case 5: return launch_conv1<5>(p, s);
    case 6: return launch_conv1<6>(p, s);
    case 7: return launch_conv1<7>(p, s);
    default: return launch_conv1<8>(p, s);
    }
}

// Whether the 3x3 LDS-transpose plan applies: fp16 NCHW rows of 16 NF
// columns (NF <= 8), stride 1, aligned buffers, and the stage fits LDS.
bool conv3_tr_ok(const ConvParams& p, int x_dt)
{
    const uint32_t nf = p.wi / 16;
    return p.ks == 3 && p.stride == 1 && x_dt == DT_F16 && p.wi % 16 == 0 && nf >= 1 && nf <= 8 && p.wo == p.wi &&
           p.ho == p.hi && ((uintptr_t)p.x % 16) == 0 && ((uintptr_t)p.out % 32) == 0 &&
           ((uintptr_t)p.residual % 32) == 0 && (size_t)cv::ci32(p.ci) * p.hi * p.wi * 2 < (1ull << 31) &&
           conv3_lds_bytes<64>(cv::ci32(p.ci), nf) <= 160u * 1024u;
}

template <int NF, int CT>
static hipError_t launch_tr_ct(const ConvParams& p, hipStream_t s)
{
    static PerDevice lds_once;
    hipError_t e = set_max_lds(lds_once, (const void*)conv3_tr_kernel<NF, CT>, 160 * 1024);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((conv3_tr_kernel<NF, CT>), dim3((p.co + CT - 1) / CT, p.ho, p.batch), dim3(CT * 16),
                       conv3_lds_bytes<CT>(cv::ci32(p.ci), NF), s, p);
    return hipGetLastError();
}

// 64 output channels per workgroup (16 waves) once 32-channel workgroups
// would need more than one per CU: each input band is then staged once per
// 64 channels, and no CU runs two workgroups back to back (config 5: 320
// workgroups of 32 channels on 256 CUs, 8.1 us; 160 of 64, 7.3 us).
template <int NF>
static hipError_t launch_tr(const ConvParams& p, hipStream_t s)
{
    int cus = 0;
    hipError_t e = device_cus(&cus);
    if (e != hipSuccess) return e;
    const uint64_t units32 = (uint64_t)((p.co + 31) / 32) * p.ho * p.batch;
    return p.co > 32 && units32 > (uint64_t)cus ? launch_tr_ct<NF, 64>(p, s) : launch_tr_ct<NF, 32>(p, s);
}

size_t conv_lds_bytes(uint32_t ci, uint32_t wi, uint32_t ks)
{
    return conv_main_lds_bytes(ci, wi, ks) + 2 * cv::CO_TILE * sizeof(float);
}

bool conv_nhwc_ok(uint32_t ci, uint32_t wi, uint32_t wo, uint32_t ks)
{
    return (ks == 1 || ks == 3) && wo <= 16u * cv::MAX_WO_FRAGS &&
           conv_lds_bytes(ci, wi, ks) <= 160u * 1024u && (size_t)ci * ks * ks * 2 <= 64u * 1024u;
}

size_t conv_packed_weight_bytes(uint32_t ci, uint32_t co, uint32_t ks)
{
    return (size_t)ks * ks * ((co + 15) / 16 * 16) * cv::ci32(ci) * 2;
}

hipError_t conv_pack_weight(half_t* dst, const half_t* w, uint32_t ci, uint32_t co, uint32_t ks, hipStream_t s)
{
    hipLaunchKernelGGL(pack_weight_kernel, dim3((co + 15) / 16 * 16), dim3(256), (size_t)ci * ks * ks * 2, s, dst, w, co, ci,
                       cv::ci32(ci), ks * ks);
    return hipGetLastError();
}

// fp16 input takes 64 output channels per workgroup (16 waves) once 32-channel
// workgroups would outnumber the CUs and the 64-channel sums fit LDS: no CU
// then runs two workgroups back to back, and each input band is staged once
// per 64 channels (as the 3x3 stride-1 kernel below does).
template <int KS, int NF>
static hipError_t launch_nf(const ConvParams& p, int x_dt, size_t lds, hipStream_t s)
{
    int cus = 0;
    hipError_t e = device_cus(&cus);
    if (e != hipSuccess) return e;
    const uint64_t units32 = (uint64_t)((p.co + 31) / 32) * p.ho * p.batch;
    const size_t lds64 = conv_main_lds_bytes(p.ci, p.wi, KS, 64, NF) + 2 * 64 * sizeof(float);
    if (x_dt == DT_F16 && p.co > 32 && units32 > (uint64_t)cus && lds64 <= 160u * 1024u) {
        static PerDevice lds_once64;
        if ((e = set_max_lds(lds_once64, (const void*)conv_kernel<KS, NF, half_t, 64>, 160 * 1024)) != hipSuccess)
            return e;
        hipLaunchKernelGGL((conv_kernel<KS, NF, half_t, 64>), dim3((p.co + 63) / 64, p.ho, p.batch), dim3(1024), lds64,
                           s, p);
        return hipGetLastError();
    }
    auto kern = x_dt == DT_F16 ? conv_kernel<KS, NF, half_t, 32> : conv_kernel<KS, NF, float, 32>;
    static PerDevice lds_once[2];
    if ((e = set_max_lds(lds_once[x_dt == DT_F16], (const void*)kern, 160 * 1024)) != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((p.co + cv::CO_TILE - 1) / cv::CO_TILE, p.ho, p.batch), dim3(512), lds, s, p);
    return hipGetLastError();
}

template <int KS>
static hipError_t launch_ks(const ConvParams& p, int x_dt, size_t lds, hipStream_t s)
{
    switch ((p.wo + 15) / 16) {
    case 1: return launch_nf<KS, 1>(p, x_dt, lds, s);
    case 2: return launch_nf<KS, 2>(p, x_dt, lds, s);
    case 3: return launch_nf<KS, 3>(p, x_dt, lds, s);
    case 4: return launch_nf<KS, 4>(p, x_dt, lds, s);
    case 5: return launch_nf<KS, 5>(p, x_dt, lds, s);
    case 6: return launch_nf<KS, 6>(p, x_dt, lds, s);
    case 7: return launch_nf<KS, 7>(p, x_dt, lds, s);
    default: return launch_nf<KS, 8>(p, x_dt, lds, s);
    }
}

hipError_t conv_launch(const ConvParams& p, int x_dt, hipStream_t s)
{
    if (conv1_pipe_ok(p, x_dt)) return launch_conv1_nb(p, s);
    if (conv3_tr_ok(p, x_dt) && cv::ci32(p.ci) <= 128) {
        switch (p.wi / 16) {
        case 1: return launch_pipe_nb<1>(p, s);
        case 2: return launch_pipe_nb<2>(p, s);
        case 3: return launch_pipe_nb<3>(p, s);
        case 4: return launch_pipe_nb<4>(p, s);
        case 5: return launch_pipe_nb<5>(p, s);
        case 6: return launch_pipe_nb<6>(p, s);
        case 7: return launch_pipe_nb<7>(p, s);
        default: return launch_pipe_nb<8>(p, s);
        }
    }
    if (conv3_tr_ok(p, x_dt)) {
        switch (p.wi / 16) {
        case 1: return launch_tr<1>(p, s);
        case 2: return launch_tr<2>(p, s);
        case 3: return launch_tr<3>(p, s);
        case 4: return launch_tr<4>(p, s);
        case 5: return launch_tr<5>(p, s);
        case 6: return launch_tr<6>(p, s);
        case 7: return launch_tr<7>(p, s);
        default: return launch_tr<8>(p, s);
        }
    }
    const size_t lds = conv_lds_bytes(p.ci, p.wi, p.ks);
    return p.ks == 1 ? launch_ks<1>(p, x_dt, lds, s) : launch_ks<3>(p, x_dt, lds, s);
}

}   // namespace vai_dev
