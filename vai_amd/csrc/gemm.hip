// gemm.hip -- MFMA-tiled GEMM C[M,N] = A[M,K] . B[N,K]^T for gfx950, with the
// fused epilogues of vAi's matmul hot path.
//
// One kernel template covers four callers that differ only in how the B side
// is read and what happens to the accumulators:
//   Linear tile path  A = I [M,K],  B = W [N,K]              (linear-tile.comp)
//   gated MLP         B = column pairs (j, H+j) of W [2H,K]  (linear + gated-mul)
//   attention scores  A = Q[h] [Tq,D], B = K[h/g] [Tkv,D]    (attention.comp qk)
//   implicit conv     A = W [Co, Ci*k*k], B = im2col(X)      (conv-*-implicit-gemm)
//
// Numerics follow the reference's tile contract (linear-tile.comp:63-69): both
// operands are staged as fp16 into LDS unless both are fp32, then fp32; the
// products accumulate in fp32 (v_mfma_f32_32x32x16_f16 / v_mfma_f32_32x32x2f32).
//
// Schedule: 256 threads = 4 waves in a 2x2 grid, each wave owning a
// (BM/2)x(BN/2) block of 32x32 MFMA fragments. K advances in BK steps through
// two LDS buffers: the global loads of step t+1 are in registers while step t
// runs on the matrix cores, so one barrier per step suffices.
#include "device_common.h"
#include "kernels.h"

namespace vai_dev {

template <bool F32> struct Stage;
template <> struct Stage<false> { typedef half_t T; static constexpr int BK = 32, VW = 8, PAD = 8; };
template <> struct Stage<true>  { typedef float T;  static constexpr int BK = 16, VW = 4, PAD = 4; };

template <typename S, typename T> __device__ __forceinline__ S cvt(T v) { return (S)v; }

// Loads VW consecutive elements of a row-major matrix into staging type,
// zero past `lim` (the valid element count of this row from `p`).
template <typename ST, typename T, int VW>
__device__ __forceinline__ void load_row_vec(ST* dst, const T* p, int lim, bool vec)
{
    if (vec && lim >= VW) {
        if constexpr (sizeof(T) * VW == 16) {
            typedef T vt __attribute__((ext_vector_type(VW)));
            vt v = *(const vt*)p;
#pragma unroll
            for (int e = 0; e < VW; ++e) dst[e] = cvt<ST>(v[e]);
        } else if constexpr (sizeof(T) * VW == 32) {
            typedef T vt __attribute__((ext_vector_type(VW / 2)));
            vt v0 = *(const vt*)p, v1 = *(const vt*)(p + VW / 2);
#pragma unroll
            for (int e = 0; e < VW / 2; ++e) { dst[e] = cvt<ST>(v0[e]); dst[e + VW / 2] = cvt<ST>(v1[e]); }
        } else {
            typedef T vt __attribute__((ext_vector_type(VW)));
            vt v = *(const vt*)p;
#pragma unroll
            for (int e = 0; e < VW; ++e) dst[e] = cvt<ST>(v[e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < VW; ++e) dst[e] = e < lim ? cvt<ST>(p[e]) : (ST)0;
    }
}

template <int BM, int BN, bool F32, typename TA, typename TB, BKind BKD, EpiKind EK>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p)
{
    typedef typename Stage<F32>::T ST;
    constexpr int BK = Stage<F32>::BK, VW = Stage<F32>::VW, PAD = Stage<F32>::PAD;
    constexpr int LDK = BK + PAD;
    constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 32, FN = WTN / 32;
    constexpr int NA = BM * BK / (256 * VW), NB = BN * BK / (256 * VW);
    static_assert(NA >= 1 && NB >= 1, "tile too small for 256 threads");
    static_assert(EK != EpiKind::Gated || FN % 2 == 0, "gated tiles pair fragments");
    __shared__ ST As[2][BM * LDK];
    __shared__ ST Bs[2][BN * LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t split = blockIdx.z % p.splits, bz = blockIdx.z / p.splits;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t M = p.M, N = p.N, K = p.K;

    // ---- scores: tiles the mask hides entirely are -inf without any MFMA ----
    if constexpr (EK == EpiKind::Scores) {
        // the tile's rows read at most keys [key_start(first row), key_end(last row))
        const uint32_t last = (m0 + BM < M ? m0 + BM : M) - 1;
        const bool hidden = (int64_t)n0 >= p.mask.key_end(last) || (int64_t)n0 + BN <= p.mask.key_start(m0);
        if (hidden) {
            float* C = (float*)p.C + bz * p.c_batch_stride;
            for (int i = tid; i < BM * BN; i += 256) {
                const uint32_t r = m0 + i / BN, c = n0 + i % BN;
                if (r < M && c < N) C[(size_t)r * N + c] = -__builtin_inff();
            }
            return;
        }
    }

    const TA* __restrict__ A = (const TA*)p.A + bz * p.a_batch_stride;
    const TB* __restrict__ B = (const TB*)p.B + (bz / p.b_group) * p.b_batch_stride;
    const uint32_t kbeg = split * p.split_size;
    const uint32_t kend = min(K, kbeg + p.split_size);
    const int ktiles = (int)((kend - kbeg + BK - 1) / BK);
    const bool vec_a = (K % VW == 0) && (kbeg % VW == 0) && ((uintptr_t)A % 16 == 0);
    const bool vec_b = (K % VW == 0) && (kbeg % VW == 0) && ((uintptr_t)B % 16 == 0);

    // Per-thread staging registers for one k-tile.
    ST ra[NA][VW], rb[NB][VW];

    auto load_a = [&](int kt) {
        const uint32_t k0 = kbeg + kt * BK;
#pragma unroll
        for (int v = 0; v < NA; ++v) {
            const int L = v * 256 + tid, row = L / (BK / VW), kk = (L % (BK / VW)) * VW;
            const uint32_t gr = m0 + row, gk = k0 + kk;
            const int lim = (gr < M) ? (int)min((int64_t)VW, (int64_t)kend - gk) : 0;
            if (lim <= 0) {
#pragma unroll
                for (int e = 0; e < VW; ++e) ra[v][e] = (ST)0;
            } else {
                load_row_vec<ST, TA, VW>(ra[v], A + (size_t)gr * K + gk, lim, vec_a);
            }
        }
    };
    auto load_b = [&](int kt) {
        const uint32_t k0 = kbeg + kt * BK;
        if constexpr (BKD == BKind::Im2col) {
            // Adjacent threads take adjacent output positions: coalesced along wo.
            const uint32_t kk2 = p.ks * p.ks;
#pragma unroll
            for (int v = 0; v < NB; ++v) {
                const int L = v * 256 + tid, row = L % BN, kq = (L / BN) * VW;
                const uint32_t pp = n0 + row;
                const int ho = (int)(pp / p.wo), wo = (int)(pp % p.wo);
#pragma unroll
                for (int e = 0; e < VW; ++e) {
                    const uint32_t k = k0 + kq + e;
                    ST val = (ST)0;
                    if (pp < N && k < kend) {
                        const uint32_t c = k / kk2, tap = k - c * kk2;
                        const uint32_t kh = tap / p.ks, kw = tap - kh * p.ks;
                        const int hi = ho * (int)p.stride + (int)kh - (int)(p.ks / 2);
                        const int wi = wo * (int)p.stride + (int)kw - (int)(p.ks / 2);
                        if (hi >= 0 && wi >= 0 && hi < (int)p.hi && wi < (int)p.wi)
                            val = cvt<ST>(B[((size_t)c * p.hi + hi) * p.wi + wi]);
                    }
                    rb[v][e] = val;
                }
            }
        } else {
#pragma unroll
            for (int v = 0; v < NB; ++v) {
                const int L = v * 256 + tid, row = L / (BK / VW), kk = (L % (BK / VW)) * VW;
                uint32_t grow = n0 + row;
                bool ok = grow < N;
                if constexpr (BKD == BKind::Gated) {
                    // logical column -> (output column jo, gate or up row)
                    const int w_n = row / WTN, within = row % WTN, fn = within / 32, j = within % 32;
                    const uint32_t jo = blockIdx.x * (BN / 2) + w_n * (WTN / 2) + (fn % (FN / 2)) * 32 + j;
                    ok = jo < p.H;
                    grow = jo + ((fn >= FN / 2) ? p.H : 0u);
                }
                const uint32_t gk = k0 + kk;
                const int lim = ok ? (int)min((int64_t)VW, (int64_t)kend - gk) : 0;
                if (lim <= 0) {
#pragma unroll
                    for (int e = 0; e < VW; ++e) rb[v][e] = (ST)0;
                } else {
                    load_row_vec<ST, TB, VW>(rb[v], B + (size_t)grow * K + gk, lim, vec_b);
                }
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int v = 0; v < NA; ++v) {
            const int L = v * 256 + tid, row = L / (BK / VW), kk = (L % (BK / VW)) * VW;
#pragma unroll
            for (int e = 0; e < VW; ++e) As[buf][row * LDK + kk + e] = ra[v][e];
        }
#pragma unroll
        for (int v = 0; v < NB; ++v) {
            int row, kk;
            if constexpr (BKD == BKind::Im2col) { const int L = v * 256 + tid; row = L % BN; kk = (L / BN) * VW; }
            else { const int L = v * 256 + tid; row = L / (BK / VW); kk = (L % (BK / VW)) * VW; }
#pragma unroll
            for (int e = 0; e < VW; ++e) Bs[buf][row * LDK + kk + e] = rb[v][e];
        }
    };

    float16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (float16v)0.f;

    if (ktiles > 0) {
        load_a(0);
        load_b(0);
        store_tiles(0);
        __syncthreads();
    }
    const int fr = lane & 31, fk = lane >> 5;   // fragment row / k-half of this lane
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) { load_a(kt + 1); load_b(kt + 1); }
        const ST* as = As[buf] + (wm * WTM + fr) * LDK;
        const ST* bs = Bs[buf] + (wn * WTN + fr) * LDK;
        if constexpr (!F32) {
#pragma unroll
            for (int ks = 0; ks < BK / 16; ++ks) {
                half8 af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = *(const half8*)(as + i * 32 * LDK + ks * 16 + fk * 8);
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = *(const half8*)(bs + j * 32 * LDK + ks * 16 + fk * 8);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < BK / 2; ++ks) {
                float af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = as[i * 32 * LDK + ks * 2 + fk];
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = bs[j * 32 * LDK + ks * 2 + fk];
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < ktiles) store_tiles(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: D[i][j] of a 32x32 fragment sits in lane j + 32*((i/4)%2),
    //      register (i%4) + 4*(i/8) ----
    const uint32_t rbase = m0 + wm * WTM, cbase = n0 + wn * WTN;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = rbase + i * 32 + 8 * (r / 4) + 4 * fk + (r % 4);
            if (row >= M) continue;
            if constexpr (EK == EpiKind::Gated) {
#pragma unroll
                for (int j = 0; j < FN / 2; ++j) {
                    const uint32_t jo = blockIdx.x * (BN / 2) + wn * (WTN / 2) + j * 32 + fr;
                    if (jo >= p.H) continue;
                    float g = acc[i][j][r], u = acc[i][j + FN / 2][r];
                    if (p.splits > 1) {
                        float* P = (float*)p.C + (size_t)split * M * (2 * p.H);
                        P[(size_t)row * 2 * p.H + jo] = g;
                        P[(size_t)row * 2 * p.H + p.H + jo] = u;
                    } else {
                        if (p.bias) {
                            g += ld(p.bias, p.bias_dtype, jo);
                            u += ld(p.bias, p.bias_dtype, p.H + jo);
                        }
                        st(p.C, p.c_dtype, (size_t)row * p.H + jo, epilogue(g, p.epilogue) * u);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const uint32_t col = cbase + j * 32 + fr;
                    if (col >= N) continue;
                    const float v = acc[i][j][r];
                    if constexpr (EK == EpiKind::Linear) {
                        const size_t o = (size_t)row * N + col;
                        if (p.splits > 1) {
                            ((float*)p.C)[(size_t)split * M * N + o] = v;
                        } else {
                            const float b = p.bias ? ld(p.bias, p.bias_dtype, p.bias_repeat ? o % p.bias_repeat : o) : 0.f;
                            const float rr = p.residual ? ld(p.residual, p.residual_dtype,
                                                             p.residual_repeat ? o % p.residual_repeat : o) : 0.f;
                            st(p.C, p.c_dtype, o, finish(v + b, rr, p.epilogue, p.residual_order, p.scalar_scale));
                        }
                    } else if constexpr (EK == EpiKind::Scores) {
                        const bool hide = (int64_t)col >= p.mask.key_end(row) || (int64_t)col < p.mask.key_start(row);
                        ((float*)p.C)[bz * p.c_batch_stride + (size_t)row * N + col] =
                            hide ? -__builtin_inff() : v * p.scalar_scale;
                    } else {   // Conv: row = output channel, col = output position
                        const float b = p.bias ? ld(p.bias, p.bias_dtype, row) : 0.f;
                        float x = p.conv_scale ? fmaf(v, ld(p.conv_scale, p.bias_dtype, row), b) : v + b;
                        const size_t o = bz * p.c_batch_stride + (size_t)row * N + col;
                        const float rr = p.residual ? ld(p.residual, p.residual_dtype, o) : 0.f;
                        if (p.residual && p.residual_order == 1) x += rr;
                        x = epilogue(x, p.epilogue);
                        if (p.residual && p.residual_order == 0) x += rr;
                        st(p.C, p.c_dtype, o, x);
                    }
                }
            }
        }
    }
}

template <int BM, int BN, bool F32, typename TA, typename TB, BKind BKD, EpiKind EK>
static hipError_t launch_tile(const GemmParams& p, hipStream_t s)
{
    const uint32_t ncols = (EK == EpiKind::Gated) ? 2 * p.H : p.N;
    dim3 grid((ncols + BN - 1) / BN, (p.M + BM - 1) / BM, p.batch * p.splits);
    if (EK == EpiKind::Gated) grid.x = (p.H + BN / 2 - 1) / (BN / 2);
    hipLaunchKernelGGL((gemm_kernel<BM, BN, F32, TA, TB, BKD, EK>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <bool F32, typename TA, typename TB, BKind BKD, EpiKind EK>
static hipError_t launch_tiles(const GemmParams& p, GemmTile t, hipStream_t s)
{
    switch (t) {
    case GemmTile::T64x64:
        if constexpr (EK != EpiKind::Gated) return launch_tile<64, 64, F32, TA, TB, BKD, EK>(p, s);
        else return launch_tile<64, 128, F32, TA, TB, BKD, EK>(p, s);
    case GemmTile::T128x64:
        if constexpr (EK != EpiKind::Gated) return launch_tile<128, 64, F32, TA, TB, BKD, EK>(p, s);
        else return launch_tile<128, 128, F32, TA, TB, BKD, EK>(p, s);
    case GemmTile::T128x128: return launch_tile<128, 128, F32, TA, TB, BKD, EK>(p, s);
    default: return launch_tile<256, 128, F32, TA, TB, BKD, EK>(p, s);
    }
}

template <BKind BKD, EpiKind EK>
static hipError_t launch_types(const GemmParams& p, GemmTile t, hipStream_t s)
{
    const bool a16 = p.a_dtype == DT_F16, b16 = p.b_dtype == DT_F16;
    if (a16 && b16) return launch_tiles<false, half_t, half_t, BKD, EK>(p, t, s);
    if (!a16 && b16) return launch_tiles<false, float, half_t, BKD, EK>(p, t, s);
    if (a16 && !b16) return launch_tiles<false, half_t, float, BKD, EK>(p, t, s);
    return launch_tiles<true, float, float, BKD, EK>(p, t, s);
}

hipError_t gemm_launch(const GemmParams& p, BKind bk, EpiKind ek, GemmTile tile, hipStream_t s)
{
    if (bk == BKind::Dense && ek == EpiKind::Linear) return launch_types<BKind::Dense, EpiKind::Linear>(p, tile, s);
    if (bk == BKind::Gated && ek == EpiKind::Gated) return launch_types<BKind::Gated, EpiKind::Gated>(p, tile, s);
    if (bk == BKind::Dense && ek == EpiKind::Scores) return launch_types<BKind::Dense, EpiKind::Scores>(p, tile, s);
    if (bk == BKind::Im2col && ek == EpiKind::Conv) return launch_types<BKind::Im2col, EpiKind::Conv>(p, tile, s);
    return hipErrorInvalidValue;
}

}   // namespace vai_dev
