/*
 * vai_oracle.c -- CPU restatement of the arithmetic of vAi's matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU kernels are
 * compared with; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product (libvai_amd.so) never links it.
 *
 * Each function restates one reference kernel's numeric contract (which
 * operands are rounded to fp16, that accumulation is fp32, where bias,
 * epilogue, residual and scale apply), not its GPU schedule. Accumulation
 * order is plain k order, so results agree with the reference to within
 * fp32 reassociation, which the tolerance tiers of the tests absorb.
 *
 * Pins (tests/test_oracle.py):
 *   - fp16 conversion: every one of the 65536 fp16 codes round-trips; normal
 *     fp32 values convert as numpy's float16 does; subnormal results flush to
 *     zero as /root/reference/vai/engine/tensor.cpp:42-90 does.
 *   - epilogues: closed forms (torch-free numpy erf/tanh), special points.
 *   - linear / reduce / gated-mul / conv / scores: float64 closed forms from
 *     numpy, brute force on tiny shapes, golden fixtures in tests/golden/.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 0, DT_F16 = 1, DT_NONE = 2 };
enum { EPI_NONE, EPI_RELU, EPI_GELU, EPI_GELU_TANH, EPI_SILU, EPI_SIGMOID };

/* ---- fp16 <-> fp32, /root/reference/vai/engine/tensor.cpp:42-90 ---------- */

/* f16 -> f32: exact, subnormal halves included (tensor.cpp:42-58). */
float orc_h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float v;
    if (e == 0)       v = ldexpf((float)m, -24);
    else if (e == 31) { uint32_t b = 0x7F800000u | (m << 13); memcpy(&v, &b, 4); }
    else              v = ldexpf((float)(m | 0x400), (int)e - 25);
    uint32_t b; memcpy(&b, &v, 4); b |= sign; memcpy(&v, &b, 4);
    return v;
}

/* f32 -> f16 round-to-nearest-even; overflow -> inf, results below the
 * smallest normal half flush to signed zero, NaN stays NaN (tensor.cpp:61-90). */
uint16_t orc_f2h(float f)
{
    uint32_t b; memcpy(&b, &f, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t expRaw = (b >> 23) & 0xFF, mant = b & 0x7FFFFF;
    if (expRaw == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int32_t e = (int32_t)expRaw - 112;
    if (e <= 0) return (uint16_t)sign;
    uint32_t m10 = mant >> 13, rest = mant & 0x1FFF;
    if (rest > 0x1000 || (rest == 0x1000 && (m10 & 1))) m10++;
    uint32_t v = (uint32_t)e * 0x400u + m10;
    if (v >= 0x7C00u) v = 0x7C00u;
    return (uint16_t)(sign | v);
}

void orc_f32_to_f16(const float* src, uint16_t* dst, size_t n)
{ for (size_t i = 0; i < n; ++i) dst[i] = orc_f2h(src[i]); }
void orc_f16_to_f32(const uint16_t* src, float* dst, size_t n)
{ for (size_t i = 0; i < n; ++i) dst[i] = orc_h2f(src[i]); }

static float rd(const void* p, int dt, size_t i)
{ return dt == DT_F16 ? orc_h2f(((const uint16_t*)p)[i]) : ((const float*)p)[i]; }
static void wr(void* p, int dt, size_t i, float v)
{ if (dt == DT_F16) ((uint16_t*)p)[i] = orc_f2h(v); else ((float*)p)[i] = v; }
/* f32 -> f16 as a shader's float16_t(v) conversion does it on the device:
 * IEEE round-to-nearest-even with subnormal halves kept (the host conversion
 * above flushes them; a GPU conversion does not). */
uint16_t orc_f2h_ieee(float f)
{
    uint32_t b; memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t expRaw = (b >> 23) & 0xFF, mant = b & 0x7FFFFF;
    if (expRaw == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int32_t e = (int32_t)expRaw - 112;
    if (e > 0) return orc_f2h(f);
    /* subnormal half: value = m * 2^-24, m = round(|f| * 2^24) (RNE) */
    const float a = fabsf(f) * 16777216.0f;   /* exact: scaling by a power of two */
    float r = nearbyintf(a);                  /* default rounding mode: to nearest even */
    return (uint16_t)(sign | (uint32_t)r);    /* r == 1024 gives the smallest normal */
}

/* What fp16 staging does to an operand element (linear-tile.comp:87-91). */
static float stage16(float v) { return orc_h2f(orc_f2h_ieee(v)); }

/* ---- epilogues, /root/reference/vai/shaders/common/activation.h:19-58 ----- */

static float erf_as(float x)   /* Abramowitz-Stegun 7.1.26 (activation.h:19-24) */
{
    const float t = 1.0f / (1.0f + 0.3275911f * fabsf(x));
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t
                     + 0.254829592f) * t;
    const float s = (x > 0.f) ? 1.f : (x < 0.f ? -1.f : 0.f);
    return s * (1.0f - p * expf(-x * x));
}

float orc_epilogue(float x, int epi)
{
    switch (epi) {
    case EPI_RELU:      return x > 0.f ? x : 0.f;
    case EPI_GELU:      return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
    case EPI_GELU_TANH: return 0.5f * x * (1.0f + tanhf(0.79788456080286535f * (x + 0.044715f * x * x * x)));
    case EPI_SILU:      return x / (1.0f + expf(-x));
    case EPI_SIGMOID:   return 1.0f / (1.0f + expf(-x));
    default:            return x;
    }
}

void orc_epilogue_vec(const float* x, float* y, size_t n, int epi)
{ for (size_t i = 0; i < n; ++i) y[i] = orc_epilogue(x[i], epi); }

/* s * epi(acc + b) + r, or s * epi(acc + b + r): linear-slab.comp:236-242,
 * linear-reduce.comp:95-98. */
static float finish(float acc, float r, int epi, int order, float s)
{ return order == 1 ? s * orc_epilogue(acc + r, epi) : s * orc_epilogue(acc, epi) + r; }

/* ---- Linear --------------------------------------------------------------
 * O[m,n] = s * epi(sum_k I[m,k] W[n,k] + B) (+R)
 *   stage: 0 = slab contract (linear-slab.comp: operands read at their own
 *   dtype, fp32 math); 1 = tile contract (linear-tile.comp:63-69,87-91: fp16
 *   staging of both operands unless both are fp32).
 *   biasRepeat / residualRepeat: 0 = [M,N], else the block length that
 *   repeats (linear.h:2333-2338); bias may be NULL (hasBias false).
 *   splitSize > 0 (tile only): partial sums per K span are folded in span
 *   order, as linear-reduce.comp:84-89 does. */
void orc_linear(void* O, int oDt, const void* I, int iDt, const void* W, int wDt,
                const void* B, int bDt, uint32_t biasRepeat,
                const void* R, uint32_t residualRepeat,
                uint32_t M, uint32_t N, uint32_t K,
                int epi, int order, float s, int stage, uint32_t splitSize)
{
    const int f16stage = stage == 1 && !(iDt == DT_F32 && wDt == DT_F32);
    if (splitSize == 0 || splitSize > K) splitSize = K;
    #pragma omp parallel
    {
        float* irow = (float*)malloc(sizeof(float) * K);
        float* wrow = (float*)malloc(sizeof(float) * K);
        #pragma omp for schedule(static)
        for (long long mm = 0; mm < (long long)M; ++mm) {
            const uint32_t m = (uint32_t)mm;
            for (uint32_t k = 0; k < K; ++k) {
                float v = rd(I, iDt, (size_t)m * K + k);
                irow[k] = f16stage ? stage16(v) : v;
            }
            for (uint32_t n = 0; n < N; ++n) {
                for (uint32_t k = 0; k < K; ++k) {
                    float v = rd(W, wDt, (size_t)n * K + k);
                    wrow[k] = f16stage ? stage16(v) : v;
                }
                const size_t idx = (size_t)m * N + n;
                float acc = B ? rd(B, bDt, biasRepeat ? idx % biasRepeat : idx) : 0.f;
                for (uint32_t k0 = 0; k0 < K; k0 += splitSize) {
                    const uint32_t k1 = (k0 + splitSize < K) ? k0 + splitSize : K;
                    float part = 0.f;
                    for (uint32_t k = k0; k < k1; ++k) part += irow[k] * wrow[k];
                    acc += part;
                }
                const float r = R ? rd(R, oDt, residualRepeat ? idx % residualRepeat : idx) : 0.f;
                wr(O, oDt, idx, finish(acc, r, epi, order, s));
            }
        }
        free(irow); free(wrow);
    }
}

/* Fast fp32-accumulating GEMM over fp32 rows, O[m,n] = sum_k A[m,k] B[n,k],
 * used for the CPU baseline timing (same contract as orc_linear's plain
 * output; the simd reduction splits each dot into vector-lane partials). */
void orc_gemm_f32(float* O, const float* A, const float* Bm, uint32_t M, uint32_t N, uint32_t K)
{
    #pragma omp parallel for schedule(static) collapse(2)
    for (long long m = 0; m < (long long)M; ++m)
        for (long long n = 0; n < (long long)N; ++n) {
            const float* a = A + (size_t)m * K;
            const float* b = Bm + (size_t)n * K;
            float acc = 0.f;
            #pragma omp simd reduction(+:acc)
            for (uint32_t k = 0; k < K; ++k) acc += a[k] * b[k];
            O[(size_t)m * N + n] = acc;
        }
}

/* ---- fp16 accumulation, Linear::setAccDtype(Fp16) -------------------------
 * linear-tile.comp:55,71,292-320: the sums are float16; each split walks its
 * K span in 4-wide steps from the span's start, one step being
 *   sum = fma(a[k],b[k], fma(a[k+1],b[k+1], fma(a[k+2],b[k+2], fma(a[k+3],b[k+3], sum))))
 * (k+3 first, each fma rounded once to fp16; elements past the span are 0),
 * then the sums are clamped to +-65504 (linear-tile.comp:317-321) and folded
 * in fp32 like any partial (linear-reduce.comp:84-98). Operands are staged
 * as fp16 (the tile contract: at least one of them is fp16 here). */

/* double -> fp16 bits, IEEE round-to-nearest-even with subnormals kept and
 * overflow to inf. The fma's exact product a*b (22 significant bits) plus the
 * fp16 sum is exact in double whenever their exponents lie within 42 of each
 * other, which holds for all but sums with vanishing terms. */
uint16_t orc_d2h(double x)
{
    const uint16_t sign = signbit(x) ? 0x8000u : 0u;
    const double a = fabs(x);
    if (isnan(x)) return 0x7E00u;
    if (a >= 65520.0) return sign | 0x7C00u;          /* past 65504 + half an ulp (a tie rounds to even: up) */
    if (a < 6.103515625e-05) {                        /* below 2^-14: subnormal, m * 2^-24 */
        const double m = nearbyint(a * 16777216.0);
        return (uint16_t)(sign | (uint16_t)m);        /* m == 1024 is the smallest normal's encoding */
    }
    int e;
    const double f = frexp(a, &e);                    /* a = f 2^e, f in [0.5, 1) */
    double m = nearbyint(ldexp(f, 11));               /* 11 significant bits */
    if (m == 2048.0) { m = 1024.0; ++e; }
    const int E = e + 14;                             /* a = (m/1024) 2^(E-15) */
    if (E >= 31) return sign | 0x7C00u;
    return (uint16_t)(sign | (uint16_t)(E << 10) | (uint16_t)((uint32_t)m - 1024u));
}

/* fp16 fused multiply-add: a*b + c rounded once to fp16 (operands fp16 bits). */
uint16_t orc_fma16(uint16_t a, uint16_t b, uint16_t c)
{
    return orc_d2h((double)orc_h2f(a) * (double)orc_h2f(b) + (double)orc_h2f(c));
}

/* One split's fp16 sum of a . b over [k0, k1), clamped, as a float. */
static float acc16_span(const uint16_t* a, const uint16_t* b, uint32_t k0, uint32_t k1)
{
    uint16_t sum = 0;
    for (uint32_t k = k0; k < k1; k += 4)
        for (int q = 3; q >= 0; --q) {
            const uint32_t kk = k + (uint32_t)q;
            sum = orc_fma16(kk < k1 ? a[kk] : 0, kk < k1 ? b[kk] : 0, sum);
        }
    const float v = orc_h2f(sum);
    return v != v ? v : fminf(fmaxf(v, -65504.f), 65504.f);   /* a NaN chain stays NaN */
}

/* O = s*epi(sum_z P_z + B) (+R), P_z the fp16-accumulated split sums; gated:
 * O[m,j] = gate_epi(g + B[j]) * (u + B[H+j]) over W = [gate rows; up rows]. */
void orc_linear_acc16(void* O, int oDt, const void* I, int iDt, const void* W, int wDt,
                      const void* B, int bDt, uint32_t biasRepeat, const void* R, uint32_t residualRepeat,
                      uint32_t M, uint32_t N, uint32_t K, int epi, int order, float s, uint32_t splitSize,
                      int gated, int gateEpi)
{
    if (splitSize == 0 || splitSize > K) splitSize = K;
    const uint32_t H = gated ? N / 2 : 0, cols = gated ? H : N;
    #pragma omp parallel
    {
        uint16_t* irow = (uint16_t*)malloc(2 * (size_t)K);
        uint16_t* w0 = (uint16_t*)malloc(2 * (size_t)K);
        uint16_t* w1 = (uint16_t*)malloc(2 * (size_t)K);
        #pragma omp for schedule(static)
        for (long long mm = 0; mm < (long long)M; ++mm) {
            const uint32_t m = (uint32_t)mm;
            for (uint32_t k = 0; k < K; ++k) irow[k] = orc_f2h_ieee(rd(I, iDt, (size_t)m * K + k));
            for (uint32_t n = 0; n < cols; ++n) {
                for (uint32_t k = 0; k < K; ++k) {
                    w0[k] = orc_f2h_ieee(rd(W, wDt, (size_t)n * K + k));
                    if (gated) w1[k] = orc_f2h_ieee(rd(W, wDt, (size_t)(H + n) * K + k));
                }
                if (gated) {
                    float g = B ? rd(B, bDt, n) : 0.f, u = B ? rd(B, bDt, H + n) : 0.f;
                    for (uint32_t k0 = 0; k0 < K; k0 += splitSize) {
                        const uint32_t k1 = k0 + splitSize < K ? k0 + splitSize : K;
                        g += acc16_span(irow, w0, k0, k1);
                        u += acc16_span(irow, w1, k0, k1);
                    }
                    wr(O, oDt, (size_t)m * H + n, orc_epilogue(g, gateEpi) * u);
                } else {
                    const size_t idx = (size_t)m * N + n;
                    float acc = B ? rd(B, bDt, biasRepeat ? idx % biasRepeat : idx) : 0.f;
                    for (uint32_t k0 = 0; k0 < K; k0 += splitSize) {
                        const uint32_t k1 = k0 + splitSize < K ? k0 + splitSize : K;
                        acc += acc16_span(irow, w0, k0, k1);
                    }
                    const float r = R ? rd(R, oDt, residualRepeat ? idx % residualRepeat : idx) : 0.f;
                    wr(O, oDt, idx, finish(acc, r, epi, order, s));
                }
            }
        }
        free(irow); free(w0); free(w1);
    }
}

/* linear-reduce.comp:80-116: O = s*epi(sum_z P[z] + B) (+R), P and R in oDt. */
void orc_linear_reduce(void* O, const void* P, int oDt, uint32_t splitCount, uint32_t MN,
                       const void* B, int bDt, uint32_t biasRepeat,
                       const void* R, uint32_t residualRepeat, int epi, int order, float s)
{
    for (size_t i = 0; i < MN; ++i) {
        float acc = B ? rd(B, bDt, biasRepeat ? i % biasRepeat : i) : 0.f;
        for (uint32_t z = 0; z < splitCount; ++z) acc += rd(P, oDt, (size_t)z * MN + i);
        const float r = R ? rd(R, oDt, residualRepeat ? i % residualRepeat : i) : 0.f;
        wr(O, oDt, i, finish(acc, r, epi, order, s));
    }
}

/* gated-mul.comp:39-49: O[r,j] = epi(I[r,j]) * I[r,H+j]. */
void orc_gated_mul(void* O, int oDt, const void* I, int iDt, uint32_t rows, uint32_t H, int epi)
{
    for (size_t r = 0; r < rows; ++r)
        for (size_t j = 0; j < H; ++j) {
            const size_t src = r * 2 * H + j;
            wr(O, oDt, r * H + j, orc_epilogue(rd(I, iDt, src), epi) * rd(I, iDt, src + H));
        }
}

/* ---- Convolution: implicit GEMM, conv-k3s1-implicit-gemm.comp:127-152 and
 * conv-implicit-gemm.comp. Same padding pad = k/2, Ho = (Hi-1)/stride + 1
 * (convolution.h:4113-4117). K index = c*k*k + kh*k + kw. Operands staged as
 * fp16 when the weight is fp16, else fp32 (conv-k3s1-implicit-gemm.comp:
 * 78-81,107-117). Bias / scale carry the weight dtype, the residual the
 * input dtype (readResidual). out = epi(acc*scale + bias (+R)) (+R). */
void orc_conv2d(void* O, int oDt, const void* X, int iDt, const void* W, int wDt,
                const void* bias, const void* scale, const void* R,
                uint32_t batch, uint32_t Ci, uint32_t Hi, uint32_t Wi, uint32_t Co,
                uint32_t ks, uint32_t stride, int epi, int order)
{
    const uint32_t Ho = (Hi - 1) / stride + 1, Wo = (Wi - 1) / stride + 1;
    const int pad = (int)ks / 2;
    const size_t Kg = (size_t)Ci * ks * ks;
    const int f16 = wDt == DT_F16;
    #pragma omp parallel
    {
        float* col = (float*)malloc(sizeof(float) * Kg);
        float* wr_ = (float*)malloc(sizeof(float) * Kg);
        #pragma omp for schedule(static) collapse(2)
        for (long long b = 0; b < (long long)batch; ++b)
            for (long long p = 0; p < (long long)Ho * Wo; ++p) {
                const int ho = (int)(p / Wo), wo = (int)(p % Wo);
                for (size_t k = 0; k < Kg; ++k) {
                    const uint32_t c = (uint32_t)(k / (ks * ks)), tap = (uint32_t)(k % (ks * ks));
                    const int hi = ho * (int)stride + (int)(tap / ks) - pad;
                    const int wi = wo * (int)stride + (int)(tap % ks) - pad;
                    float v = 0.f;
                    if (hi >= 0 && wi >= 0 && hi < (int)Hi && wi < (int)Wi)
                        v = rd(X, iDt, (((size_t)b * Ci + c) * Hi + hi) * Wi + wi);
                    col[k] = f16 ? stage16(v) : v;
                }
                for (uint32_t co = 0; co < Co; ++co) {
                    float acc = 0.f;
                    for (size_t k = 0; k < Kg; ++k) {
                        float w = rd(W, wDt, co * Kg + k);
                        acc += (f16 ? stage16(w) : w) * col[k];
                    }
                    const float bv = bias ? rd(bias, wDt, co) : 0.f;
                    float v = scale ? fmaf(acc, rd(scale, wDt, co), bv) : acc + bv;
                    const size_t oi = (((size_t)b * Co + co) * Ho + ho) * Wo + wo;
                    const float r = R ? rd(R, iDt, oi) : 0.f;
                    if (R && order == 1) v += r;
                    v = orc_epilogue(v, epi);
                    if (R && order == 0) v += r;
                    wr(O, oDt, oi, v);
                }
            }
        free(col); free(wr_);
    }
}

/* ---- Attention scores: the Q.K^T stage of attention.comp:155-182 and
 * attention-fa.comp:581-591. S[h,i,j] = (sum_d Q[h,i,d] K[hk,j,d]) * scale,
 * fp32 accumulation; hk = h / (Hq/Hkv) (GQA). Mask (common/causal_mask.h:
 * 25-42, attention-fa.comp:135-146 without a KV cache): queries align with
 * the keys' end, query i at key position pos = i + Tkv - Tq. Its new-token end
 * comes from the block list -- nBlocks blocks, block k causal iff bit
 * (nBlocks-1-k) of bits, ends[k] the end row of block k < nBlocks-1 (the last
 * ends at Tq) -- as i+1 in a causal block and the block's end otherwise (no
 * blocks: Tq); key j is visible iff j < end + Tkv - Tq. nBlocks == 0 with
 * causal != 0 is one causal block. span > 0 also hides j < pos + 1 - span.
 * Hidden entries are -inf. */
static long long new_token_end(uint32_t t, uint32_t Tq, uint32_t nBlocks, uint32_t bits, const uint32_t* ends)
{
    if (nBlocks == 0) return Tq;
    uint32_t k = 0, e = Tq;
    while (k + 1 < nBlocks) {
        const uint32_t b = ends[k] < Tq ? ends[k] : Tq;
        if (t < b) { e = b; break; }
        ++k;
    }
    return ((bits >> (nBlocks - 1 - k)) & 1u) ? (long long)t + 1 : (long long)e;
}

void orc_attn_scores_blocks(float* S, const void* Q, const void* Kt, int dt,
                            uint32_t Hq, uint32_t Hkv, uint32_t Tq, uint32_t Tkv, uint32_t D,
                            float scale, int causal, uint32_t span, uint32_t nBlocks, uint32_t bits,
                            const uint32_t* ends)
{
    if (nBlocks == 0 && causal) { nBlocks = 1; bits = 1; }
    const uint32_t group = Hq / Hkv;
    #pragma omp parallel for schedule(static) collapse(2)
    for (long long h = 0; h < (long long)Hq; ++h)
        for (long long i = 0; i < (long long)Tq; ++i) {
            const uint32_t hk = (uint32_t)h / group;
            const long long pos = i + (long long)Tkv - (long long)Tq;
            const long long kend = new_token_end((uint32_t)i, Tq, nBlocks, bits, ends) + (long long)Tkv - (long long)Tq;
            for (uint32_t j = 0; j < Tkv; ++j) {
                int visible = (long long)j < kend;
                if (span && pos >= (long long)span && (long long)j < pos + 1 - (long long)span) visible = 0;
                float acc = 0.f;
                if (visible)
                    for (uint32_t d = 0; d < D; ++d)
                        acc += rd(Q, dt, ((size_t)h * Tq + i) * D + d) * rd(Kt, dt, ((size_t)hk * Tkv + j) * D + d);
                S[((size_t)h * Tq + i) * Tkv + j] = visible ? acc * scale : -INFINITY;
            }
        }
}

void orc_attn_scores(float* S, const void* Q, const void* Kt, int dt,
                     uint32_t Hq, uint32_t Hkv, uint32_t Tq, uint32_t Tkv, uint32_t D,
                     float scale, int causal, uint32_t span)
{
    orc_attn_scores_blocks(S, Q, Kt, dt, Hq, Hkv, Tq, Tkv, D, scale, causal, span, 0, 0, NULL);
}

int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
