/*
 * cpu_baseline.c -- the CPU baseline bench.py reports beside each GPU config:
 * an OpenMP, AVX2/FMA/F16C restatement of the same five computations.
 *
 * TEST INFRASTRUCTURE ONLY, like vai_oracle.c (it lives in the same library):
 * only tests/ and bench.py's cpu_baseline leg load it, and the product never
 * links it. It stands in for the reference's lavapipe run (Vulkan on the host
 * CPU, /root/reference/.github/workflows/ci.yml:308-341), which needs a Vulkan
 * runtime this machine does not have.
 *
 * Same arithmetic contract as the GPU path: fp16 operands widened exactly to
 * fp32, fp32 accumulation, fp32 output; the schedule is a CPU one:
 *   - cpb_linear, M <= 8: the decode GEMV of linear-slab.comp:121-137 -- each
 *     thread streams its rows of W once, converting 8 halves per F16C
 *     instruction, against all M input rows held in fp32.
 *   - cpb_linear, M > 8 (configs 1 and 3): a cache-blocked A.B^T -- 64-row
 *     blocks of X against 48-row blocks of W, K in 512-wide chunks that fit
 *     L2, a 4x3 register micro-tile of 8-wide fp32 FMA accumulators.
 *   - cpb_conv2d (config 5): implicit GEMM, one output row per task. The row's
 *     im2col panel is built with the reference's K order k = c*k*k + kh*k + kw
 *     (conv-k3s1-implicit-gemm.comp:127-139), which is also the weight's own
 *     [Co][C][k][k] memory order, so the fp16 weight is read in place.
 *   - cpb_attn_scores (config 4): the blocked A.B^T per head over 64x64 tiles;
 *     tiles the causal mask hides entirely are written as -inf untouched.
 * Pins: tests/test_cpu_baseline.py (float64 closed forms with Higham bounds).
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 0, DT_F16 = 1 };
float orc_epilogue(float x, int epi);
float orc_h2f(uint16_t h);

#define KC 512   /* K chunk: a 64x512 fp32 X block + a 48x512 W block fit in L2 */
#define MB 64
#define NB 48

static inline float hsum8(__m256 v)
{
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

static inline __m256 load8(const void* p, int dt, size_t i)
{
    if (dt == DT_F16) return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)((const uint16_t*)p + i)));
    return _mm256_loadu_ps((const float*)p + i);
}

static inline float load1(const void* p, int dt, size_t i)
{
    return dt == DT_F16 ? _cvtsh_ss(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

/* C[i*ldc + j] += sum_{k<K} A[i*lda + k] * B[j*ldb + k] for an m x n block;
 * A fp32, B fp32 or fp16 bits. */
static void block_abt(float* C, size_t ldc, const float* A, size_t lda, const void* B, int bdt, size_t ldb,
                      int m, int n, int K)
{
    const int K8 = K & ~7;
    int i = 0;
    for (; i + 4 <= m; i += 4) {
        int j = 0;
        for (; j + 3 <= n; j += 3) {
            __m256 c00 = _mm256_setzero_ps(), c01 = c00, c02 = c00, c10 = c00, c11 = c00, c12 = c00;
            __m256 c20 = c00, c21 = c00, c22 = c00, c30 = c00, c31 = c00, c32 = c00;
            const float* a0 = A + (size_t)i * lda;
            for (int k = 0; k < K8; k += 8) {
                const __m256 b0 = load8(B, bdt, (size_t)j * ldb + k);
                const __m256 b1 = load8(B, bdt, (size_t)(j + 1) * ldb + k);
                const __m256 b2 = load8(B, bdt, (size_t)(j + 2) * ldb + k);
                __m256 a = _mm256_loadu_ps(a0 + k);
                c00 = _mm256_fmadd_ps(a, b0, c00); c01 = _mm256_fmadd_ps(a, b1, c01); c02 = _mm256_fmadd_ps(a, b2, c02);
                a = _mm256_loadu_ps(a0 + lda + k);
                c10 = _mm256_fmadd_ps(a, b0, c10); c11 = _mm256_fmadd_ps(a, b1, c11); c12 = _mm256_fmadd_ps(a, b2, c12);
                a = _mm256_loadu_ps(a0 + 2 * lda + k);
                c20 = _mm256_fmadd_ps(a, b0, c20); c21 = _mm256_fmadd_ps(a, b1, c21); c22 = _mm256_fmadd_ps(a, b2, c22);
                a = _mm256_loadu_ps(a0 + 3 * lda + k);
                c30 = _mm256_fmadd_ps(a, b0, c30); c31 = _mm256_fmadd_ps(a, b1, c31); c32 = _mm256_fmadd_ps(a, b2, c32);
            }
            float t[4][3] = {{hsum8(c00), hsum8(c01), hsum8(c02)}, {hsum8(c10), hsum8(c11), hsum8(c12)},
                             {hsum8(c20), hsum8(c21), hsum8(c22)}, {hsum8(c30), hsum8(c31), hsum8(c32)}};
            for (int k = K8; k < K; ++k)
                for (int r = 0; r < 4; ++r)
                    for (int s = 0; s < 3; ++s) t[r][s] += a0[r * lda + k] * load1(B, bdt, (size_t)(j + s) * ldb + k);
            for (int r = 0; r < 4; ++r)
                for (int s = 0; s < 3; ++s) C[(size_t)(i + r) * ldc + j + s] += t[r][s];
        }
        for (; j < n; ++j)
            for (int r = 0; r < 4; ++r) {
                const float* a = A + (size_t)(i + r) * lda;
                __m256 c = _mm256_setzero_ps();
                for (int k = 0; k < K8; k += 8) c = _mm256_fmadd_ps(_mm256_loadu_ps(a + k), load8(B, bdt, (size_t)j * ldb + k), c);
                float t = hsum8(c);
                for (int k = K8; k < K; ++k) t += a[k] * load1(B, bdt, (size_t)j * ldb + k);
                C[(size_t)(i + r) * ldc + j] += t;
            }
    }
    for (; i < m; ++i) {
        const float* a = A + (size_t)i * lda;
        for (int j = 0; j < n; ++j) {
            __m256 c = _mm256_setzero_ps();
            for (int k = 0; k < K8; k += 8) c = _mm256_fmadd_ps(_mm256_loadu_ps(a + k), load8(B, bdt, (size_t)j * ldb + k), c);
            float t = hsum8(c);
            for (int k = K8; k < K; ++k) t += a[k] * load1(B, bdt, (size_t)j * ldb + k);
            C[(size_t)i * ldc + j] += t;
        }
    }
}

/* C = A.B^T over a whole m x n block, K chunked. */
static void tile_abt(float* C, size_t ldc, const float* A, size_t lda, const void* B, int bdt, size_t ldb,
                     int m, int n, int K)
{
    for (int i = 0; i < m; ++i) memset(C + (size_t)i * ldc, 0, sizeof(float) * (size_t)n);
    for (int k0 = 0; k0 < K; k0 += KC) {
        const int kc = K - k0 < KC ? K - k0 : KC;
        const size_t boff = (size_t)k0 * (bdt == DT_F16 ? 2 : 4);
        block_abt(C, ldc, A + k0, lda, (const char*)B + boff, bdt, ldb, m, n, kc);
    }
}

static float* widen(const void* X, int dt, size_t n)
{
    float* f = (float*)aligned_alloc(64, (n * sizeof(float) + 63) & ~(size_t)63);
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) f[i] = load1(X, dt, (size_t)i);
    return f;
}

/* Y[r,n] = sum_k X[r,k] W[n,k] for R (compile-time) rows of X; U independent
 * accumulator chains per row so that one row's FMA latency does not bound it. */
static inline __attribute__((always_inline)) void gemv_rows(float* Y, const float* Xf, const void* W, int wdt,
                                                            uint32_t N, uint32_t K, const int R, const int U)
{
    #pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; ++n) {
        __m256 acc[8][4];
        for (int r = 0; r < R; ++r)
            for (int u = 0; u < U; ++u) acc[r][u] = _mm256_setzero_ps();
        const uint32_t step = 8u * (uint32_t)U, Ks = K / step * step;
        for (uint32_t k = 0; k < Ks; k += step)
            for (int u = 0; u < U; ++u) {
                const __m256 w = load8(W, wdt, (size_t)n * K + k + 8 * u);
                for (int r = 0; r < R; ++r)
                    acc[r][u] = _mm256_fmadd_ps(_mm256_loadu_ps(Xf + (size_t)r * K + k + 8 * u), w, acc[r][u]);
            }
        for (int r = 0; r < R; ++r) {
            __m256 a = acc[r][0];
            for (int u = 1; u < U; ++u) a = _mm256_add_ps(a, acc[r][u]);
            float t = hsum8(a);
            for (uint32_t k = Ks; k < K; ++k) t += Xf[(size_t)r * K + k] * load1(W, wdt, (size_t)n * K + k);
            Y[(size_t)r * N + n] = t;
        }
    }
}

/* Linear, fp32 output: O = epi(X W^T + b); gated: O[m,j] = gate_epi(Y[m,j]) Y[m,H+j]
 * with Y = X W^T + b, W [2H,K]. bias fp32 [N] or NULL. */
void cpb_linear(float* O, const void* X, int xdt, const void* W, int wdt, const float* bias,
                uint32_t M, uint32_t N, uint32_t K, int epi, int gated, int gate_epi)
{
    float* Xf = widen(X, xdt, (size_t)M * K);
    const uint32_t H = gated ? N / 2 : 0;
    if (M <= 8) {
        /* decode GEMV: W streamed once; every row of W against all M inputs */
        float* Y = gated ? (float*)malloc(sizeof(float) * M * N) : O;
        switch (M) {
        case 1: gemv_rows(Y, Xf, W, wdt, N, K, 1, 4); break;
        case 2: gemv_rows(Y, Xf, W, wdt, N, K, 2, 2); break;
        case 3: gemv_rows(Y, Xf, W, wdt, N, K, 3, 1); break;
        case 4: gemv_rows(Y, Xf, W, wdt, N, K, 4, 1); break;
        case 5: gemv_rows(Y, Xf, W, wdt, N, K, 5, 1); break;
        case 6: gemv_rows(Y, Xf, W, wdt, N, K, 6, 1); break;
        case 7: gemv_rows(Y, Xf, W, wdt, N, K, 7, 1); break;
        default: gemv_rows(Y, Xf, W, wdt, N, K, 8, 1); break;
        }
        for (uint32_t r = 0; r < M; ++r)
            for (uint32_t n = 0; n < N; ++n) {
                const float t = Y[(size_t)r * N + n] + (bias ? bias[n] : 0.f);
                if (gated) Y[(size_t)r * N + n] = t;
                else O[(size_t)r * N + n] = orc_epilogue(t, epi);
            }
        if (gated) {
            for (uint32_t r = 0; r < M; ++r)
                for (uint32_t j = 0; j < H; ++j)
                    O[(size_t)r * H + j] = orc_epilogue(Y[(size_t)r * N + j], gate_epi) * Y[(size_t)r * N + H + j];
            free(Y);
        }
        free(Xf);
        return;
    }
    /* GEMM: a task is MB rows of X x NB output columns (gated: NB/2 gate
     * columns and their NB/2 up columns, so the product finishes in the task) */
    const uint32_t cols = gated ? H : N, cb = gated ? NB / 2 : NB;
    const uint32_t tm = (M + MB - 1) / MB, tn = (cols + cb - 1) / cb;
    const size_t wb = wdt == DT_F16 ? 2 : 4;
    #pragma omp parallel
    {
        float* C = (float*)malloc(sizeof(float) * MB * NB);
        #pragma omp for schedule(dynamic, 1)
        for (long long t = 0; t < (long long)tm * tn; ++t) {
            const uint32_t i0 = (uint32_t)(t / tn) * MB, j0 = (uint32_t)(t % tn) * cb;
            const int m = (int)(M - i0 < MB ? M - i0 : MB), n = (int)(cols - j0 < cb ? cols - j0 : cb);
            if (!gated) {
                tile_abt(C, NB, Xf + (size_t)i0 * K, K, (const char*)W + (size_t)j0 * K * wb, wdt, K, m, n, (int)K);
                for (int i = 0; i < m; ++i)
                    for (int j = 0; j < n; ++j)
                        O[(size_t)(i0 + i) * N + j0 + j] = orc_epilogue(C[i * NB + j] + (bias ? bias[j0 + j] : 0.f), epi);
            } else {
                tile_abt(C, NB, Xf + (size_t)i0 * K, K, (const char*)W + (size_t)j0 * K * wb, wdt, K, m, n, (int)K);
                tile_abt(C + cb, NB, Xf + (size_t)i0 * K, K, (const char*)W + (size_t)(H + j0) * K * wb, wdt, K, m, n,
                         (int)K);
                for (int i = 0; i < m; ++i)
                    for (int j = 0; j < n; ++j) {
                        const float g = C[i * NB + j] + (bias ? bias[j0 + j] : 0.f);
                        const float u = C[i * NB + cb + j] + (bias ? bias[H + j0 + j] : 0.f);
                        O[(size_t)(i0 + i) * H + j0 + j] = orc_epilogue(g, gate_epi) * u;
                    }
            }
        }
        free(C);
    }
    free(Xf);
}

/* Same-padded conv, one image: O[co,ho,wo] = epi(sum W[co,c,kh,kw] X[c,ho*s+kh-p,wo*s+kw-p] + b[co]),
 * X [Ci,Hi,Wi], W [Co,Ci,ks,ks] (dtypes xdt, wdt), bias fp32 [Co] or NULL. */
void cpb_conv2d(float* O, const void* X, int xdt, const void* W, int wdt, const float* bias,
                uint32_t Ci, uint32_t Hi, uint32_t Wi, uint32_t Co, uint32_t ks, uint32_t stride, int epi)
{
    const uint32_t Ho = (Hi - 1) / stride + 1, Wo = (Wi - 1) / stride + 1;
    const int pad = (int)ks / 2;
    const uint32_t Kg = Ci * ks * ks;
    #pragma omp parallel
    {
        float* P = (float*)aligned_alloc(64, (sizeof(float) * (size_t)Wo * Kg + 63) & ~(size_t)63);
        float* C = (float*)malloc(sizeof(float) * (size_t)Wo * Co);
        #pragma omp for schedule(dynamic, 1)
        for (long long ho = 0; ho < (long long)Ho; ++ho) {
            /* im2col panel of this output row: P[wo][c*ks*ks + kh*ks + kw] */
            for (uint32_t wo = 0; wo < Wo; ++wo)
                for (uint32_t c = 0; c < Ci; ++c)
                    for (uint32_t kh = 0; kh < ks; ++kh) {
                        const int hi = (int)ho * (int)stride + (int)kh - pad;
                        for (uint32_t kw = 0; kw < ks; ++kw) {
                            const int wi = (int)(wo * stride + kw) - pad;
                            float v = 0.f;
                            if (hi >= 0 && hi < (int)Hi && wi >= 0 && wi < (int)Wi)
                                v = load1(X, xdt, ((size_t)c * Hi + hi) * Wi + wi);
                            P[(size_t)wo * Kg + (c * ks + kh) * ks + kw] = v;
                        }
                    }
            tile_abt(C, Co, P, Kg, W, wdt, Kg, (int)Wo, (int)Co, (int)Kg);
            for (uint32_t co = 0; co < Co; ++co)
                for (uint32_t wo = 0; wo < Wo; ++wo)
                    O[((size_t)co * Ho + ho) * Wo + wo] = orc_epilogue(C[(size_t)wo * Co + co] + (bias ? bias[co] : 0.f), epi);
        }
        free(P); free(C);
    }
}

/* Attention scores, fp16 Q [H,Tq,D] and K [H,Tkv,D]: S = scale Q K^T, key j
 * hidden from query i when causal and j > i + Tkv - Tq (-inf). */
void cpb_attn_scores(float* S, const uint16_t* Q, const uint16_t* Kt, uint32_t H, uint32_t Tq, uint32_t Tkv,
                     uint32_t D, float scale, int causal)
{
    float* Qf = widen(Q, DT_F16, (size_t)H * Tq * D);
    const uint32_t T = 64, ti = (Tq + T - 1) / T, tj = (Tkv + T - 1) / T;
    const long long off = (long long)Tkv - (long long)Tq;
    #pragma omp parallel
    {
        float* C = (float*)malloc(sizeof(float) * T * T);
        #pragma omp for schedule(dynamic, 1)
        for (long long t = 0; t < (long long)H * ti * tj; ++t) {
            const uint32_t h = (uint32_t)(t / ((long long)ti * tj)), r = (uint32_t)(t % ((long long)ti * tj));
            const uint32_t i0 = (r / tj) * T, j0 = (r % tj) * T;
            const int m = (int)(Tq - i0 < T ? Tq - i0 : T), n = (int)(Tkv - j0 < T ? Tkv - j0 : T);
            float* Sh = S + (size_t)h * Tq * Tkv;
            if (causal && (long long)j0 > (long long)(i0 + m - 1) + off) {
                for (int i = 0; i < m; ++i)
                    for (int j = 0; j < n; ++j) Sh[(size_t)(i0 + i) * Tkv + j0 + j] = -INFINITY;
                continue;
            }
            tile_abt(C, T, Qf + ((size_t)h * Tq + i0) * D, D, Kt + ((size_t)h * Tkv + j0) * D, DT_F16, D, m, n, (int)D);
            for (int i = 0; i < m; ++i)
                for (int j = 0; j < n; ++j) {
                    const int hidden = causal && (long long)(j0 + j) > (long long)(i0 + i) + off;
                    Sh[(size_t)(i0 + i) * Tkv + j0 + j] = hidden ? -INFINITY : C[i * T + j] * scale;
                }
        }
        free(C);
    }
    free(Qf);
}

/* Attention, fp16 Q [H,Tq,D], K and V [H,Tkv,D] (one KV head per query head):
 * O = softmax(scale Q K^T + causal mask) V in fp32, rows with no visible key
 * give 0. Per 64-query block: scores over the visible keys (blocked A.B^T),
 * an fp32 softmax per row, then P.V as a blocked A.B^T against V^T. */
void cpb_attention(float* O, const uint16_t* Q, const uint16_t* Kt, const uint16_t* V, uint32_t H, uint32_t Tq,
                   uint32_t Tkv, uint32_t D, float scale, int causal)
{
    float* Qf = widen(Q, DT_F16, (size_t)H * Tq * D);
    float* Vt = (float*)aligned_alloc(64, (sizeof(float) * (size_t)H * D * Tkv + 63) & ~(size_t)63);
    #pragma omp parallel for schedule(static)
    for (long long hd = 0; hd < (long long)H * D; ++hd) {
        const size_t h = (size_t)hd / D, d = (size_t)hd % D;
        for (uint32_t j = 0; j < Tkv; ++j) Vt[hd * (size_t)Tkv + j] = _cvtsh_ss(V[(h * Tkv + j) * D + d]);
    }
    const uint32_t T = 64, ti = (Tq + T - 1) / T;
    const long long off = (long long)Tkv - (long long)Tq;
    #pragma omp parallel
    {
        float* S = (float*)malloc(sizeof(float) * T * Tkv);
        float* Ob = (float*)malloc(sizeof(float) * T * D);
        #pragma omp for schedule(dynamic, 1)
        for (long long t = 0; t < (long long)H * ti; ++t) {
            const uint32_t h = (uint32_t)(t / ti), i0 = (uint32_t)(t % ti) * T;
            const int m = (int)(Tq - i0 < T ? Tq - i0 : T);
            long long last = causal ? (long long)(i0 + m - 1) + off + 1 : (long long)Tkv;   /* keys [0, last) */
            if (last > (long long)Tkv) last = Tkv;
            const int nvis = last > 0 ? (int)last : 0;
            float* Oh = O + ((size_t)h * Tq + i0) * D;
            if (nvis == 0) { memset(Oh, 0, sizeof(float) * (size_t)m * D); continue; }
            tile_abt(S, Tkv, Qf + ((size_t)h * Tq + i0) * D, D, Kt + (size_t)h * Tkv * D, DT_F16, D, m, nvis, (int)D);
            float rsum[64];
            for (int i = 0; i < m; ++i) {
                float* s = S + (size_t)i * Tkv;
                const long long lim = causal ? (long long)(i0 + i) + off : (long long)Tkv - 1;   /* last visible key */
                float mx = -INFINITY;
                for (int j = 0; j < nvis; ++j) if (j <= lim && s[j] * scale > mx) mx = s[j] * scale;
                float sum = 0.f;
                for (int j = 0; j < nvis; ++j) {
                    const float p = (j <= lim) ? expf(s[j] * scale - mx) : 0.f;
                    s[j] = p;
                    sum += p;
                }
                rsum[i] = sum;
            }
            tile_abt(Ob, D, S, Tkv, Vt + (size_t)h * D * Tkv, DT_F32, Tkv, m, (int)D, nvis);
            for (int i = 0; i < m; ++i)
                for (uint32_t d = 0; d < D; ++d)
                    Oh[(size_t)i * D + d] = rsum[i] > 0.f ? Ob[(size_t)i * D + d] / rsum[i] : 0.f;
        }
        free(S); free(Ob);
    }
    free(Qf); free(Vt);
}
