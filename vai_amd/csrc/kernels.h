// kernels.h -- host-visible launch entry points of the gfx950 kernels (internal
// to libvai_amd; the public surface is include/vai_amd.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vai_dev {

typedef _Float16 half_t_storage;

struct SlabParams {
    void* out;
    const void* in;
    const void* weight;
    const void* bias;
    const void* residual;
    uint32_t M, N, K;
    int o_dtype, i_dtype, w_dtype, b_dtype;
    uint32_t epilogue, residual_order, bias_repeat, residual_repeat;
    float scalar_scale;
};
bool slab_vec_ok(const SlabParams& a);
bool gemv_mfma_ok(const SlabParams& a);
hipError_t slab_launch(const SlabParams& a, hipStream_t s);
// fp16 I and W, M <= 8, over the packed weight of gemm_pack_weight (same
// layout as the prefill path). Gated: writes the raw [M, 2H] Linear output to
// ygated in the original row order (the gating pass follows); otherwise O with
// the full epilogue.
hipError_t gemv_packed_launch(const SlabParams& a, const void* packed, bool gated, float* ygated, hipStream_t s);

// The operand a GEMM's "B" side reads: C[M,N] = A[M,K] . B[N,K]^T.
enum class BKind : int {
    Dense = 0,   // B rows are rows of a row-major [N, K] matrix
    Gated = 1,   // logical column pairs (j, H + j) of a [2H, K] matrix
    Im2col = 2,  // B[p, k] gathered from an NCHW image (implicit-GEMM conv)
};

// What the GEMM does with its accumulators.
enum class EpiKind : int {
    Linear = 0,    // bias / epilogue / residual / scale, or a split-K partial
    Gated = 1,     // gate_epi(g + bg) * (u + bu) into O[M, H]
    Scores = 2,    // scale, causal mask -> -inf, fp32 out
    Conv = 3,      // per-row (channel) scale / bias, epilogue, residual
};

// The attention mask of /root/reference/vai/shaders/common/causal_mask.h:25-42
// for the no-cache case: query t (0 <= t < tq) sits at key position
// t + tkv - tq and reads keys [key_start(t), key_end(t)). The token end comes
// from a list of blocks, each causal or not (the first block in the highest of
// `blocks` bits, ends end[0..blocks-2] in query rows, the last block ends at
// tq); 0 blocks is no mask. span > 0 keeps only the last span keys of each
// query (a sliding window). Both bounds are non-decreasing in t, so a range
// of rows [t0, t1) reads at most [key_start(t0), key_end(t1 - 1)).
struct MaskRule {
    uint32_t tq, tkv;
    uint32_t blocks, bits;
    uint32_t end[31];
    uint32_t span;

    __host__ __device__ uint32_t new_token_end(uint32_t t) const
    {
        if (blocks == 0) return tq;
        uint32_t k = 0, e = tq;
        for (; k + 1 < blocks; ++k) {
            const uint32_t b = end[k] < tq ? end[k] : tq;
            if (t < b) { e = b; break; }
        }
        return ((bits >> (blocks - 1 - k)) & 1u) ? t + 1 : e;
    }
    __host__ __device__ int64_t key_end(uint32_t t) const
    {
        const int64_t e = (int64_t)new_token_end(t) + tkv - tq;
        return e < 0 ? 0 : (e > (int64_t)tkv ? (int64_t)tkv : e);
    }
    __host__ __device__ int64_t key_start(uint32_t t) const { return key_start_cached(t, 0); }
    // With a KV cache holding `cached` positions ahead of the tkv new keys
    // (keys in global positions [0, cached + tkv)): the reference's
    // kvCacheCount + keyEnd(t) and keyStart(keyPos(t)), keyPos(t) = cached +
    // max(t + tkv - tq, 0) (/root/reference/vai/shaders/attention-fa.comp:
    // 137-146, 470-478). cached = 0 is the plain rule.
    __host__ __device__ int64_t key_end_cached(uint32_t t, uint32_t cached) const { return cached + key_end(t); }
    __host__ __device__ int64_t key_start_cached(uint32_t t, uint32_t cached) const
    {
        const int64_t pos = (int64_t)t + tkv - tq;
        const int64_t p = (int64_t)cached + (pos < 0 ? 0 : pos);
        return (span == 0 || p < (int64_t)span) ? 0 : p + 1 - span;
    }
};

struct GemmParams {
    // A [M, K] row-major (lda = K), B per BKind, C per EpiKind.
    const void* A;
    const void* B;
    void* C;
    int a_dtype, b_dtype, c_dtype;
    uint32_t M, N, K;
    // batching over blockIdx.z: element strides per batch entry
    uint32_t batch;
    size_t a_batch_stride, b_batch_stride, c_batch_stride;
    uint32_t b_group;             // B batch index = z / b_group (GQA)
    // split-K: span per split; splits > 1 writes fp32 partials to C + z*M*N
    uint32_t split_size, splits;
    // Linear / Gated epilogue
    const void* bias;
    int bias_dtype;
    uint32_t bias_repeat;
    const void* residual;
    int residual_dtype;
    uint32_t residual_repeat;
    uint32_t epilogue, residual_order;
    float scalar_scale;
    uint32_t H;                   // Gated: half width of W
    // Scores
    uint32_t causal, span;
    int32_t causal_offset;        // Tkv - Tq
    MaskRule mask;                // mask.blocks > 1: the block list rules (causal unused)
    // Conv: image geometry (B side is the gathered input)
    const void* conv_scale;
    uint32_t ci, hi, wi, wo, ks, stride;
};

// The tile shapes the launcher offers.
enum class GemmTile : int { T64x64 = 0, T128x64 = 1, T128x128 = 2, T256x128 = 3 };

hipError_t gemm_launch(const GemmParams& p, BKind bk, EpiKind ek, GemmTile tile, hipStream_t s);

// The 256x256x64 fp16 MFMA GEMM for large, K%64 == 0 shapes (Linear / gated).
bool gemm_big_ok(const GemmParams& p, bool gated);
hipError_t gemm_big_launch(const GemmParams& p, bool gated, hipStream_t s);

// The same shapes with a pre-packed fp16 weight (K % 128 == 0): the weight
// streams into VGPRs in fragment order and only A goes through LDS.
bool gemm_packed_ok(const GemmParams& p, bool gated);
size_t gemm_packed_weight_bytes(uint32_t N, uint32_t K, uint32_t H, bool gated);
hipError_t gemm_pack_weight(void* dst, const void* w, uint32_t N, uint32_t K, uint32_t H, bool gated, hipStream_t s);
hipError_t gemm_packed_launch(const GemmParams& p, const void* packed, bool gated, hipStream_t s);

// Linear with fp16 accumulation in the reference's exact fma order (any shape;
// vector ALU, not the matrix cores, which accumulate in fp32 only).
hipError_t gemm_acc16_launch(const GemmParams& p, bool gated, hipStream_t s);

// fp32 Linear for small problems: a 32 x 16*nf tile per workgroup over the
// full K (the waves split K and sum through LDS), no split-K workspace.
bool gemm_f32_ok(const GemmParams& p);
int gemm_f32_nf(uint32_t M, uint32_t N, uint32_t cus);
hipError_t gemm_f32_launch(const GemmParams& p, int nf, hipStream_t s);

// Attention scores for fp16 Q/K with head_dim % 64 == 0.
bool scores_fast_ok(const GemmParams& p);
hipError_t scores_launch(const GemmParams& p, hipStream_t s);

// Fused attention forward. Q [batch, hq, tq, head_dim] in q_dtype, K / V
// [batch, hkv, tkv, head_dim] in kv_dtype, O token-major [batch, tq, hq,
// head_dim] in o_dtype (the layout of /root/reference/vai/shaders/
// attention-fa.comp:8,96). Two paths: the MFMA flash kernel for head_dim % 8
// == 0, 16 <= head_dim <= 256 (padded to dp = 64, 128 or 256 inside the
// kernel; fp32 K / V are first rounded to fp16 copies in the workspace), and
// a plain fp32 kernel for every other head dim (the reference's naive path).
struct AttnParams {
    void* out;                    // [batch, tq, hq, head_dim], o_dtype
    const void* q;
    const void* k;
    const void* v;
    int o_dtype, q_dtype, kv_dtype;
    uint32_t batch, hq, hkv, tq, tkv, head_dim;
    uint32_t dp;                  // flash kernel's padded head dim; 0: the naive kernel
    // Key rows. Without a cache, k / v hold [batch, hkv, tkv, head_dim] and
    // kv_rows = tkv. With one (batch 1), k / v are the cache planes [hkv,
    // kv_rows, head_dim], keys sit in global positions [0, cached + tkv),
    // position j at row j (ring: j % kv_rows), and cached = *cache_count is
    // read by the kernels at run time (the reference's kvCacheCount uniform,
    // which the model rewrites before each forward).
    const uint32_t* cache_count;  // null: no cache, cached = 0
    uint32_t kv_rows;
    uint32_t ring;
    const void* k_new;            // with a cache: the tkv new rows [hkv, tkv, head_dim] in new_dtype,
    const void* v_new;            // appended to the cache before the attention reads it
    int new_dtype;
    float scale;
    uint32_t causal, span;
    MaskRule mask;                // the same rule; blocks > 1 takes the general per-row bounds
    // Key-range split (0 units: each workgroup walks all of its keys and
    // writes O). Otherwise each query tile's keys are cut into chunks of
    // chunk_tiles 64-key tiles, `units` work units per head; partial O and
    // (max, sum) go to ws_o / ws_ml and a merge pass combines them, finding
    // each query tile's first unit and chunk count in qt_tab.
    uint32_t units, chunk_tiles;
    float* ws_o;                  // [batch*hq*units][128][dp] (fp32, or fp16 O / l for fp16 output)
    float* ws_ml;                 // [batch*hq*units][128][2]
    void* ws_kv;                  // fp16 copies of fp32 K then V (flash path), else null
    // Split launches run a 1-D grid of units * hq * batch <= FA_WG_TAB
    // workgroups (one round on the GPU, a head's units on one XCD), and
    // attention_plan tabulates what each needs: workgroup w -> [2w] query
    // tile | key chunk << 16 | the tile's chunk count << 24, [2w + 1] unit |
    // head << 10 | batch << 20. One scalar load, issued with the kernel's
    // other argument loads, then no divisions.
    static constexpr uint32_t FA_WG_TAB = 256;
    uint32_t wg_tab[2 * FA_WG_TAB];
    // the merge pass's index, the same for every head: query tile qt's first
    // unit | its chunk count << 16 (a head has at most FA_WG_TAB units, so at
    // most that many query tiles)
    uint32_t qt_tab[FA_WG_TAB];
};
bool attention_ok(const AttnParams& p);
// Units per head for p's shape (0 when no query tile needs splitting), and
// the workspace the split needs.
uint32_t attention_units(const AttnParams& p, uint32_t chunk_tiles);
// Chooses the path (dp) and the key split (chunk_tiles, units) for a GPU of
// `cus` compute units.
void attention_plan(AttnParams& p, uint32_t cus);
size_t attention_workspace_bytes(const AttnParams& p);
void attention_set_workspace(AttnParams& p, void* ws);
hipError_t attention_launch(const AttnParams& p, hipStream_t s);

// Implicit-GEMM convolution, fp16 weights packed per tap in MFMA fragment order.
struct ConvParams {
    void* out;
    const void* x;                // input [B][Ci][Hi][Wi], fp16 or fp32
    const half_t_storage* wp;     // packed weight [k*k][Co/16][C32/32][64 lanes][8]
    const void* bias;             // fp16 [Co] or null
    const void* scale;            // fp16 [Co] or null
    const void* residual;         // [B][Co][Ho][Wo] (residual_dtype) or null
    int o_dtype, residual_dtype;
    uint32_t batch, ci, hi, wi, co, ho, wo, ks, stride;
    uint32_t epilogue, residual_order;
};
bool conv_nhwc_ok(uint32_t ci, uint32_t wi, uint32_t wo, uint32_t ks);
size_t conv_packed_weight_bytes(uint32_t ci, uint32_t co, uint32_t ks);
hipError_t conv_pack_weight(half_t_storage* dst, const half_t_storage* w, uint32_t ci, uint32_t co, uint32_t ks,
                            hipStream_t s);
hipError_t conv_launch(const ConvParams& p, int x_dt, hipStream_t s);

// Split-K fold for Linear: O = s*epi(sum_z P[z] + B) (+R).
hipError_t linear_reduce_launch(void* out, int o_dtype, const float* partials, uint32_t splits, size_t MN,
                                const void* bias, int b_dtype, uint32_t bias_repeat,
                                const void* residual, uint32_t residual_repeat,
                                uint32_t epi, uint32_t order, float s, uint32_t gated_H, uint32_t gate_epi,
                                uint32_t N, hipStream_t st);

hipError_t gated_mul_launch(void* out, int o_dtype, const void* in, int i_dtype, uint32_t rows, uint32_t H,
                            uint32_t epi, hipStream_t s);

}   // namespace vai_dev
