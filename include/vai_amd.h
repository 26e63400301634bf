/*
 * vai_amd.h -- C ABI of the MI355X (gfx950) kernels behind vAi's matmul hot path.
 *
 * Plain pointers and sizes only. Every buffer is device memory the caller owns
 * (hipMalloc'd, or any device-visible pointer); every launch is asynchronous on
 * the given stream and returns a vai_status (0 = success). Nothing throws
 * across this boundary. The library keeps no per-call state: besides its
 * kernels it holds only per-device launch settings made once (thread-safe),
 * and the scratch array of vai_linear_launch_noalloc.
 *
 * Callers: the C++ nodes in vai_amd/engine (Linear::run, Convolution::run,
 * AttentionScores::run, GatedMul::run), which replace the reference's
 * pipelinePool().request(...) + descriptor write + dispatch sequence.
 */
#ifndef VAI_AMD_H
#define VAI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vai_stream_t;   /* == hipStream_t */

/* Status codes. Values >= 1000 are the library's own argument checks; other
 * non-zero values are hipError_t codes passed through. */
typedef enum {
    VAI_OK = 0,
    VAI_ERR_INVALID_ARG = 1001,    /* null pointer, zero size, bad enum */
    VAI_ERR_SHAPE = 1002,          /* shapes that do not fit together */
    VAI_ERR_DTYPE = 1003,          /* a dtype combination the reference rejects */
    VAI_ERR_WORKSPACE = 1004,      /* workspace missing or too small */
    VAI_ERR_UNSUPPORTED = 1005,    /* valid, but not implemented here */
} vai_status;

/* Dtype codes: the reference's DTYPE_F32 / DTYPE_F16 / DTYPE_NONE
 * (/root/reference/vai/shaders/common/spec_constants.h:6-8). */
enum { VAI_DTYPE_F32 = 0, VAI_DTYPE_F16 = 1, VAI_DTYPE_NONE = 2 };

/* Epilogue codes in the order of vai::Epilogue
 * (/root/reference/vai/nodes/common.h:31-39). */
enum { VAI_EPI_NONE = 0, VAI_EPI_RELU, VAI_EPI_GELU, VAI_EPI_GELU_TANH, VAI_EPI_SILU, VAI_EPI_SIGMOID };

/* vai::ResidualOrder (/root/reference/vai/nodes/common.h:42-45). */
enum { VAI_RESIDUAL_AFTER_EPILOGUE = 0, VAI_RESIDUAL_BEFORE_EPILOGUE = 1 };

/* ---------------------------------------------------------------------------
 * Linear: O = s * epi(I . W^T + bias) + R        (residual_order AFTER)
 *         O = s * epi(I . W^T + bias + R)        (residual_order BEFORE)
 * I [M,K] (i_dtype), W [N,K] (w_dtype), O [M,N] (o_dtype), bias (b_dtype),
 * residual R (o_dtype). bias_repeat / residual_repeat: 0 when the operand
 * covers [M,N], else its element count, read modulo (a [N] row that repeats).
 * M <= 8 runs the HBM-streaming GEMV (fp32 math on the operands as stored,
 * the linear-slab contract); M > 8 runs the MFMA GEMM (fp16 staging unless I
 * and W are both fp32, then fp32 MFMA -- the linear-tile contract).
 * split_size > 0 forces split-K with K spans of that length (>= 32);
 * 0 lets the library choose. Split-K needs a workspace of
 * vai_linear_workspace_size() bytes.
 *
 * gated != 0 fuses the reference's GatedMul after this Linear
 * (/root/reference/vai/nodes/gated-mul.h:9-20): W holds [2H, K] rows (the
 * activated half first), O is [M, H] with
 *   O[m,j] = gate_epilogue(Y[m,j]) * Y[m,H+j],  Y = I . W^T + bias,
 * and epilogue must be NONE, scalar_scale 1, no residual.
 *
 * Replaces Linear::prepare/run's dispatches (/root/reference/vai/nodes/
 * linear.h:2291-2798): linear-slab, linear-tile / linear-cm, linear-reduce.
 * ------------------------------------------------------------------------- */
typedef struct {
    void* out;
    const void* in;
    const void* weight;
    const void* bias;        /* NULL: no bias (Linear::hasBias() false) */
    const void* residual;    /* NULL: no residual */
    void* workspace;         /* split-K partials; may be NULL when not needed */
    size_t workspace_bytes;
    uint32_t M, N, K;        /* N = outDim (= 2H when gated) */
    int32_t o_dtype, i_dtype, w_dtype, b_dtype;
    uint32_t epilogue;
    uint32_t residual_order;
    uint32_t bias_repeat;
    uint32_t residual_repeat;
    float scalar_scale;
    uint32_t split_size;
    uint32_t gated;
    uint32_t gate_epilogue;
    /* NULL, or vai_linear_pack_weight()'s output for this weight: prefill
     * shapes (M > 8, fp16 I and W) then stream W into the matrix cores from
     * that fragment-major copy instead of staging it through LDS. */
    const void* packed_weight;
    /* Accumulator dtype, Linear::setAccDtype (/root/reference/vai/nodes/
     * linear.h:289,2320): VAI_DTYPE_F32 (0, the default and the reference's
     * AMD default) or VAI_DTYPE_F16. F16 applies where the reference's tile
     * kernel honours it -- M > 8 with at least one fp16 operand -- and then
     * sums in fp16 in the order of linear-tile.comp:292-320 (4-wide k steps
     * from each split's start, k+3 first, every fma rounded to fp16), clamps
     * the sums to +-65504 and finishes in fp32. The GEMV (M <= 8) and fp32 x
     * fp32 products accumulate in fp32 whatever is asked, as the reference's
     * do. Split-K only when split_size asks for it. */
    int32_t acc_dtype;
} vai_linear_args;

vai_status vai_linear_launch(const vai_linear_args* args, vai_stream_t stream);
size_t vai_linear_workspace_size(const vai_linear_args* args);

/* vai_linear_launch for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. Same arguments, kernels and results as
 * vai_linear_launch, but args->workspace is ignored: the split-K partials and
 * the M <= 8 gated intermediate go to a device array inside the library
 * (VAI_NOALLOC_SCRATCH_BYTES = 64 MiB per GPU, held from the library's load until the
 * process ends). Returns VAI_ERR_WORKSPACE when the launch needs more than that
 * (vai_linear_workspace_size() tells in advance). Nothing is allocated. All
 * calls on one GPU share its array: calls that overlap in time on that GPU
 * (two streams, two threads) race on it and must be serialised by the caller. */
#define VAI_NOALLOC_SCRATCH_BYTES (64u << 20)
vai_status vai_linear_launch_noalloc(const vai_linear_args* args, vai_stream_t stream);

/* Size of, and the one-time fill of, the packed copy of args->weight that
 * packed_weight takes (0 / VAI_ERR_UNSUPPORTED when the shape or dtypes have
 * no packed path: fp16 I and W, K % 128 == 0, K >= 256). Depends on N, K,
 * the dtypes and `gated`, not on M. The weight-side counterpart of the
 * reference preparing a Linear's weights once at prepare time
 * (/root/reference/vai/nodes/linear.h:2291-2704). */
size_t vai_linear_packed_weight_size(const vai_linear_args* args);
vai_status vai_linear_pack_weight(const vai_linear_args* args, void* packed, size_t packed_bytes,
                                  vai_stream_t stream);

/* Which kernel vai_linear_launch picks for args (for tests and reports):
 * writes a short name ("slab", "slab_scalar", "tile_f16_128x128", ...). */
vai_status vai_linear_plan(const vai_linear_args* args, char* name, size_t name_len, uint32_t* split_count);

/* GatedMul alone: O[r,j] = epi(I[r,j]) * I[r,H+j], I [rows, 2H].
 * Replaces gated-mul.comp (/root/reference/vai/nodes/gated-mul.h:75-114). */
vai_status vai_gated_mul_launch(void* out, int32_t o_dtype, const void* in, int32_t i_dtype,
                                uint32_t rows, uint32_t H, uint32_t epilogue, vai_stream_t stream);

/* ---------------------------------------------------------------------------
 * Convolution (implicit GEMM): same-padded odd kernel, NCHW.
 *   out[b,co,ho,wo] = epi(scale[co] * sum_{c,kh,kw} W[co,c,kh,kw] X[b,c,ho*s+kh-p,wo*s+kw-p]
 *                         + bias[co] (+R)) (+R),   p = kernel/2, Ho = (Hi-1)/s+1.
 * bias / scale carry w_dtype and may be NULL; residual carries i_dtype.
 * fp16 weights stage both operands as fp16 (fp16 MFMA); fp32 weights stage
 * fp32 (fp32 MFMA). fp16 input needs fp16 weights; fp16 output needs fp16
 * weights (Convolution::validateInputs, /root/reference/vai/nodes/
 * convolution.h:4137-4160). Replaces runK3S1Implicit / the implicit-GEMM
 * plan (/root/reference/vai/nodes/convolution.h:6237-6283, 6616-6644).
 * With fp16 weights the kernel reads them packed per tap in MFMA fragment
 * order (output channels padded to a multiple of 16, input channels to a
 * multiple of 32): pass a buffer that vai_conv2d_pack_weight()
 * filled once as packed_weight (the reference transforms conv weights once,
 * /root/reference/vai/nodes/convolution.h:6224-6235), or leave it NULL and
 * pass a workspace of vai_conv2d_workspace_size() bytes in which every call
 * packs them first.
 * ------------------------------------------------------------------------- */
typedef struct {
    void* out;
    const void* in;
    const void* weight;
    const void* bias;
    const void* scale;
    const void* residual;
    uint32_t batch, ci, hi, wi, co, kernel, stride;
    int32_t o_dtype, i_dtype, w_dtype;
    uint32_t epilogue;
    uint32_t residual_order;
    void* workspace;
    size_t workspace_bytes;
    const void* packed_weight;   /* NULL, or vai_conv2d_pack_weight()'s output */
} vai_conv2d_args;

vai_status vai_conv2d_launch(const vai_conv2d_args* args, vai_stream_t stream);
size_t vai_conv2d_workspace_size(const vai_conv2d_args* args);
/* Size of, and the one-time fill of, the packed weight for args (0 / no-op
 * when args take the fp32 path, which reads the weight as given). */
size_t vai_conv2d_packed_weight_size(const vai_conv2d_args* args);
vai_status vai_conv2d_pack_weight(const vai_conv2d_args* args, void* packed, size_t packed_bytes,
                                  vai_stream_t stream);

/* The reference's MAX_CAUSAL_BLOCKS (/root/reference/vai/shaders/common/
 * spec_constants.h:35). */
#define VAI_MAX_CAUSAL_BLOCKS 32

/* ---------------------------------------------------------------------------
 * Attention scores: S[b,h,i,j] = scale * sum_d Q[b,h,i,d] K[b,h/g,j,d],
 * g = Hq/Hkv, fp32 accumulation, S fp32. causal != 0 hides key j from query i
 * when j > i + (Tkv - Tq) (queries align with the keys' end); span > 0 also
 * hides j < i + Tkv - Tq + 1 - span. Hidden entries are -inf.
 * A block mask (mask_blocks > 0, causal must then be 0) replaces the causal
 * flag with the reference's list of blocks, each causal or fully visible
 * (writeCausalMask, /root/reference/vai/nodes/attention.h:40-55): bit
 * (mask_blocks - 1 - k) of mask_bits marks block k causal, mask_block_end
 * holds the ends (query rows, increasing) of every block but the last, which
 * ends at Tq. A query in a causal block sees keys up to itself, one in a full
 * block sees keys up to its block's end (common/causal_mask.h:25-38): a
 * prefix-LM mask is {2 blocks, bits 0b01, end {prefix}}.
 * Q [batch,Hq,Tq,D], K [batch,Hkv,Tkv,D], same dtype (f16 or f32).
 * The Q.K^T stage of the reference's attention kernels
 * (/root/reference/vai/shaders/attention.comp:155-182,
 *  attention-fa.comp:581-591, common/causal_mask.h:25-42).
 * ------------------------------------------------------------------------- */
typedef struct {
    float* scores;
    const void* q;
    const void* k;
    uint32_t batch, hq, hkv, tq, tkv, head_dim;
    int32_t dtype;
    float scale;
    uint32_t causal;
    uint32_t span;
    uint32_t mask_blocks;                                  /* 0: the causal flag alone */
    uint32_t mask_bits;
    uint32_t mask_block_end[VAI_MAX_CAUSAL_BLOCKS - 1];
} vai_attn_scores_args;

vai_status vai_attn_scores_launch(const vai_attn_scores_args* args, vai_stream_t stream);

/* ---------------------------------------------------------------------------
 * Attention: O[b,i,h,:] = sum_j softmax_j(scale * Q[b,h,i,:].K[b,h/g,j,:] +
 * mask) V[b,h/g,j,:], g = Hq/Hkv -- the reference's Attention node, with or
 * without its KV cache (/root/reference/vai/nodes/attention.h:77-140,
 * 216-245, 979-1304; shaders/attention-fa.comp, attention.comp,
 * attention-fa-reduce.comp).
 *   Q [batch,Hq,Tq,D] in q_dtype, K / V [batch,Hkv,Tkv,D] in kv_dtype (f32 or
 *   f16 each, as typeI / typeKV, attention.h:86-88); O token-major
 *   [batch,Tq,Hq,D] in o_dtype (attention-fa.comp:8,96 and attention.h:
 *   1220-1223), so that [batch,Tq,Hq*D] is a reshape.
 *   Queries and keys align at their ends (query i sits at key i + Tkv - Tq).
 *   The mask is vai_attn_scores_launch's: causal = 0 and mask_blocks = 0 is
 *   no mask at all, the reference's default when setCausalMask was never
 *   called (attention.h:129). A query with no visible key gives zeros.
 *   Any head dim 1..2048. D % 8 == 0 with 16 <= D <= 256 (the reference's
 *   flash-attention gate, attention.h:916-945) and 16-byte aligned operands
 *   take the MFMA flash kernel: fp32 softmax statistics and accumulation,
 *   Q.K^T and P.V on fp16 operands (fp32 Q is rounded to fp16 as the
 *   reference's f16-staged tiles do, fp32 K / V are rounded into workspace
 *   copies first, P enters P.V as fp16). Every other head dim takes a plain
 *   fp32 kernel (the reference's naive attention.comp role).
 *   Long key ranges may be split over workgroups and merged; fp32 K / V and
 *   the split need vai_attention_workspace_size() bytes of workspace.
 * ------------------------------------------------------------------------- */
typedef struct {
    void* out;
    const void* q;
    const void* k;
    const void* v;
    int32_t o_dtype;
    int32_t q_dtype;              /* VAI_DTYPE_F32 or VAI_DTYPE_F16 */
    int32_t kv_dtype;             /* VAI_DTYPE_F32 or VAI_DTYPE_F16, K and V alike */
    uint32_t batch, hq, hkv, tq, tkv, head_dim;
    float scale;                  /* 0: 1/sqrt(head_dim), as attention.h:1254 */
    uint32_t causal;
    uint32_t span;
    void* workspace;              /* vai_attention_workspace_size() bytes, or NULL when that is 0 */
    size_t workspace_bytes;
    uint32_t mask_blocks;                                  /* as vai_attn_scores_args */
    uint32_t mask_bits;
    uint32_t mask_block_end[VAI_MAX_CAUSAL_BLOCKS - 1];
    /* The KV cache (kvCacheSize / kvCacheDtype / kvCacheRing and the counter,
     * attention.h:108-140, 216-245, 1003-1023): cache_size = 0 turns it off.
     * With a cache (batch 1), k_cache / v_cache hold [Hkv, cache_size, D] in
     * cache_dtype, and cache_count points at a device-readable uint32: the
     * positions the cache held before this call, read by the kernels when
     * they run (the reference's kvCacheCount, which the model rewrites before
     * each forward, so a recorded graph follows it). The call appends its Tkv
     * new K / V rows at positions count .. count + Tkv - 1 (row p, or
     * p % cache_size for a ring, whose size must be a multiple of 64), then
     * attends positions [0, count + Tkv): query i sits at position count +
     * max(i + Tkv - Tq, 0) and sees up to count + (its mask end among the
     * new keys), attention-fa.comp:137-146,470-478. K / V may be NULL with
     * Tkv = 0: the call attends the cache alone. The caller keeps count + Tkv
     * <= cache_size without a ring, and advances the count itself. */
    void* k_cache;
    void* v_cache;
    const uint32_t* cache_count;
    uint32_t cache_size;
    int32_t cache_dtype;          /* VAI_DTYPE_F32 or VAI_DTYPE_F16 */
    uint32_t cache_ring;
} vai_attention_args;

vai_status vai_attention_launch(const vai_attention_args* args, vai_stream_t stream);
/* Bytes of workspace a launch needs: nonzero when fp32 K / V take the flash
 * kernel (their fp16 copies), or when the query tiles alone do not fill the
 * GPU and long key ranges are split over workgroups (partial results merged by
 * a second pass, the split-K of attention-fa-reduce.comp). */
size_t vai_attention_workspace_size(const vai_attention_args* args);

/* ---------------------------------------------------------------------------
 * Device memory and streams: what the host side (vai::Tensor's pooled
 * buffers, the reference's eva::Buffer role) and the tests use.
 * ------------------------------------------------------------------------- */
vai_status vai_device_count(int* count);
vai_status vai_set_device(int device);
vai_status vai_malloc(void** ptr, size_t bytes);
vai_status vai_free(void* ptr);
vai_status vai_memcpy_h2d(void* dst, const void* src, size_t bytes, vai_stream_t stream);
vai_status vai_memcpy_d2h(void* dst, const void* src, size_t bytes, vai_stream_t stream);
vai_status vai_memcpy_d2d(void* dst, const void* src, size_t bytes, vai_stream_t stream);
vai_status vai_memset(void* dst, int value, size_t bytes, vai_stream_t stream);
vai_status vai_stream_create(vai_stream_t* stream);
vai_status vai_stream_destroy(vai_stream_t stream);
vai_status vai_stream_sync(vai_stream_t stream);
vai_status vai_device_sync(void);
const char* vai_status_string(vai_status status);

/* Timing: launches fn-equivalent work is the caller's; these wrap hipEvents
 * recorded on the stream the kernels run on. */
typedef struct ihipEvent_t* vai_event_t;
vai_status vai_event_create(vai_event_t* ev);
vai_status vai_event_destroy(vai_event_t ev);
vai_status vai_event_record(vai_event_t ev, vai_stream_t stream);
vai_status vai_event_sync(vai_event_t ev);
vai_status vai_event_elapsed_ms(float* ms, vai_event_t start, vai_event_t stop);

/* Record once, replay: the launches a stream sees between begin and end are
 * captured into a HIP graph and replayed by vai_graph_launch. This is the
 * gfx950 form of NeuralNet's command buffer that is recorded once and
 * resubmitted while shapes stay the same (/root/reference/vai/engine/
 * neural-net.h:377-449). The stream must not be the null stream. */
typedef struct vai_graph_s* vai_graph_t;
vai_status vai_graph_begin_capture(vai_stream_t stream);
vai_status vai_graph_end_capture(vai_stream_t stream, vai_graph_t* graph);
vai_status vai_graph_launch(vai_graph_t graph, vai_stream_t stream);
vai_status vai_graph_destroy(vai_graph_t graph);

#ifdef __cplusplus
}
#endif
#endif /* VAI_AMD_H */
