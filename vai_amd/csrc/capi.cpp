// capi.cpp -- the extern "C" boundary (include/vai_amd.h): argument checks,
// kernel selection by shape and dtype, and the device-memory helpers.
//
// Selection replaces the reference's per-vendor tables (selectLinearTile,
// /root/reference/vai/nodes/linear.h:2101-2119; selectConvPlan,
// /root/reference/vai/nodes/convolution.h:5408-5443) with one rule set for
// gfx950: M <= 8 streams W through the slab GEMV (linear.h:320), larger M
// takes the MFMA GEMM with the largest tile that still gives the 256 CUs at
// least one workgroup each, and split-K when even the smallest tile leaves
// most CUs idle and K is long.
#include <cmath>
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include "../../include/vai_amd.h"
#include "kernels.h"
#include "launch_once.h"

using namespace vai_dev;

namespace {

// The current device's CU count for the plans; 256 (an MI355X) when no
// device is visible, so that host-only plan queries see the target's plans.
uint32_t plan_cus()
{
    int cus = 0;
    return device_cus(&cus) == hipSuccess && cus > 0 ? (uint32_t)cus : 256u;
}

bool dtype_ok(int32_t d) { return d == VAI_DTYPE_F32 || d == VAI_DTYPE_F16; }
size_t dtype_bytes(int32_t d) { return d == VAI_DTYPE_F16 ? 2 : 4; }
vai_status hip_status(hipError_t e) { return e == hipSuccess ? VAI_OK : (vai_status)e; }

struct LinearPlan {
    enum Kind { Slab, SlabThenGate, Tile, BigTile, PackedTile, F32Small, Acc16Tile } kind;
    bool packed_gemv;   // Slab / SlabThenGate over the packed weight
    GemmTile tile;
    uint32_t bm, bn;
    uint32_t split_size, splits;
    size_t workspace;
};

uint32_t tiles_of(uint32_t M, uint32_t N, uint32_t bm, uint32_t bn)
{
    return ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

vai_status check_linear(const vai_linear_args* a)
{
    if (!a || !a->out || !a->in || !a->weight) return VAI_ERR_INVALID_ARG;
    if (a->M == 0 || a->N == 0 || a->K == 0) return VAI_ERR_SHAPE;
    if (!dtype_ok(a->o_dtype) || !dtype_ok(a->i_dtype) || !dtype_ok(a->w_dtype)) return VAI_ERR_DTYPE;
    if (a->bias && !dtype_ok(a->b_dtype)) return VAI_ERR_DTYPE;
    if (a->epilogue > VAI_EPI_SIGMOID || a->residual_order > 1) return VAI_ERR_INVALID_ARG;
    const uint64_t MN = (uint64_t)a->M * a->N;
    if (a->bias && a->bias_repeat && (a->bias_repeat % a->N != 0 || MN % a->bias_repeat != 0)) return VAI_ERR_SHAPE;
    if (a->residual && a->residual_repeat && (a->residual_repeat % a->N != 0 || MN % a->residual_repeat != 0))
        return VAI_ERR_SHAPE;
    if (a->split_size && a->split_size < 32) return VAI_ERR_INVALID_ARG;
    if (a->acc_dtype != VAI_DTYPE_F32 && a->acc_dtype != VAI_DTYPE_F16 && a->acc_dtype != VAI_DTYPE_NONE)
        return VAI_ERR_DTYPE;
    if (a->gated) {
        if (a->N % 2 != 0 || a->gate_epilogue > VAI_EPI_SIGMOID) return VAI_ERR_SHAPE;
        if (a->epilogue != VAI_EPI_NONE || a->residual || a->scalar_scale != 1.0f) return VAI_ERR_UNSUPPORTED;
        if (a->bias && a->bias_repeat != a->N) return VAI_ERR_UNSUPPORTED;   // a [2H] bias row only
    }
    return VAI_OK;
}

// The packed weight's shapes: fp16 I and W, K % 128 == 0, K >= 256.
bool linear_packable(const vai_linear_args* a)
{
    return a && a->i_dtype == VAI_DTYPE_F16 && a->w_dtype == VAI_DTYPE_F16 && a->N > 0 && a->K >= 256 &&
           a->K % 128 == 0 && (!a->gated || a->N % 2 == 0);
}

}   // namespace

// ggmlSplitSize (/root/reference/vai/nodes/linear.h:600-604): the span each of
// `splits` splits covers, rounded up to whole 256-blocks.
uint32_t acc16_split_size(uint32_t K, uint32_t splits)
{
    return ((K + splits - 1) / splits + 255) / 256 * 256;
}

// The split count the reference gives an fp16-accumulating Linear with
// splitSize 0 on the scalar tile path (otherLinearSplitCount -> ggmlGuessSplitCount,
// linear.h:606-632, 2079-2084): the tile is ggml's scalar warptile of the
// shape's tier (ggmlGuessTier / ggmlScalarWarptile, linear.h:485-546:
// S = 32x32 when M or N <= 32, M = 64x64 when M or N <= 64, else L =
// 128x128; wgM is the same for every subgroup size), split only a grid of at
// most half (cores / tiles splits) or two thirds (3 splits) of the cores with
// K >= 2048, at most 8, fewer while the last 256-rounded span would be empty.
// `cores` is the device's compute-unit count, as computeBlockCount() reports.
uint32_t acc16_guess_splits(uint32_t M, uint32_t N, uint32_t K, uint32_t cores)
{
    const uint32_t wg = (M <= 32 || N <= 32) ? 32 : (M <= 64 || N <= 64) ? 64 : 128;
    if (cores == 0 || N < wg || M < wg || K < 2048) return 1;
    const uint32_t tiles = ((M + wg - 1) / wg) * ((N + wg - 1) / wg);
    uint32_t s = 1;
    if (tiles <= cores / 2) s = cores / tiles;
    else if (tiles <= cores * 2 / 3) s = 3;
    s = std::min(s, 8u);
    while (s > 1 && acc16_split_size(K, s) * (s - 1) >= K) --s;
    return s;
}

namespace {

LinearPlan plan_linear(const vai_linear_args* a)
{
    LinearPlan p{};
    const uint32_t M = a->M, N = a->N, K = a->K;
    if (M <= 8) {
        p.kind = a->gated ? LinearPlan::SlabThenGate : LinearPlan::Slab;
        // From 3 rows on, the matrix cores over the packed weight (whole 1 KB
        // fragments per load) beat the VALU dot products; 1-2 rows stream W
        // rows directly (measured on config 2: 6.4 vs 7.2 us at M = 1).
        p.packed_gemv = a->packed_weight && M >= 3 && linear_packable(a) &&
                        ((uintptr_t)a->packed_weight % 16) == 0 && ((uintptr_t)a->in % 16) == 0;
        p.splits = 1;
        p.split_size = K;
        p.workspace = a->gated ? (size_t)M * N * 4 : 0;
        return p;
    }
    if (a->acc_dtype == VAI_DTYPE_F16 && !(a->i_dtype == VAI_DTYPE_F32 && a->w_dtype == VAI_DTYPE_F32)) {
        // fp16 accumulation in the reference's order. Each split starts its
        // own fp16 chain, so the split count is the reference's: the
        // requested span, else ggml's guess for its scalar tile.
        p.kind = LinearPlan::Acc16Tile;
        if (a->split_size) {
            p.split_size = a->split_size;
        } else {
            const uint32_t s = acc16_guess_splits(M, N, K, plan_cus());
            p.split_size = s > 1 ? acc16_split_size(K, s) : K;
        }
        p.splits = (K + p.split_size - 1) / p.split_size;
        p.workspace = p.splits > 1 ? (size_t)p.splits * M * N * 4 : 0;
        return p;
    }
    p.kind = LinearPlan::Tile;
    {
        GemmParams g{};
        g.a_dtype = a->i_dtype; g.b_dtype = a->w_dtype; g.M = M; g.N = N; g.K = K; g.H = a->gated ? N / 2 : 0;
        g.A = a->in; g.B = a->weight; g.splits = 1; g.batch = 1;
        if (a->split_size == 0 && a->packed_weight) {
            // Fewer 256x256 tiles than half the CUs (a down projection: M=2048,
            // N=3072 is 96 tiles): split K so the units fill the chip, the
            // partial planes summed by the reduce pass.
            const uint32_t tiles = tiles_of(M, a->gated ? N / 2 : N, 256, a->gated ? 128 : 256);
            uint32_t splits = 1;
            if (!a->gated && tiles < plan_cus() / 2) {
                splits = std::max<uint32_t>(1, std::min<uint32_t>(plan_cus() / tiles, K / 256));
                while (splits > 1 && K % (splits * 128) != 0) --splits;
            }
            g.splits = splits;
            if (gemm_packed_ok(g, a->gated)) {
                p.kind = LinearPlan::PackedTile;
                p.splits = splits;
                p.split_size = K / splits;
                p.workspace = splits > 1 ? (size_t)splits * M * N * 4 : 0;
                return p;
            }
            g.splits = 1;
        }
        // fp32 problems with fewer 64x64 tiles than CUs: one launch over the
        // full K with a CU-filling tile count, instead of split-K + reduce
        if (a->split_size == 0 && !a->gated && gemm_f32_ok(g) && tiles_of(M, N, 64, 64) < plan_cus()) {
            const int nf = gemm_f32_nf(M, N, plan_cus());
            p.kind = LinearPlan::F32Small;
            p.bm = 32;
            p.bn = 16 * nf;
            p.splits = 1;
            p.split_size = K;
            p.workspace = 0;
            return p;
        }
        if (a->split_size == 0 && gemm_big_ok(g, a->gated)) {
            p.kind = LinearPlan::BigTile;
            p.splits = 1;
            p.split_size = K;
            p.workspace = 0;
            return p;
        }
    }
    const bool f32 = a->i_dtype == VAI_DTYPE_F32 && a->w_dtype == VAI_DTYPE_F32;
    const uint32_t bk = f32 ? 16 : 32;
    // Candidate tiles, largest first (the gated kernel pairs fragments, so its
    // smallest N tile is 128 columns = 64 output columns).
    struct Cand { GemmTile t; uint32_t bm, bn; };
    const Cand cands[] = {
        {GemmTile::T256x128, 256, 128}, {GemmTile::T128x128, 128, 128},
        {GemmTile::T128x64, 128, a->gated ? 128u : 64u}, {GemmTile::T64x64, 64, a->gated ? 128u : 64u},
    };
    const uint32_t ncols = N;   // gated: 2H logical columns
    Cand pick = cands[3];
    for (const Cand& c : cands) {
        if (f32 && c.bm == 256) continue;   // fp32 staging keeps 128-row tiles (LDS, registers)
        if (tiles_of(M, ncols, c.bm, c.bn) >= plan_cus()) { pick = c; break; }
    }
    p.tile = pick.t;
    p.bm = pick.bm;
    p.bn = pick.bn;
    const uint32_t tiles = tiles_of(M, ncols, pick.bm, pick.bn);
    if (a->split_size) {
        p.split_size = a->split_size;
        p.splits = (K + a->split_size - 1) / a->split_size;
    } else {
        uint32_t splits = 1;
        if (f32 && tiles < plan_cus() && K >= 256) {
            // fp32 matrix cores run at 1/16 of the fp16 rate, so a small fp32
            // GEMM is bound by how many SIMDs it keeps busy: aim at ~1.5
            // workgroups per CU (config 1, 96 tiles, K 768: 4 splits, 19 us,
            // against 36.7 us unsplit and 21 us with 3 or 6 splits)
            splits = std::min<uint32_t>((3 * plan_cus() / 2 + tiles / 2) / tiles, K / 128);
            splits = std::max<uint32_t>(splits, 1);
        } else if (tiles < plan_cus() / 2 && K >= 1024) {
            splits = std::min<uint32_t>((plan_cus() + tiles - 1) / tiles, K / 256);
            splits = std::max<uint32_t>(splits, 1);
        }
        p.split_size = splits > 1 ? ((K + splits - 1) / splits + bk - 1) / bk * bk : K;
        p.splits = (K + p.split_size - 1) / p.split_size;
    }
    p.workspace = p.splits > 1 ? (size_t)p.splits * M * N * 4 : 0;
    return p;
}

const char* tile_name(GemmTile t, bool gated)
{
    switch (t) {
    case GemmTile::T64x64: return gated ? "64x128" : "64x64";
    case GemmTile::T128x64: return gated ? "128x128" : "128x64";
    case GemmTile::T128x128: return "128x128";
    default: return "256x128";
    }
}

}   // namespace

extern "C" {

size_t vai_linear_workspace_size(const vai_linear_args* a)
{
    if (check_linear(a) != VAI_OK) return 0;
    return plan_linear(a).workspace;
}

vai_status vai_linear_plan(const vai_linear_args* a, char* name, size_t name_len, uint32_t* split_count)
{
    const vai_status st = check_linear(a);
    if (st != VAI_OK) return st;
    const LinearPlan p = plan_linear(a);
    char buf[64];
    if (p.kind == LinearPlan::Slab || p.kind == LinearPlan::SlabThenGate) {
        SlabParams sp{};
        sp.K = a->K; sp.w_dtype = a->w_dtype; sp.i_dtype = a->i_dtype; sp.weight = a->weight; sp.in = a->in;
        sp.M = a->M;
        snprintf(buf, sizeof buf, "%s%s",
                 p.packed_gemv ? "slab_packed"
                 : (sp.M >= 5 && gemv_mfma_ok(sp)) ? "slab_mfma"
                 : slab_vec_ok(sp) ? "slab" : "slab_scalar",
                 p.kind == LinearPlan::SlabThenGate ? "+gate" : "");
    } else if (p.kind == LinearPlan::Acc16Tile) {
        snprintf(buf, sizeof buf, "tile_acc16_64x64%s", a->gated ? "_gated" : "");
    } else if (p.kind == LinearPlan::F32Small) {
        snprintf(buf, sizeof buf, "tile_f32_32x%u_kwaves", p.bn);
    } else if (p.kind == LinearPlan::BigTile || p.kind == LinearPlan::PackedTile) {
        snprintf(buf, sizeof buf, "tile_f16_256x256%s%s", p.kind == LinearPlan::PackedTile ? "_packed" : "",
                 a->gated ? "_gated" : "");
    } else {
        const bool f32 = a->i_dtype == VAI_DTYPE_F32 && a->w_dtype == VAI_DTYPE_F32;
        snprintf(buf, sizeof buf, "tile_%s_%s%s", f32 ? "f32" : "f16", tile_name(p.tile, a->gated),
                 a->gated ? "_gated" : "");
    }
    if (name && name_len) { strncpy(name, buf, name_len - 1); name[name_len - 1] = 0; }
    if (split_count) *split_count = p.splits;
    return VAI_OK;
}

// The launches of one Linear; `a` is checked, `p` its plan, and when the plan
// needs a workspace, a->workspace holds at least p.workspace bytes.
static vai_status linear_run(const vai_linear_args* a, const LinearPlan& p, hipStream_t s)
{

    if (p.kind == LinearPlan::Slab || p.kind == LinearPlan::SlabThenGate) {
        SlabParams sp{};
        sp.in = a->in; sp.weight = a->weight; sp.bias = a->bias; sp.residual = a->residual;
        sp.M = a->M; sp.N = a->N; sp.K = a->K;
        sp.i_dtype = a->i_dtype; sp.w_dtype = a->w_dtype; sp.b_dtype = a->b_dtype;
        sp.epilogue = a->epilogue; sp.residual_order = a->residual_order;
        sp.bias_repeat = a->bias_repeat; sp.residual_repeat = a->residual_repeat;
        sp.scalar_scale = a->scalar_scale;
        if (p.kind == LinearPlan::Slab) {
            sp.out = a->out; sp.o_dtype = a->o_dtype;
            if (p.packed_gemv) return hip_status(gemv_packed_launch(sp, a->packed_weight, false, nullptr, s));
            return hip_status(slab_launch(sp, s));
        }
        // Gated at M <= 8: the fp32 Linear output, then the gating pass.
        sp.out = a->workspace; sp.o_dtype = VAI_DTYPE_F32;
        hipError_t e = p.packed_gemv ? gemv_packed_launch(sp, a->packed_weight, true, (float*)a->workspace, s)
                                     : slab_launch(sp, s);
        if (e != hipSuccess) return hip_status(e);
        return hip_status(gated_mul_launch(a->out, a->o_dtype, a->workspace, VAI_DTYPE_F32, a->M, a->N / 2,
                                           a->gate_epilogue, s));
    }

    GemmParams g{};
    g.A = a->in; g.B = a->weight;
    g.a_dtype = a->i_dtype; g.b_dtype = a->w_dtype;
    g.M = a->M; g.N = a->N; g.K = a->K;
    g.batch = 1; g.b_group = 1;
    g.split_size = p.split_size; g.splits = p.splits;
    g.bias = a->bias; g.bias_dtype = a->b_dtype; g.bias_repeat = a->bias_repeat;
    g.residual = a->residual; g.residual_dtype = a->o_dtype; g.residual_repeat = a->residual_repeat;
    g.epilogue = a->gated ? a->gate_epilogue : a->epilogue;
    g.residual_order = a->residual_order; g.scalar_scale = a->scalar_scale;
    g.H = a->gated ? a->N / 2 : 0;
    if (p.splits > 1) { g.C = a->workspace; g.c_dtype = VAI_DTYPE_F32; }
    else { g.C = a->out; g.c_dtype = a->o_dtype; }
    if (p.kind == LinearPlan::PackedTile) {
        hipError_t e = gemm_packed_launch(g, a->packed_weight, a->gated != 0, s);
        if (e != hipSuccess || p.splits == 1) return hip_status(e);
        return hip_status(linear_reduce_launch(a->out, a->o_dtype, (const float*)a->workspace, p.splits,
                                               (size_t)a->M * a->N, a->bias, a->b_dtype, a->bias_repeat, a->residual,
                                               a->residual_repeat, a->epilogue, a->residual_order, a->scalar_scale, 0,
                                               0, a->N, s));
    }
    if (p.kind == LinearPlan::BigTile) return hip_status(gemm_big_launch(g, a->gated != 0, s));
    if (p.kind == LinearPlan::Acc16Tile) {
        hipError_t e = gemm_acc16_launch(g, a->gated != 0, s);
        if (e != hipSuccess || p.splits == 1) return hip_status(e);
        return hip_status(linear_reduce_launch(a->out, a->o_dtype, (const float*)a->workspace, p.splits,
                                               (size_t)a->M * (a->gated ? a->N / 2 : a->N), a->bias, a->b_dtype,
                                               a->bias_repeat, a->residual, a->residual_repeat, a->epilogue,
                                               a->residual_order, a->scalar_scale, a->gated ? a->N / 2 : 0,
                                               a->gate_epilogue, a->N, s));
    }
    if (p.kind == LinearPlan::F32Small) return hip_status(gemm_f32_launch(g, (int)(p.bn / 16), s));
    hipError_t e = gemm_launch(g, a->gated ? BKind::Gated : BKind::Dense,
                               a->gated ? EpiKind::Gated : EpiKind::Linear, p.tile, s);
    if (e != hipSuccess || p.splits == 1) return hip_status(e);
    const size_t MN = (size_t)a->M * (a->gated ? a->N / 2 : a->N);
    return hip_status(linear_reduce_launch(a->out, a->o_dtype, (const float*)a->workspace, p.splits, MN,
                                           a->bias, a->b_dtype, a->bias_repeat, a->residual, a->residual_repeat,
                                           a->epilogue, a->residual_order, a->scalar_scale,
                                           a->gated ? a->N / 2 : 0, a->gate_epilogue, a->N, s));
}

vai_status vai_linear_launch(const vai_linear_args* a, vai_stream_t stream)
{
    const vai_status st = check_linear(a);
    if (st != VAI_OK) return st;
    const LinearPlan p = plan_linear(a);
    if (p.workspace && (!a->workspace || a->workspace_bytes < p.workspace)) return VAI_ERR_WORKSPACE;
    return linear_run(a, p, (hipStream_t)stream);
}

// ---- vai_linear_launch_noalloc: the workspace is a file-scope device array.
// Each device holds its own copy from the library's load until the process
// ends. Host code must use the address hipGetSymbolAddress returns for the
// current device, never the array's name (a host-side stand-in).
static __device__ __align__(256) unsigned char scratch[VAI_NOALLOC_SCRATCH_BYTES];

static hipError_t scratch_address(void** ptr)
{
    static PerDevice once;
    static void* addr[kMaxDevices] = {};
    const hipError_t e = once.run([](int d) { return hipGetSymbolAddress(&addr[d], HIP_SYMBOL(scratch)); });
    if (e != hipSuccess) return e;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    *ptr = addr[dev];
    return *ptr ? hipSuccess : hipErrorInvalidSymbol;
}

vai_status vai_linear_launch_noalloc(const vai_linear_args* a, vai_stream_t stream)
{
    const vai_status st = check_linear(a);
    if (st != VAI_OK) return st;
    const LinearPlan p = plan_linear(a);
    if (p.workspace > VAI_NOALLOC_SCRATCH_BYTES) return VAI_ERR_WORKSPACE;
    vai_linear_args b = *a;
    b.workspace = nullptr;
    b.workspace_bytes = 0;
    if (p.workspace) {
        // Every kernel that uses the workspace writes each element it later
        // reads (split-K planes, the ungated GEMV output), so the array needs
        // no clearing between calls.
        const hipError_t e = scratch_address(&b.workspace);
        if (e != hipSuccess) return hip_status(e);
        b.workspace_bytes = VAI_NOALLOC_SCRATCH_BYTES;
    }
    return linear_run(&b, p, (hipStream_t)stream);
}

size_t vai_linear_packed_weight_size(const vai_linear_args* a)
{
    if (!linear_packable(a)) return 0;
    return gemm_packed_weight_bytes(a->N, a->K, a->gated ? a->N / 2 : 0, a->gated != 0);
}

vai_status vai_linear_pack_weight(const vai_linear_args* a, void* packed, size_t packed_bytes, vai_stream_t stream)
{
    if (!a || !a->weight || !packed) return VAI_ERR_INVALID_ARG;
    if (!linear_packable(a)) return VAI_ERR_UNSUPPORTED;
    const size_t need = vai_linear_packed_weight_size(a);
    if (packed_bytes < need) return VAI_ERR_WORKSPACE;
    return hip_status(gemm_pack_weight(packed, a->weight, a->N, a->K, a->gated ? a->N / 2 : 0, a->gated != 0,
                                       (hipStream_t)stream));
}

// The kernels' mask rule from the causal flag or a block list; checks the list
// as writeCausalMask does (attention.h:46-55): at most 32 blocks, ends
// increasing and nonzero.
static vai_status make_mask(MaskRule& m, uint32_t tq, uint32_t tkv, uint32_t causal, uint32_t span,
                            uint32_t blocks, uint32_t bits, const uint32_t* ends)
{
    m = MaskRule{};
    m.tq = tq; m.tkv = tkv; m.span = span;
    if (blocks == 0) {
        m.blocks = causal ? 1 : 0;
        m.bits = 1;
        return VAI_OK;
    }
    if (causal || blocks > VAI_MAX_CAUSAL_BLOCKS) return VAI_ERR_INVALID_ARG;
    for (uint32_t k = 0; k + 1 < blocks; ++k) {
        if (ends[k] == 0 || (k > 0 && ends[k] <= ends[k - 1])) return VAI_ERR_INVALID_ARG;
        m.end[k] = ends[k];
    }
    if (blocks == 1) {   // one block: causal or no mask at all
        m.blocks = bits & 1u;
        m.bits = 1;
        return VAI_OK;
    }
    m.blocks = blocks;
    m.bits = blocks == 32 ? bits : bits & ((1u << blocks) - 1);
    return VAI_OK;
}

static vai_status attention_params(const vai_attention_args* a, AttnParams& p)
{
    if (!a || !a->q) return VAI_ERR_INVALID_ARG;
    const bool cache = a->cache_size > 0;
    // K / V: needed unless a cache supplies every key (Tkv = 0)
    if ((a->tkv > 0 || !cache) && (!a->k || !a->v)) return VAI_ERR_INVALID_ARG;
    if (cache && (!a->k_cache || !a->v_cache || !a->cache_count)) return VAI_ERR_INVALID_ARG;
    const auto f32_or_f16 = [](int32_t d) { return d == VAI_DTYPE_F32 || d == VAI_DTYPE_F16; };
    if (!f32_or_f16(a->q_dtype) || !dtype_ok(a->o_dtype)) return VAI_ERR_DTYPE;
    if (a->tkv > 0 && !f32_or_f16(a->kv_dtype)) return VAI_ERR_DTYPE;
    if (cache && !f32_or_f16(a->cache_dtype)) return VAI_ERR_DTYPE;
    if (a->batch == 0 || a->hq == 0 || a->hkv == 0 || a->tq == 0 || (a->tkv == 0 && !cache) || a->head_dim == 0 ||
        a->hq % a->hkv != 0)
        return VAI_ERR_SHAPE;
    // one counter per call: cached sequences cannot sit at different positions
    // (attention.h:1016); a ring's tiles must not wrap it; without a ring the
    // new rows must fit
    if (cache && (a->batch != 1 || (a->cache_ring && a->cache_size % 64 != 0) ||
                  (!a->cache_ring && a->tkv > a->cache_size)))
        return VAI_ERR_SHAPE;
    p = AttnParams{};
    p.out = a->out; p.q = a->q;
    p.o_dtype = a->o_dtype; p.q_dtype = a->q_dtype;
    p.batch = a->batch; p.hq = a->hq; p.hkv = a->hkv; p.tq = a->tq; p.tkv = a->tkv; p.head_dim = a->head_dim;
    if (cache) {
        p.k = a->k_cache; p.v = a->v_cache; p.kv_dtype = a->cache_dtype;
        p.cache_count = a->cache_count; p.kv_rows = a->cache_size; p.ring = a->cache_ring ? 1u : 0u;
        p.k_new = a->k; p.v_new = a->v; p.new_dtype = a->kv_dtype;
    } else {
        p.k = a->k; p.v = a->v; p.kv_dtype = a->kv_dtype; p.kv_rows = a->tkv;
    }
    p.scale = a->scale != 0.f ? a->scale : 1.0f / std::sqrt((float)a->head_dim);
    p.span = a->span;
    if (vai_status st = make_mask(p.mask, a->tq, a->tkv, a->causal, a->span, a->mask_blocks, a->mask_bits,
                                  a->mask_block_end); st != VAI_OK)
        return st;
    p.causal = p.mask.blocks == 1;
    if (!attention_ok(p)) return VAI_ERR_UNSUPPORTED;
    attention_plan(p, plan_cus());
    return VAI_OK;
}

size_t vai_attention_workspace_size(const vai_attention_args* a)
{
    AttnParams p;
    if (attention_params(a, p) != VAI_OK) return 0;
    return attention_workspace_bytes(p);
}

vai_status vai_attention_launch(const vai_attention_args* a, vai_stream_t stream)
{
    AttnParams p;
    if (a && !a->out) return VAI_ERR_INVALID_ARG;
    vai_status st = attention_params(a, p);
    if (st != VAI_OK) return st;
    const size_t need = attention_workspace_bytes(p);
    if (need) {
        if (!a->workspace || a->workspace_bytes < need) return VAI_ERR_WORKSPACE;
        attention_set_workspace(p, a->workspace);
    }
    return hip_status(attention_launch(p, (hipStream_t)stream));
}

vai_status vai_gated_mul_launch(void* out, int32_t o_dtype, const void* in, int32_t i_dtype, uint32_t rows,
                                uint32_t H, uint32_t epilogue, vai_stream_t stream)
{
    if (!out || !in) return VAI_ERR_INVALID_ARG;
    if (!dtype_ok(o_dtype) || !dtype_ok(i_dtype)) return VAI_ERR_DTYPE;
    if (rows == 0 || H == 0) return VAI_ERR_SHAPE;
    if (epilogue > VAI_EPI_SIGMOID) return VAI_ERR_INVALID_ARG;
    return hip_status(gated_mul_launch(out, o_dtype, in, i_dtype, rows, H, epilogue, (hipStream_t)stream));
}

static vai_status check_conv(const vai_conv2d_args* a)
{
    if (!a || !a->out || !a->in || !a->weight) return VAI_ERR_INVALID_ARG;
    if (!dtype_ok(a->o_dtype) || !dtype_ok(a->i_dtype) || !dtype_ok(a->w_dtype)) return VAI_ERR_DTYPE;
    // fp16 activations and fp16 outputs need fp16 weights (convolution.h:4140-4142).
    if (a->w_dtype == VAI_DTYPE_F32 && (a->i_dtype == VAI_DTYPE_F16 || a->o_dtype == VAI_DTYPE_F16))
        return VAI_ERR_DTYPE;
    if (a->batch == 0 || a->ci == 0 || a->co == 0 || a->hi == 0 || a->wi == 0 || a->stride == 0)
        return VAI_ERR_SHAPE;
    if (a->kernel == 0 || a->kernel % 2 == 0) return VAI_ERR_SHAPE;
    if (a->epilogue > VAI_EPI_SIGMOID || a->residual_order > 1) return VAI_ERR_INVALID_ARG;
    return VAI_OK;
}

// fp16 weights and a band that fits in LDS take the packed NHWC kernel.
static bool conv_packed(const vai_conv2d_args* a)
{
    const uint32_t wo = (a->wi - 1) / a->stride + 1;
    return a->w_dtype == VAI_DTYPE_F16 && conv_nhwc_ok(a->ci, a->wi, wo, a->kernel);
}

size_t vai_conv2d_packed_weight_size(const vai_conv2d_args* a)
{
    if (check_conv(a) != VAI_OK || !conv_packed(a)) return 0;
    return conv_packed_weight_bytes(a->ci, a->co, a->kernel);
}

size_t vai_conv2d_workspace_size(const vai_conv2d_args* a)
{
    if (a && a->packed_weight) return 0;
    return vai_conv2d_packed_weight_size(a);
}

vai_status vai_conv2d_pack_weight(const vai_conv2d_args* a, void* packed, size_t bytes, vai_stream_t stream)
{
    const vai_status st = check_conv(a);
    if (st != VAI_OK) return st;
    if (!conv_packed(a)) return VAI_OK;
    if (!packed || bytes < conv_packed_weight_bytes(a->ci, a->co, a->kernel)) return VAI_ERR_WORKSPACE;
    return hip_status(conv_pack_weight((half_t_storage*)packed, (const half_t_storage*)a->weight, a->ci, a->co,
                                       a->kernel, (hipStream_t)stream));
}

vai_status vai_conv2d_launch(const vai_conv2d_args* a, vai_stream_t stream)
{
    const vai_status st = check_conv(a);
    if (st != VAI_OK) return st;
    const uint32_t ho = (a->hi - 1) / a->stride + 1, wo = (a->wi - 1) / a->stride + 1;
    if (conv_packed(a)) {
        const void* wp = a->packed_weight;
        if (!wp) {
            const size_t need = conv_packed_weight_bytes(a->ci, a->co, a->kernel);
            if (!a->workspace || a->workspace_bytes < need) return VAI_ERR_WORKSPACE;
            hipError_t e = conv_pack_weight((half_t_storage*)a->workspace, (const half_t_storage*)a->weight, a->ci,
                                            a->co, a->kernel, (hipStream_t)stream);
            if (e != hipSuccess) return hip_status(e);
            wp = a->workspace;
        }
        ConvParams c{};
        c.out = a->out; c.x = a->in; c.wp = (const half_t_storage*)wp;
        c.bias = a->bias; c.scale = a->scale; c.residual = a->residual;
        c.o_dtype = a->o_dtype; c.residual_dtype = a->i_dtype;
        c.batch = a->batch; c.ci = a->ci; c.hi = a->hi; c.wi = a->wi; c.co = a->co; c.ho = ho; c.wo = wo;
        c.ks = a->kernel; c.stride = a->stride; c.epilogue = a->epilogue; c.residual_order = a->residual_order;
        return hip_status(conv_launch(c, a->i_dtype, (hipStream_t)stream));
    }
    GemmParams g{};
    g.A = a->weight; g.B = a->in; g.C = a->out;
    g.a_dtype = a->w_dtype; g.b_dtype = a->i_dtype; g.c_dtype = a->o_dtype;
    g.M = a->co; g.N = ho * wo; g.K = a->ci * a->kernel * a->kernel;
    g.batch = a->batch; g.b_group = 1;
    g.a_batch_stride = 0;
    g.b_batch_stride = (size_t)a->ci * a->hi * a->wi;
    g.c_batch_stride = (size_t)a->co * ho * wo;
    g.split_size = g.K; g.splits = 1;
    g.bias = a->bias; g.bias_dtype = a->w_dtype; g.conv_scale = a->scale;
    g.residual = a->residual; g.residual_dtype = a->i_dtype;
    g.epilogue = a->epilogue; g.residual_order = a->residual_order; g.scalar_scale = 1.f;
    g.ci = a->ci; g.hi = a->hi; g.wi = a->wi; g.wo = wo; g.ks = a->kernel; g.stride = a->stride;
    const GemmTile t = tiles_of(g.M, g.N, 128, 64) * a->batch >= plan_cus() ? GemmTile::T128x64 : GemmTile::T64x64;
    return hip_status(gemm_launch(g, BKind::Im2col, EpiKind::Conv, t, (hipStream_t)stream));
}

vai_status vai_attn_scores_launch(const vai_attn_scores_args* a, vai_stream_t stream)
{
    if (!a || !a->scores || !a->q || !a->k) return VAI_ERR_INVALID_ARG;
    if (!dtype_ok(a->dtype)) return VAI_ERR_DTYPE;
    if (a->batch == 0 || a->hq == 0 || a->hkv == 0 || a->tq == 0 || a->tkv == 0 || a->head_dim == 0)
        return VAI_ERR_SHAPE;
    if (a->hq % a->hkv != 0) return VAI_ERR_SHAPE;
    GemmParams g{};
    g.A = a->q; g.B = a->k; g.C = a->scores;
    g.a_dtype = a->dtype; g.b_dtype = a->dtype; g.c_dtype = VAI_DTYPE_F32;
    g.M = a->tq; g.N = a->tkv; g.K = a->head_dim;
    g.batch = a->batch * a->hq; g.b_group = a->hq / a->hkv;
    g.a_batch_stride = (size_t)a->tq * a->head_dim;
    g.b_batch_stride = (size_t)a->tkv * a->head_dim;
    g.c_batch_stride = (size_t)a->tq * a->tkv;
    g.split_size = g.K; g.splits = 1;
    g.scalar_scale = a->scale; g.causal = a->causal; g.span = a->span;
    g.causal_offset = (int32_t)a->tkv - (int32_t)a->tq;
    if (vai_status st = make_mask(g.mask, a->tq, a->tkv, a->causal, a->span, a->mask_blocks, a->mask_bits,
                                  a->mask_block_end); st != VAI_OK)
        return st;
    g.causal = g.mask.blocks == 1;   // the diagonal fast path's flag (a block list takes the general one)
    if (scores_fast_ok(g)) return hip_status(scores_launch(g, (hipStream_t)stream));
    const GemmTile t = tiles_of(g.M, g.N, 128, 128) * g.batch >= plan_cus() ? GemmTile::T128x128 : GemmTile::T64x64;
    return hip_status(gemm_launch(g, BKind::Dense, EpiKind::Scores, t, (hipStream_t)stream));
}

// ---- device memory / streams / events ----
vai_status vai_device_count(int* count) { return hip_status(hipGetDeviceCount(count)); }
vai_status vai_set_device(int device) { return hip_status(hipSetDevice(device)); }
vai_status vai_malloc(void** ptr, size_t bytes) { return hip_status(hipMalloc(ptr, bytes)); }
vai_status vai_free(void* ptr) { return hip_status(hipFree(ptr)); }
vai_status vai_memcpy_h2d(void* dst, const void* src, size_t bytes, vai_stream_t s)
{
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)s);
    return hip_status(e);
}
vai_status vai_memcpy_d2h(void* dst, const void* src, size_t bytes, vai_stream_t s)
{
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)s);
    return hip_status(e);
}
vai_status vai_memcpy_d2d(void* dst, const void* src, size_t bytes, vai_stream_t s)
{
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)s));
}
vai_status vai_memset(void* dst, int value, size_t bytes, vai_stream_t s)
{
    return hip_status(hipMemsetAsync(dst, value, bytes, (hipStream_t)s));
}
vai_status vai_stream_create(vai_stream_t* s) { return hip_status(hipStreamCreate((hipStream_t*)s)); }
vai_status vai_stream_destroy(vai_stream_t s) { return hip_status(hipStreamDestroy((hipStream_t)s)); }
vai_status vai_stream_sync(vai_stream_t s) { return hip_status(hipStreamSynchronize((hipStream_t)s)); }
vai_status vai_device_sync(void) { return hip_status(hipDeviceSynchronize()); }
vai_status vai_event_create(vai_event_t* ev) { return hip_status(hipEventCreate((hipEvent_t*)ev)); }
vai_status vai_event_destroy(vai_event_t ev) { return hip_status(hipEventDestroy((hipEvent_t)ev)); }
vai_status vai_event_record(vai_event_t ev, vai_stream_t s)
{
    return hip_status(hipEventRecord((hipEvent_t)ev, (hipStream_t)s));
}
vai_status vai_event_sync(vai_event_t ev) { return hip_status(hipEventSynchronize((hipEvent_t)ev)); }
vai_status vai_event_elapsed_ms(float* ms, vai_event_t a, vai_event_t b)
{
    return hip_status(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
}

struct vai_graph_s {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

vai_status vai_graph_begin_capture(vai_stream_t s)
{
    if (!s) return VAI_ERR_INVALID_ARG;
    return hip_status(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal));
}

vai_status vai_graph_end_capture(vai_stream_t s, vai_graph_t* out)
{
    if (!s || !out) return VAI_ERR_INVALID_ARG;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)s, &g);
    if (e != hipSuccess) return hip_status(e);
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) { hipGraphDestroy(g); return hip_status(e); }
    *out = new vai_graph_s{g, x};
    return VAI_OK;
}

vai_status vai_graph_launch(vai_graph_t g, vai_stream_t s)
{
    if (!g) return VAI_ERR_INVALID_ARG;
    return hip_status(hipGraphLaunch(g->exec, (hipStream_t)s));
}

vai_status vai_graph_destroy(vai_graph_t g)
{
    if (!g) return VAI_OK;
    hipGraphExecDestroy(g->exec);
    hipGraphDestroy(g->graph);
    delete g;
    return VAI_OK;
}

const char* vai_status_string(vai_status s)
{
    switch ((int)s) {
    case VAI_OK: return "ok";
    case VAI_ERR_INVALID_ARG: return "invalid argument";
    case VAI_ERR_SHAPE: return "shape mismatch";
    case VAI_ERR_DTYPE: return "unsupported dtype combination";
    case VAI_ERR_WORKSPACE: return "workspace missing or too small";
    case VAI_ERR_UNSUPPORTED: return "unsupported configuration";
    default: return hipGetErrorString((hipError_t)s);
    }
}

}   // extern "C"
