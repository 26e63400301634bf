// nodes.cpp -- prepare()/run() of the matmul-path nodes.
#include <cstring>
#include "nodes.h"

#include <cmath>
#include <stdexcept>

namespace vai::node {

static int32_t code(Dtype d)
{
    switch (d) {
    case Dtype::Fp32: return VAI_DTYPE_F32;
    case Dtype::Fp16: return VAI_DTYPE_F16;
    default: return VAI_DTYPE_NONE;
    }
}

static void check(vai_status st, const char* what)
{
    if (st != VAI_OK) throw std::runtime_error(std::string(what) + ": " + vai_status_string(st));
}

static void* ptrOrNull(const Tensor& t) { return t.validShape() ? t.devicePtr() : nullptr; }

// causal / span from the node's config, or the block mask when one is set
template <class Args>
static void apply_mask(Args& a, bool causal, uint32_t span, const CausalMask& m)
{
    a.causal = causal ? 1 : 0;
    a.span = span;
    if (m.blockCount == 0) return;
    a.causal = 0;
    a.span = m.span;
    a.mask_blocks = m.blockCount;
    a.mask_bits = m.bits;
    for (uint32_t k = 0; k + 1 < m.blockCount; ++k) a.mask_block_end[k] = m.blockEnd[k];
}

// ---------------------------------------------------------------- Linear ----

Linear::Linear(Config config) : config_(config)
{
    require(config_.inDim > 0 && config_.outDim > 0, "Linear: inDim and outDim must be positive");
    require(config_.epilogue < Epilogue::Max, "Linear: bad epilogue");
    addSlot("out0", NodeSlot::output);
    addSlot("in0", NodeSlot::input);
    addSlot("weight", NodeSlot::persistent);
    addSlot("partial", NodeSlot::temporary);   // split-K partial sums, bound only when used
    addSlot("bias", NodeSlot::persistent);
    if (config_.acceptResidual) addSlot("residual", NodeSlot::input);
}

vai_linear_args Linear::args(bool withPointers) const
{
    vai_linear_args a{};
    const Tensor& in = (*this)["in0"];
    const Tensor& w = (*this)["weight"];
    a.M = M_;
    a.N = config_.outDim;
    a.K = config_.inDim;
    a.i_dtype = code(in.dtype());
    a.w_dtype = code(w.dtype());
    a.o_dtype = code(outputDtype());
    a.b_dtype = hasBias() ? code((*this)["bias"].dtype()) : VAI_DTYPE_NONE;
    a.epilogue = uint32_t(config_.epilogue);
    a.residual_order = uint32_t(config_.residualOrder);
    a.bias_repeat = biasRepeat_;
    a.residual_repeat = residualRepeat_;
    a.scalar_scale = config_.scalarScale;
    a.split_size = config_.splitSize;
    a.acc_dtype = accDtype_ == Dtype::Fp16 ? VAI_DTYPE_F16 : VAI_DTYPE_F32;
    if (fused_) {
        a.gated = 1;
        a.gate_epilogue = uint32_t(fused_->config_.activation);
        a.o_dtype = code(fused_->outputDtype());
    }
    if (withPointers) {
        a.in = in.devicePtr();
        a.weight = w.devicePtr();
        a.bias = hasBias() ? (*this)["bias"].devicePtr() : nullptr;
        a.residual = config_.acceptResidual ? ptrOrNull((*this)["residual"]) : nullptr;
        a.out = fused_ ? (*fused_)["out0"].devicePtr() : (*this)["out0"].devicePtr();
        const Tensor& part = (*this)["partial"];
        a.workspace = ptrOrNull(part);
        a.workspace_bytes = part.validShape() ? part.numBytes() : 0;
        a.packed_weight = packedMatches(a) ? packed_.ptr() : nullptr;
    } else {
        // placeholders so argument checks see non-null operands
        a.in = a.weight = a.out = reinterpret_cast<void*>(256);
        a.bias = hasBias() ? reinterpret_cast<void*>(256) : nullptr;
        a.residual = config_.acceptResidual ? reinterpret_cast<void*>(256) : nullptr;
    }
    return a;
}

bool Linear::packedMatches(const vai_linear_args& a) const
{
    return packed_ && packedFrom_ == (*this)["weight"].uploadId() && packedGated_ == (a.gated != 0);
}

bool Linear::canFuseGate(const GatedMul& gm) const
{
    (void)gm;
    const bool biasRow = !hasBias() || (*this)["bias"].numElements() == config_.outDim;
    return !config_.acceptResidual && config_.epilogue == Epilogue::None && config_.scalarScale == 1.0f &&
           config_.outDim % 2 == 0 && biasRow;
}

void Linear::prepare()
{
    const Tensor& in = (*this)["in0"];
    const Tensor& w = (*this)["weight"];
    const uint32_t N = config_.outDim, K = config_.inDim;
    require(in.validShape() && in.shape().back() == K, "Linear: input's last axis must be inDim");
    require(w.isShapeOf({N, K}), "Linear: weight must be [outDim, inDim]");
    require(w.gpuBufferBound(), "Linear: weight was not uploaded");
    M_ = outerSize(in.shape());
    // An operand covering O reads directly; a shorter one repeats over M (linear.h:2333-2338).
    auto repeatOf = [&](const Tensor& t) {
        const uint64_t outElems = uint64_t(M_) * N, elems = t.numElements();
        require(t.shape().back() == N && elems > 0 && outElems % elems == 0,
                "Linear: bias / residual must be [..., outDim] rows that tile the output");
        return elems == outElems ? 0u : uint32_t(elems);
    };
    biasRepeat_ = hasBias() ? repeatOf((*this)["bias"]) : 0;
    residualRepeat_ = 0;
    if (config_.acceptResidual) {
        const Tensor& r = (*this)["residual"];
        require(r.dtype() == outputDtype(), "Linear: residual must have the output dtype");
        residualRepeat_ = repeatOf(r);
    }
    std::vector<uint32_t> shape = in.shape();
    shape.back() = N;
    (*this)["out0"] = Tensor(shape, outputDtype());

    vai_linear_args a = args(false);
    // Prefill shapes and decode GEMVs of 3-8 rows stream a fragment-major copy
    // of the weight into the matrix cores; it is made once per weight buffer
    // and layout (a fused gate changes the layout), as the reference prepares
    // its weights once. The library's plan says whether this shape uses it.
    vai_linear_args probe = a;
    probe.packed_weight = reinterpret_cast<void*>(256);
    char probeName[64] = {0};
    uint32_t probeSplits = 0;
    const bool usesPacked = vai_linear_plan(&probe, probeName, sizeof probeName, &probeSplits) == VAI_OK &&
                            std::strstr(probeName, "packed") != nullptr;
    const size_t pbytes = usesPacked ? vai_linear_packed_weight_size(&a) : 0;
    if (pbytes && (!packed_ || packedFrom_ != w.uploadId() || packedGated_ != (a.gated != 0))) {
        packed_ = bufferPool().requestBuffer(pbytes);
        vai_linear_args pa = a;
        pa.weight = w.devicePtr();
        check(vai_linear_pack_weight(&pa, packed_.ptr(), packed_.size(), (vai_stream_t)net().stream()), "Linear");
        check(vai_stream_sync((vai_stream_t)net().stream()), "Linear");
        packedFrom_ = w.uploadId();
        packedGated_ = a.gated != 0;
    }
    a.packed_weight = packedMatches(a) ? packed_.ptr() : nullptr;
    char name[64] = {0};
    check(vai_linear_plan(&a, name, sizeof name, &splitCount_), "Linear");
    plan_ = name;
    const size_t ws = vai_linear_workspace_size(&a);
    (*this)["partial"] = ws ? Tensor({uint32_t((ws + 3) / 4)}, Dtype::Fp32) : Tensor();
}

void Linear::run(CommandStream& cmd)
{
    vai_linear_args a = args(true);
    check(vai_linear_launch(&a, (vai_stream_t)cmd.stream()), "Linear");
}

// -------------------------------------------------------------- GatedMul ----

GatedMul::GatedMul() : GatedMul(Config()) {}

GatedMul::GatedMul(Config config) : config_(config)
{
    require(config_.activation < Epilogue::Max, "GatedMul: bad activation");
    addSlot("out0", NodeSlot::output);
    addSlot("in0", NodeSlot::input);
}

bool GatedMul::fusedInto() const
{
    const NodeSlot* in = findSlot("in0");
    if (!in || in->connections().empty()) return false;
    auto* lin = dynamic_cast<const Linear*>(&in->connections()[0]->parent());
    return lin && lin->fusedGate() == this;
}

void GatedMul::prepare()
{
    const Tensor& in = (*this)["in0"];
    require(in.validShape() && in.shape().back() % 2 == 0, "GatedMul: the last axis must be even");
    std::vector<uint32_t> shape = in.shape();
    shape.back() /= 2;
    (*this)["out0"] = Tensor(shape, outputDtype());
}

void GatedMul::run(CommandStream& cmd)
{
    if (fusedInto()) return;   // the producing Linear wrote out0 already
    const Tensor& in = (*this)["in0"];
    const Tensor& out = (*this)["out0"];
    const uint32_t H = out.shape().back();
    check(vai_gated_mul_launch(out.devicePtr(), code(out.dtype()), in.devicePtr(), code(in.dtype()),
                               outerSize(out.shape()), H, uint32_t(config_.activation), (vai_stream_t)cmd.stream()),
          "GatedMul");
}

// ----------------------------------------------------------- Convolution ----

Convolution::Convolution(Config config) : config_(config)
{
    require(config_.inChannels != 0 && config_.outChannels != 0, "Convolution: channel counts must be positive");
    require(config_.kernelSize != 0 && config_.kernelSize % 2 != 0, "Convolution: the kernel size must be odd");
    require(config_.stride != 0, "Convolution: stride must be positive");
    require(config_.epilogue < Epilogue::Max, "Convolution: bad epilogue");
    addSlot("out0", NodeSlot::output);
    addSlot("in0", NodeSlot::input);
    addSlot("weight", NodeSlot::persistent);
    addSlot("bias", NodeSlot::persistent);
    addSlot("scale", NodeSlot::persistent);
    if (config_.acceptResidual) addSlot("residual", NodeSlot::input);
    addSlot("split", NodeSlot::temporary);   // per-call weight pack when none is cached
}

vai_conv2d_args Convolution::args(bool withPointers) const
{
    vai_conv2d_args a{};
    const Tensor& in = (*this)["in0"];
    const Tensor& w = (*this)["weight"];
    a.batch = batch_;
    a.ci = config_.inChannels;
    a.hi = hi_;
    a.wi = wi_;
    a.co = config_.outChannels;
    a.kernel = config_.kernelSize;
    a.stride = config_.stride;
    a.i_dtype = code(in.dtype());
    a.w_dtype = code(w.dtype());
    a.o_dtype = code(outputDtype());
    a.epilogue = uint32_t(config_.epilogue);
    a.residual_order = uint32_t(config_.residualOrder);
    if (withPointers) {
        a.in = in.devicePtr();
        a.weight = w.devicePtr();
        a.out = (*this)["out0"].devicePtr();
        a.bias = hasBias() ? (*this)["bias"].devicePtr() : nullptr;
        a.scale = hasScale() ? (*this)["scale"].devicePtr() : nullptr;
        a.residual = config_.acceptResidual ? ptrOrNull((*this)["residual"]) : nullptr;
        a.packed_weight = packed_ ? packed_.ptr() : nullptr;
        const Tensor& ws = (*this)["split"];
        a.workspace = ptrOrNull(ws);
        a.workspace_bytes = ws.validShape() ? ws.numBytes() : 0;
    } else {
        a.in = a.weight = a.out = reinterpret_cast<void*>(256);
    }
    return a;
}

void Convolution::prepare()
{
    const Tensor& in = (*this)["in0"];
    const Tensor& w = (*this)["weight"];
    const auto& s = in.shape();
    require(s.size() >= 3, "Convolution: input must be [..., Ci, Hi, Wi]");
    require(s[s.size() - 3] == config_.inChannels, "Convolution: input channels differ from inChannels");
    const uint32_t k = config_.kernelSize;
    require(w.isShapeOf({config_.outChannels, config_.inChannels, k, k}), "Convolution: weight must be [Co, Ci, k, k]");
    require(w.gpuBufferBound(), "Convolution: weight was not uploaded");
    // convolution.h:4137-4160
    require(w.dtype() == Dtype::Fp16 || outputDtype() != Dtype::Fp16, "Convolution: fp16 output needs fp16 weights");
    require(w.dtype() == Dtype::Fp16 || in.dtype() != Dtype::Fp16, "Convolution: fp16 input needs fp16 weights");
    if (hasBias()) require((*this)["bias"].dtype() == w.dtype() && (*this)["bias"].isShapeOf({config_.outChannels}),
                           "Convolution: bias must be [Co] in the weight dtype");
    if (hasScale()) require((*this)["scale"].dtype() == w.dtype() && (*this)["scale"].isShapeOf({config_.outChannels}),
                            "Convolution: scale must be [Co] in the weight dtype");
    batch_ = outerSize(s, 3);
    hi_ = s[s.size() - 2];
    wi_ = s[s.size() - 1];
    const uint32_t ho = (hi_ - 1) / config_.stride + 1, wo = (wi_ - 1) / config_.stride + 1;
    std::vector<uint32_t> os(s.begin(), s.end() - 3);
    os.insert(os.end(), {config_.outChannels, ho, wo});
    (*this)["out0"] = Tensor(os, outputDtype());
    if (config_.acceptResidual) {
        const Tensor& r = (*this)["residual"];
        require(r.isShapeOf(os) && r.dtype() == in.dtype(), "Convolution: residual must match the output, input dtype");
    }
    // The weight is packed once, like the reference's one-shot transform
    // (convolution.h:6224-6235); a new weight upload repacks.
    vai_conv2d_args a = args(false);
    const size_t pbytes = vai_conv2d_packed_weight_size(&a);
    if (pbytes && (!packed_ || packedFrom_ != w.uploadId())) {
        packed_ = bufferPool().requestBuffer(pbytes);
        a.weight = w.devicePtr();
        check(vai_conv2d_pack_weight(&a, packed_.ptr(), packed_.size(), (vai_stream_t)net().stream()), "Convolution");
        check(vai_stream_sync((vai_stream_t)net().stream()), "Convolution");
        packedFrom_ = w.uploadId();
    }
    (*this)["split"] = Tensor();
}

void Convolution::run(CommandStream& cmd)
{
    vai_conv2d_args a = args(true);
    check(vai_conv2d_launch(&a, (vai_stream_t)cmd.stream()), "Convolution");
}

// ------------------------------------------------------- AttentionScores ----

AttentionScores::AttentionScores(Config config) : config_(config)
{
    if (config_.numKVHeads == 0) config_.numKVHeads = config_.numQHeads;
    require(config_.numQHeads > 0 && config_.headDim > 0, "AttentionScores: heads and headDim must be positive");
    require(config_.numQHeads % config_.numKVHeads == 0, "AttentionScores: numQHeads must be a multiple of numKVHeads");
    addSlot("out0", NodeSlot::output);
    addSlot("in0", NodeSlot::input);   // Q [..., Hq, Tq, D]
    addSlot("K", NodeSlot::input);     // K [..., Hkv, Tkv, D]
}

void AttentionScores::prepare()
{
    const Tensor& q = (*this)["in0"];
    const Tensor& k = (*this)["K"];
    const auto& qs = q.shape();
    const auto& ks = k.shape();
    require(qs.size() >= 3 && ks.size() == qs.size(), "AttentionScores: Q and K must be [..., H, T, D]");
    require(qs.back() == config_.headDim && ks.back() == config_.headDim, "AttentionScores: headDim mismatch");
    require(qs[qs.size() - 3] == config_.numQHeads && ks[ks.size() - 3] == config_.numKVHeads,
            "AttentionScores: head counts mismatch");
    require(q.dtype() == k.dtype(), "AttentionScores: Q and K must share a dtype");
    batch_ = outerSize(qs, 3);
    require(outerSize(ks, 3) == batch_, "AttentionScores: Q and K batch axes differ");
    tq_ = qs[qs.size() - 2];
    tkv_ = ks[ks.size() - 2];
    std::vector<uint32_t> os(qs.begin(), qs.end() - 1);
    os.push_back(tkv_);
    (*this)["out0"] = Tensor(os, Dtype::Fp32);
}

void AttentionScores::run(CommandStream& cmd)
{
    vai_attn_scores_args a{};
    a.scores = static_cast<float*>((*this)["out0"].devicePtr());
    a.q = (*this)["in0"].devicePtr();
    a.k = (*this)["K"].devicePtr();
    a.batch = batch_;
    a.hq = config_.numQHeads;
    a.hkv = config_.numKVHeads;
    a.tq = tq_;
    a.tkv = tkv_;
    a.head_dim = config_.headDim;
    a.dtype = code((*this)["in0"].dtype());
    a.scale = config_.scale != 0.0f ? config_.scale : 1.0f / std::sqrt(float(config_.headDim));
    apply_mask(a, config_.causal, config_.span, mask_);
    check(vai_attn_scores_launch(&a, (vai_stream_t)cmd.stream()), "AttentionScores");
}

void AttentionScores::setCausalMask(const CausalMask& mask)
{
    mask_ = mask;
    if (ownedNet_) ownedNet_->invalidateCommandBuffer();
}

// ------------------------------------------------------------- Attention ----

void Attention::setCausalMask(const CausalMask& mask)
{
    mask_ = mask;
    if (ownedNet_) ownedNet_->invalidateCommandBuffer();
}

void Attention::setKvCacheCounter(const uint32_t* counter)
{
    require(config_.kvCacheSize > 0, "Attention: a counter needs a KV cache (attention.h:244)");
    kvCacheCounter_ = counter;
    if (ownedNet_) ownedNet_->invalidateCommandBuffer();
}

Attention::Attention(Config config) : config_(config)
{
    if (config_.numKVHeads == 0) config_.numKVHeads = config_.numQHeads;
    require(config_.numQHeads > 0 && config_.headDim > 0, "Attention: heads and headDim must be positive");
    require(config_.numQHeads % config_.numKVHeads == 0, "Attention: numQHeads must be a multiple of numKVHeads");
    require(config_.kvCacheSize == 0 || config_.kvCacheDtype == Dtype::Fp16 || config_.kvCacheDtype == Dtype::Fp32,
            "Attention: a KV cache needs kvCacheDtype fp16 or fp32 (attention.h:959)");
    require(!config_.kvCacheRing || config_.kvCacheSize > 0, "Attention: a ring needs kvCacheSize (attention.h:960)");
    if (config_.kvCacheRing)
        config_.kvCacheSize = (config_.kvCacheSize + kvRingAlign - 1) / kvRingAlign * kvRingAlign;
    addSlot("out0", NodeSlot::output);
    addSlot("Q", NodeSlot::input);
    addSlot("K", NodeSlot::input);
    addSlot("V", NodeSlot::input);
    addSlot("partialO", NodeSlot::temporary);
    if (config_.kvCacheSize > 0) {
        addSlot("K_cache", NodeSlot::persistent);
        addSlot("V_cache", NodeSlot::persistent);
        (*this)["K_cache"] = Tensor({config_.numKVHeads, config_.kvCacheSize, config_.headDim}, config_.kvCacheDtype);
        (*this)["V_cache"] = Tensor({config_.numKVHeads, config_.kvCacheSize, config_.headDim}, config_.kvCacheDtype);
    }
}

vai_attention_args Attention::args(bool withBuffers) const
{
    vai_attention_args a{};
    const bool hasKv = tkv_ > 0;
    a.o_dtype = code(outputDtype());
    a.q_dtype = code((*this)["Q"].dtype());
    a.kv_dtype = hasKv ? code((*this)["K"].dtype()) : VAI_DTYPE_NONE;
    a.batch = batch_;
    a.hq = config_.numQHeads;
    a.hkv = config_.numKVHeads;
    a.tq = tq_;
    a.tkv = tkv_;
    a.head_dim = config_.headDim;
    a.scale = 0.0f;   // 1/sqrt(headDim), attention.h:1254
    apply_mask(a, false, 0, mask_);
    // the size query needs non-null, 16-byte aligned operands (as the pool's
    // buffers are); their values do not matter
    alignas(16) static char dummy[16];
    a.q = dummy;
    a.k = a.v = hasKv ? dummy : nullptr;
    a.out = dummy;
    if (config_.kvCacheSize > 0) {
        a.k_cache = a.v_cache = dummy;
        a.cache_count = reinterpret_cast<const uint32_t*>(dummy);
        a.cache_size = config_.kvCacheSize;
        a.cache_dtype = code(config_.kvCacheDtype);
        a.cache_ring = config_.kvCacheRing ? 1u : 0u;
    }
    if (withBuffers) {
        a.out = (*this)["out0"].devicePtr();
        a.q = (*this)["Q"].devicePtr();
        if (hasKv) {
            a.k = (*this)["K"].devicePtr();
            a.v = (*this)["V"].devicePtr();
        }
        if (config_.kvCacheSize > 0) {
            require(kvCacheCounter_ != nullptr, "Attention: a KV cache needs setKvCacheCounter");
            a.k_cache = (*this)["K_cache"].devicePtr();
            a.v_cache = (*this)["V_cache"].devicePtr();
            a.cache_count = kvCacheCounter_;
        }
        const Tensor& part = (*this)["partialO"];
        a.workspace = part.validShape() ? part.devicePtr() : nullptr;
        a.workspace_bytes = part.validShape() ? part.numBytes() : 0;
    }
    return a;
}

void Attention::prepare()
{
    const Tensor& q = (*this)["Q"];
    const Tensor& k = (*this)["K"];
    const Tensor& v = (*this)["V"];
    const auto& qs = q.shape();
    // without K / V (Tkv = 0) the keys are the cache's alone (attention.h:1001-1004)
    const bool hasKv = k.validShape();
    require(hasKv == v.validShape(), "Attention: K and V are wired together");
    require(hasKv || config_.kvCacheSize > 0, "Attention: K / V unwired without a KV cache");
    require(qs.size() >= 3 && qs.back() == config_.headDim && qs[qs.size() - 3] == config_.numQHeads,
            "Attention: Q must be [..., numQHeads, Tq, headDim]");
    require(q.dtype() != Dtype::None, "Attention: Q needs a dtype");
    batch_ = outerSize(qs, 3);
    tq_ = qs[qs.size() - 2];
    tkv_ = 0;
    if (hasKv) {
        const auto& ks = k.shape();
        require(ks.size() == qs.size() && v.shape() == ks, "Attention: Q, K, V must be [..., H, T, D]");
        require(ks.back() == config_.headDim && ks[ks.size() - 3] == config_.numKVHeads,
                "Attention: K / V head count or headDim mismatch");
        require(k.dtype() != Dtype::None && v.dtype() == k.dtype(), "Attention: K and V must share a dtype (attention.h:1014)");
        require(outerSize(ks, 3) == batch_, "Attention: Q and K batch axes differ");
        tkv_ = ks[ks.size() - 2];
    }
    // one counter per dispatch: one sequence with a cache (attention.h:1016)
    require(batch_ == 1 || config_.kvCacheSize == 0, "Attention: a KV cache serves one sequence");
    for (const char* name : {"K_cache", "V_cache"})
        if (config_.kvCacheSize > 0 && !(*this)[name].gpuBufferBound())
            (*this)[name].bindBuffer(bufferPool().requestBuffer((*this)[name].numBytes()));
    // token-major [..., Tq, Hq, Dh] (attention.h:1220-1223): leading axes as they came
    std::vector<uint32_t> os = qs;
    os[os.size() - 3] = tq_;
    os[os.size() - 2] = config_.numQHeads;
    (*this)["out0"] = Tensor(os, outputDtype());
    const vai_attention_args a = args(false);
    const size_t ws = vai_attention_workspace_size(&a);
    (*this)["partialO"] = ws ? Tensor({uint32_t((ws + 3) / 4)}, Dtype::Fp32) : Tensor();
}

void Attention::run(CommandStream& cmd)
{
    const vai_attention_args a = args(true);
    check(vai_attention_launch(&a, (vai_stream_t)cmd.stream()), "Attention");
}

}   // namespace vai::node
