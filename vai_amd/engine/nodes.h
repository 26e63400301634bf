// nodes.h -- the matmul-path nodes of the reference, on the MI355X kernels.
//   Linear        /root/reference/vai/nodes/linear.h:59-348
//   GatedMul      /root/reference/vai/nodes/gated-mul.h:21-44
//   Convolution   /root/reference/vai/nodes/convolution.h:2453-2609
//   AttentionScores  the S = scale * Q.K^T (+ causal mask) stage of
//                 /root/reference/vai/nodes/attention.h:144-280, as a node of
//                 its own (the reference fuses it into flash attention).
// Configs keep the reference's field names and defaults; prepare() validates
// and picks the kernel through the C ABI, run() launches on the net's stream.
#pragma once
#include <array>
#include <cstdint>

#include "../../include/vai_amd.h"
#include "graph-flow.h"
#include "neural-net.h"

namespace vai {

// /root/reference/vai/nodes/common.h:31-45.
enum class Epilogue : uint32_t { None, Relu, Gelu, GeluTanh, Silu, Sigmoid, Max };
enum class ResidualOrder : uint32_t { AfterEpilogue = 0, BeforeEpilogue = 1 };

// The product of the axes ahead of the last innerAxes (common.h:67-73).
inline uint32_t outerSize(const std::vector<uint32_t>& shape, size_t innerAxes = 1)
{
    uint32_t n = 1;
    for (size_t i = 0; i + innerAxes < shape.size(); ++i) n *= shape[i];
    return n;
}

namespace node {

class GatedMul;

class Linear : public Node
{
public:
    struct Config {
        uint32_t inDim;
        uint32_t outDim;
        bool acceptResidual = false;
        ResidualOrder residualOrder = ResidualOrder::AfterEpilogue;
        Epilogue epilogue = Epilogue::None;
        float scalarScale = 1.0f;
        uint32_t splitSize = 0;   // split-K span; 0 lets the library choose per shape
    } config_;

    explicit Linear(Config config);
    void prepare() override;
    void run(CommandStream& cmd) override;
    const char* kind() const override { return "Linear"; }

    bool hasBias() const { return (*this)["bias"].validShape(); }
    // Accumulator dtype (linear.h:289,2320). None and Fp32 accumulate in fp32,
    // the reference's AMD default; Fp16 sums in fp16 in the reference tile
    // kernel's order wherever that kernel would (M > 8, an fp16 operand).
    // A change after the first forward takes effect at the next one (re-record).
    void setAccDtype(Dtype dtype, DtypeKey)
    {
        if (dtype != accDtype_ && ownedNet_) ownedNet_->invalidateCommandBuffer();
        accDtype_ = dtype;
    }
    Dtype accDtype() const { return accDtype_; }

    // The kernel prepare() chose ("slab", "tile_f16_256x256_gated", ...) and its split count.
    const std::string& plan() const { return plan_; }
    uint32_t splitCount() const { return splitCount_; }

    // Record-time fusion with a following GatedMul (see NeuralNet::bindFusion).
    bool canFuseGate(const GatedMul& gm) const;
    void setFusedGate(GatedMul* gm) { fused_ = gm; }
    GatedMul* fusedGate() const { return fused_; }

private:
    Dtype accDtype_ = Dtype::None;
    GatedMul* fused_ = nullptr;
    PooledBuffer packed_;              // fragment-major copy of the weight for prefill shapes
    uint64_t packedFrom_ = 0;          // uploadId() of the weight it was made from
    bool packedGated_ = false;
    uint32_t M_ = 0, biasRepeat_ = 0, residualRepeat_ = 0;
    std::string plan_;
    uint32_t splitCount_ = 1;
    vai_linear_args args(bool withPointers) const;
    bool packedMatches(const vai_linear_args& a) const;
};

class GatedMul : public Node
{
    friend class Linear;

public:
    struct Config {
        Epilogue activation = Epilogue::Silu;
    } config_;

    GatedMul();
    explicit GatedMul(Config config);
    void prepare() override;
    void run(CommandStream& cmd) override;
    const char* kind() const override { return "GatedMul"; }

private:
    bool fusedInto() const;
};

class Convolution : public Node
{
public:
    struct Config {
        uint32_t inChannels;
        uint32_t outChannels;
        uint32_t kernelSize;
        uint32_t stride;
        bool acceptResidual = false;
        ResidualOrder residualOrder = ResidualOrder::AfterEpilogue;
        Epilogue epilogue = Epilogue::None;
    } config_;

    explicit Convolution(Config config);
    void prepare() override;
    void run(CommandStream& cmd) override;
    const char* kind() const override { return "Convolution"; }

    bool hasBias() const { return (*this)["bias"].validShape(); }
    bool hasScale() const { return (*this)["scale"].validShape(); }

private:
    vai_conv2d_args args(bool withPointers) const;
    PooledBuffer packed_;          // weight packed once for the fp16 kernel
    uint64_t packedFrom_ = 0;      // uploadId() of the weight it was made from
    uint32_t batch_ = 1, hi_ = 0, wi_ = 0;
};

// A block mask as the reference's writeCausalMask sets it (/root/reference/
// vai/nodes/attention.h:40-55): blockEnd lists every block end but the last
// (query rows, increasing, the list stops at its first 0), bit (count - 1 - k)
// of bits marks block k causal, span > 0 is a sliding window.
using CausalBlockEnd = std::array<uint32_t, VAI_MAX_CAUSAL_BLOCKS - 1>;
struct CausalMask {
    uint32_t blockCount = 0;   // 0: none (AttentionScores: its causal flag; Attention: no mask)
    uint32_t bits = 0;
    CausalBlockEnd blockEnd{};
    uint32_t span = 0;
    static CausalMask make(uint32_t bits, const CausalBlockEnd& blockEnd = {}, uint32_t span = 0)
    {
        CausalMask m{1, bits, blockEnd, span};
        while (m.blockCount < VAI_MAX_CAUSAL_BLOCKS && blockEnd[m.blockCount - 1] != 0) ++m.blockCount;
        return m;
    }
};

class AttentionScores : public Node
{
public:
    struct Config {
        uint32_t numQHeads;
        uint32_t numKVHeads = 0;   // 0: numQHeads (no GQA)
        uint32_t headDim;
        bool causal = true;
        uint32_t span = 0;         // sliding window; 0: none
        float scale = 0.0f;        // 0: 1/sqrt(headDim), as attention.h:1254
    } config_;

    explicit AttentionScores(Config config);
    void prepare() override;
    void run(CommandStream& cmd) override;
    const char* kind() const override { return "AttentionScores"; }
    // Replaces causal/span with the block mask; the next forward re-records.
    void setCausalMask(const CausalMask& mask);

private:
    uint32_t batch_ = 1, tq_ = 0, tkv_ = 0;
    CausalMask mask_;
};

// The reference's Attention node (/root/reference/vai/nodes/attention.h:
// 77-140, 216-245, 959-1304): out0 = softmax(Q K^T / sqrt(headDim) + mask) V
// per head. Q [..., numQHeads, Tq, headDim] fp32 or fp16, K / V [...,
// numKVHeads, Tkv, headDim] in their own dtype (fp32 or fp16), out0
// token-major [..., Tq, numQHeads, headDim] in the node's output dtype.
// Queries and keys align at their ends. No mask until setCausalMask is
// called: every query attends every key. Any head dim.
// kvCacheSize > 0 adds the KV cache: the persistent slots "K_cache" /
// "V_cache" [numKVHeads, kvCacheSize, headDim] in kvCacheDtype (a ring rounds
// its size up to kvRingAlign) and a counter the model owns and rewrites
// before each forward (setKvCacheCounter: a device-readable uint32, read when
// the kernels run, so a recorded forward follows it). Each forward appends
// its Tkv new K / V rows after the cached ones and attends both; K / V may
// stay unwired (Tkv = 0) to attend the cache alone. One sequence only.
// "partialO" holds the workspace (fp16 K / V copies, key-split partials)
// when a launch needs one.
class Attention : public Node
{
public:
    struct Config {
        uint32_t headDim;
        uint32_t numQHeads;
        uint32_t numKVHeads = 0;              // for GQA (Hkv < numQHeads); 0: numQHeads
        uint32_t kvCacheSize = 0;             // tokens the cache holds; 0: no cache at all
        Dtype kvCacheDtype = Dtype::None;     // required with a cache
        bool kvCacheRing = false;             // keep the last kvCacheSize positions (rounded up to kvRingAlign)
    } config_;
    static constexpr uint32_t kvRingAlign = 256;

    explicit Attention(Config config);
    void prepare() override;
    void run(CommandStream& cmd) override;
    const char* kind() const override { return "Attention"; }
    // The reference's setCausalMask role (a CausalMask made as
    // writeCausalMask makes it; CausalMask::make(1) is plain causal). The
    // reference rewrites a uniform buffer without re-recording; here the mask
    // is part of the recorded launch, so the next forward re-records.
    void setCausalMask(const CausalMask& mask);
    // The positions the cache holds (attention.h:242-246): a device-readable
    // uint32 the model writes before each forward; the node never writes it.
    void setKvCacheCounter(const uint32_t* counter);

private:
    vai_attention_args args(bool withBuffers) const;
    const uint32_t* kvCacheCounter_ = nullptr;
    uint32_t batch_ = 1, tq_ = 0, tkv_ = 0;
    CausalMask mask_;
};

}   // namespace node
}   // namespace vai
