// groups.h -- node groups: subgraphs that wire like one node (the reference's
// vai/groups/). A group owns its member nodes, connects them in its
// constructor, and republishes the slots a caller wires to.
#pragma once
#include <cstdint>

#include "graph-flow.h"
#include "nodes.h"

namespace vai::group {

// The gated MLP of /root/reference/vai/groups/gated-feed-forward.h:23-54:
//   out0 = out(activation(gate(in0)) * value(in0)) (+ residual)
// One projection produces gate and value ([..., 2 * hiddenDim] over the
// weights concat(gate rows, value rows)); GatedMul applies the GLU (SiLU:
// SwiGLU, GELU: GEGLU); the output projection folds the block's skip add in
// when acceptResidual opens the "residual" slot. Config field names and
// defaults are the reference's. In this engine the gateValue -> gatedMul pair
// records as one fused GEMM when the net's fuseGatedLinear is on.
struct GatedFeedForward : public vai::NodeGroup
{
    vai::node::Linear gateValue;   // [..., inDim] -> [..., 2 * hiddenDim]
    vai::node::GatedMul gatedMul;  // [..., 2 * hiddenDim] -> [..., hiddenDim]
    vai::node::Linear out;         // [..., hiddenDim] -> [..., outDim]

    struct Config {
        uint32_t inDim;
        uint32_t hiddenDim;
        uint32_t outDim;
        vai::Epilogue activation = vai::Epilogue::Silu;
        bool acceptResidual = false;
    };

    explicit GatedFeedForward(Config config)
    : gateValue(vai::node::Linear::Config{.inDim = config.inDim, .outDim = 2 * config.hiddenDim}),
      gatedMul(vai::node::GatedMul::Config{.activation = config.activation}),
      out(vai::node::Linear::Config{
          .inDim = config.hiddenDim, .outDim = config.outDim, .acceptResidual = config.acceptResidual})
    {
        gateValue - gatedMul - out;
        defineSlot("in0", gateValue.slot("in0"));
        if (config.acceptResidual) defineSlot("residual", out.slot("residual"));
        defineSlot("out0", out.slot("out0"));
    }
};

}   // namespace vai::group
