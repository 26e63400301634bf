// gated_ffn_block.cpp -- the full gated MLP block, as a model net uses it:
// a NeuralNet holding vai::group::GatedFeedForward, wired with the flow DSL.
//
//   gated_ffn_block <dir> <M> <K> <H> <N> <residual 0|1> <act silu|gelu_tanh> <odt f32|f16> [checkpoint dir]
//
// reads <dir>/x.f32 [M,K], <dir>/w1.f32 [2H,K] (gate rows, then value rows),
// <dir>/w2.f32 [N,H], and with residual <dir>/r.f32 [M,N]. With a checkpoint
// folder the weights come from its .safetensors shards instead, under the
// Llama names mlp.gate_proj.weight [H,K], mlp.up_proj.weight [H,K] and
// mlp.down_proj.weight [N,H], the gate/value weight being concat(gate, up)
// as the reference's meta-weights.h:53-57 builds it. Weights are fp16
// (the net default); x, the residual and the activations between the nodes
// use <odt> (the net's output default). Runs the block twice (record, then replay), writes
// <dir>/y.f32 [M,N] and prints the two Linear plans and the record/submit
// counts.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "graph-flow.h"
#include "groups.h"
#include "nodes.h"
#include "safetensors.h"

namespace {

std::vector<float> readFloats(const std::string& path, size_t count)
{
    std::vector<float> v(count);
    std::ifstream f(path, std::ios::binary);
    if (!f.read(reinterpret_cast<char*>(v.data()), count * sizeof(float)))
        throw std::runtime_error("cannot read " + std::to_string(count) + " floats from " + path);
    return v;
}

vai::NeuralNetConfig netConfig(vai::Dtype odt)
{
    vai::NeuralNetConfig c{};
    c.oDefaultDtype = odt;
    return c;
}

struct Block : vai::NeuralNet
{
    vai::group::GatedFeedForward ffn;
    Block(uint32_t K, uint32_t H, uint32_t N, bool residual, vai::Epilogue act, vai::Dtype odt)
    : vai::NeuralNet(netConfig(odt)),
      ffn(vai::group::GatedFeedForward::Config{
          .inDim = K, .hiddenDim = H, .outDim = N, .activation = act, .acceptResidual = residual})
    {
        input("x") - ffn - output("y");
        if (residual) input("r") - ("residual" / ffn);
    }
};

}   // namespace

int main(int argc, char** argv)
{
    if (argc != 9 && argc != 10) {
        std::fprintf(stderr, "usage: %s <dir> <M> <K> <H> <N> <residual> <silu|gelu_tanh> <f32|f16> [ckpt]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const uint32_t M = std::atoi(argv[2]), K = std::atoi(argv[3]), H = std::atoi(argv[4]), N = std::atoi(argv[5]);
    const bool residual = std::atoi(argv[6]) != 0;
    const vai::Epilogue act = std::strcmp(argv[7], "silu") == 0 ? vai::Epilogue::Silu : vai::Epilogue::GeluTanh;
    const vai::Dtype odt = std::strcmp(argv[8], "f16") == 0 ? vai::Dtype::Fp16 : vai::Dtype::Fp32;
    try {
        Block net(K, H, N, residual, act, odt);
        if (argc == 10) {
            const vai::Checkpoint ck(argv[9]);
            const vai::Tensor gate = vai::loadTensor(ck["mlp.gate_proj.weight"], vai::Dtype::Fp16);
            const vai::Tensor up = vai::loadTensor(ck["mlp.up_proj.weight"], vai::Dtype::Fp16);
            if (!gate.isShapeOf({H, K}) || !up.isShapeOf({H, K})) throw std::runtime_error("gate/up shape");
            net.ffn.gateValue["weight"] = gate.concat({up});
            net.ffn.out["weight"] = vai::loadTensor(ck["mlp.down_proj.weight"], vai::Dtype::Fp16);
            if (!net.ffn.out["weight"].isShapeOf({N, H})) throw std::runtime_error("down shape");
        } else {
            net.ffn.gateValue["weight"] = vai::Tensor({2 * H, K}, vai::Dtype::Fp16);
            net.ffn.gateValue["weight"].setFloats(readFloats(dir + "/w1.f32", size_t(2) * H * K));
            net.ffn.out["weight"] = vai::Tensor({N, H}, vai::Dtype::Fp16);
            net.ffn.out["weight"].setFloats(readFloats(dir + "/w2.f32", size_t(N) * H));
        }

        vai::Tensor x({M, K}, odt);
        x.setFloats(readFloats(dir + "/x.f32", size_t(M) * K));
        vai::Tensor r;
        if (residual) {
            r = vai::Tensor({M, N}, odt);
            r.setFloats(readFloats(dir + "/r.f32", size_t(M) * N));
        }
        vai::Tensor y;
        for (int i = 0; i < 2; ++i) {
            if (residual) net({{"x", x}, {"r", r}}, {{"y", &y}});
            else net({{"x", x}}, {{"y", &y}});
        }
        net.sync();

        std::vector<float> out = y.toFloats();
        if (out.size() != size_t(M) * N) throw std::runtime_error("output has the wrong size");
        std::ofstream(dir + "/y.f32", std::ios::binary)
            .write(reinterpret_cast<const char*>(out.data()), out.size() * sizeof(float));
        std::printf("plan1=%s plan2=%s fused=%d records=%llu submits=%llu\n", net.ffn.gateValue.plan().c_str(),
                    net.ffn.out.plan().c_str(), net.ffn.gateValue.fusedGate() != nullptr,
                    (unsigned long long)net.recordCount(), (unsigned long long)net.submitCount());
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
