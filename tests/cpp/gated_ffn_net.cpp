// gated_ffn_net.cpp -- a C++ user of the engine, written the way a vAi model
// net is (/root/reference/vai/nodes/gated-feed-forward.h:23-54 composes
// `gateValue - gatedMul`): a NeuralNet subclass owns its nodes as members and
// wires them with the flow DSL in its constructor.
//
//   gated_ffn_net <dir> <M> <K> <H>
//
// reads <dir>/x.f32 [M,K], <dir>/w.f32 [2H,K] (gate rows, then up rows),
// <dir>/b.f32 [2H]; runs input("x") - Linear(K -> 2H, bias) - GatedMul(SiLU)
// - output("y") with fp16 weights (the net default) twice, the second forward
// being a replay of the recorded graph; writes <dir>/y.f32 [M,H] and prints
// the plan Linear chose and how often the net recorded and submitted.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "graph-flow.h"
#include "nodes.h"

namespace {

std::vector<float> readFloats(const std::string& path, size_t count)
{
    std::vector<float> v(count);
    std::ifstream f(path, std::ios::binary);
    if (!f.read(reinterpret_cast<char*>(v.data()), count * sizeof(float)))
        throw std::runtime_error("cannot read " + std::to_string(count) + " floats from " + path);
    return v;
}

struct GatedFfn : vai::NeuralNet
{
    vai::node::Linear gateValue;
    vai::node::GatedMul gatedMul;

    GatedFfn(uint32_t K, uint32_t H)
    : vai::NeuralNet(vai::NeuralNetConfig{}),
      gateValue(vai::node::Linear::Config{.inDim = K, .outDim = 2 * H}),
      gatedMul(vai::node::GatedMul::Config{.activation = vai::Epilogue::Silu})
    {
        input("x") - gateValue - gatedMul - output("y");
    }
};

}   // namespace

int main(int argc, char** argv)
{
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <dir> <M> <K> <H>\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const uint32_t M = std::atoi(argv[2]), K = std::atoi(argv[3]), H = std::atoi(argv[4]);
    try {
        GatedFfn net(K, H);
        net.gateValue["weight"] = vai::Tensor({2 * H, K}, vai::Dtype::Fp16);
        net.gateValue["weight"].setFloats(readFloats(dir + "/w.f32", size_t(2) * H * K));
        net.gateValue["bias"] = vai::Tensor({2 * H}, vai::Dtype::Fp16);
        net.gateValue["bias"].setFloats(readFloats(dir + "/b.f32", size_t(2) * H));

        vai::Tensor x({M, K}, vai::Dtype::Fp32);
        x.setFloats(readFloats(dir + "/x.f32", size_t(M) * K));
        vai::Tensor y;
        for (int i = 0; i < 2; ++i) net({{"x", x}}, {{"y", &y}});
        net.sync();

        std::vector<float> out = y.toFloats();
        if (out.size() != size_t(M) * H) throw std::runtime_error("output has the wrong size");
        std::ofstream(dir + "/y.f32", std::ios::binary)
            .write(reinterpret_cast<const char*>(out.data()), out.size() * sizeof(float));
        std::printf("plan=%s fused=%d records=%llu submits=%llu\n", net.gateValue.plan().c_str(),
                    net.gateValue.fusedGate() != nullptr, (unsigned long long)net.recordCount(),
                    (unsigned long long)net.submitCount());
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
