// safetensors_read.cpp -- checkpoint ingest from C++ (vai::Checkpoint,
// vai::loadTensor), host side only: no GPU is touched.
//
//   safetensors_read <checkpoint dir> <out dir> <f32|f16>
//
// For every tensor of the checkpoint (all shards) prints
// "tensor <name> <dtype> <d0>x<d1>... <bytes>", loads it as an engine Tensor
// of the requested dtype and writes its values as <out dir>/<name>.f32; then
// checks a partial read against the full one and prints "partial=ok", and
// prints "missing=<message>" for a key the checkpoint lacks.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "safetensors.h"

int main(int argc, char** argv)
{
    if (argc != 4) {
        std::fprintf(stderr, "usage: %s <checkpoint dir> <out dir> <f32|f16>\n", argv[0]);
        return 2;
    }
    const vai::Dtype dt = std::strcmp(argv[3], "f16") == 0 ? vai::Dtype::Fp16 : vai::Dtype::Fp32;
    try {
        vai::Checkpoint ck(argv[1]);
        const std::vector<std::string> names = ck.getTensorNames();
        for (const std::string& name : names) {
            const vai::SafetensorRef ref = ck[name];
            std::string shape;
            for (uint32_t d : ref.getShape()) shape += (shape.empty() ? "" : "x") + std::to_string(d);
            std::printf("tensor %s %s %s %zu\n", name.c_str(), ref.getDataType().c_str(),
                        shape.empty() ? "scalar" : shape.c_str(), ref.byteSize());
            vai::Tensor t = vai::loadTensor(ref, dt);
            const std::vector<float> v = t.toFloats();
            std::ofstream(std::string(argv[2]) + "/" + name + ".f32", std::ios::binary)
                .write(reinterpret_cast<const char*>(v.data()), v.size() * sizeof(float));
        }
        const vai::SafetensorRef first = ck[names.front()];
        const size_t n = first.byteSize(), half = n / 2;
        std::vector<unsigned char> all(n), tail(n - half);
        first.readInto(all.data());
        first.readInto(tail.data(), half, n - half);
        if (std::memcmp(all.data() + half, tail.data(), n - half) != 0) throw std::runtime_error("partial read differs");
        std::printf("partial=ok\n");
        try {
            first.readInto(tail.data(), half, n);   // runs past the end
            std::printf("overrun=accepted\n");
        } catch (const std::exception& e) {
            std::printf("overrun=refused\n");
        }
        try {
            (void)ck["no.such.tensor"];
            std::printf("missing=accepted\n");
        } catch (const std::exception& e) {
            std::printf("missing=%s\n", e.what());
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
