// safetensors.h -- checkpoint ingest (the reference's vai/engine/
// safetensors-parser.h:15-56 and weights.h:38-70): a .safetensors file is an
// 8-byte little-endian header length, a JSON header mapping tensor names to
// {dtype, shape, data_offsets}, then the raw tensor bytes.
//
// The file is memory-mapped read-only once; a tensor's bytes are read from
// the mapping straight into the caller's buffer (or into a Tensor's host
// data, which the net uploads to HBM on first use), so the checkpoint is
// never held in memory a second time. Names, signatures and error behaviour
// (std::runtime_error, std::out_of_range for an unknown key) follow the
// reference.
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "tensor.h"

namespace vai {

class SafetensorsParser;

struct SafetensorRef
{
    const SafetensorsParser* parser;
    std::string key;

    std::vector<uint32_t> getShape() const;
    std::string getDataType() const;
    size_t byteSize() const;
    void readInto(void* dst) const;
    void readInto(void* dst, size_t byteOffset, size_t byteCount) const;
};

class SafetensorsParser
{
    struct Impl;
    std::unique_ptr<Impl> impl_;

public:
    explicit SafetensorsParser(const char* safetensorsFilePath);
    ~SafetensorsParser();
    SafetensorsParser(const SafetensorsParser&) = delete;
    SafetensorsParser& operator=(const SafetensorsParser&) = delete;

    std::vector<std::string> getTensorNames() const;   // in header order
    SafetensorRef operator[](std::string_view key) const { return {this, std::string(key)}; }
    std::vector<uint32_t> getShape(std::string_view key) const;
    std::string getDataType(std::string_view key) const;   // "F32", "F16", "BF16", ...
    size_t byteSize(std::string_view key) const;            // bytes as stored
    void readInto(std::string_view key, void* dst) const;
    void readInto(std::string_view key, void* dst, size_t byteOffset, size_t byteCount) const;
    // The stored bytes in place (valid while the parser lives).
    const void* data(std::string_view key) const;
};

inline std::vector<uint32_t> SafetensorRef::getShape() const { return parser->getShape(key); }
inline std::string SafetensorRef::getDataType() const { return parser->getDataType(key); }
inline size_t SafetensorRef::byteSize() const { return parser->byteSize(key); }
inline void SafetensorRef::readInto(void* dst) const { parser->readInto(key, dst); }
inline void SafetensorRef::readInto(void* dst, size_t byteOffset, size_t byteCount) const
{
    parser->readInto(key, dst, byteOffset, byteCount);
}

// Every *.safetensors file of a checkpoint folder, read by tensor name (a key
// is served by whichever shard holds it).
class Checkpoint
{
    std::vector<std::unique_ptr<SafetensorsParser>> shards_;
    std::unordered_map<std::string, const SafetensorsParser*> owner_;

public:
    explicit Checkpoint(const std::string& dir);
    bool contains(std::string_view key) const { return owner_.count(std::string(key)) != 0; }
    SafetensorRef operator[](std::string_view key) const;
    std::vector<std::string> getTensorNames() const;   // sorted
};

// A stored tensor as an engine Tensor of `dtype` (F32, F16 and BF16 sources;
// same-dtype data is copied as stored, the rest converts through fp32 with
// the engine's fp32 -> fp16 rounding). The net uploads it on first use.
Tensor loadTensor(const SafetensorRef& ref, Dtype dtype);

}   // namespace vai
