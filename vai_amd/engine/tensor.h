// tensor.h -- vai::Tensor for the MI355X build: the reference's handle
// (/root/reference/vai/engine/tensor.h:19-332) with device storage in
// hipMalloc'd buffers from a size-bucketed pool instead of Vulkan buffers.
#pragma once
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <array>
#include <utility>
#include <vector>

#include "buffer-pool.h"
#include "error.h"

namespace vai {

class NeuralNet;

// /root/reference/vai/engine/tensor.h:19
enum class Dtype { Fp32, Fp16, None };

constexpr size_t bytesPerElement(Dtype dt) noexcept
{
    switch (dt) {
    case Dtype::Fp16: return 2;
    case Dtype::Fp32: return 4;
    case Dtype::None: return 0;
    }
    return 4;
}

// Host conversion of `count` elements, fp32 <-> fp16, as the reference does it
// (tensor.cpp:42-90): round-to-nearest-even, results below the smallest
// normal half flush to zero, overflow saturates to inf, NaN stays NaN.
void convertDtype(const void* src, Dtype srcDtype, void* dst, Dtype dstDtype, size_t count);

using HostBuffer = std::vector<char>;

class TensorData
{
    friend class Tensor;
    friend class NeuralNet;

    HostBuffer hostData_;
    bool hostUploaded_ = false;     // hostData_ is already on the device; a setter clears it
    uint64_t uploadId_ = 0;         // distinct per upload: identifies the device contents
    const Dtype dtype_;
    PooledBuffer buffer_;
    std::pair<NeuralNet*, uint64_t> lastSubmission_{nullptr, 0};

public:
    explicit TensorData(Dtype dt = Dtype::Fp32) : dtype_(dt) { VAI_ASSERT(dt != Dtype::None); }
};

class Tensor
{
    friend class NeuralNet;

    std::shared_ptr<TensorData> data_;
    std::vector<uint32_t> shape_;
    uint32_t baseOffset_ = 0;   // in elements; != 0 means a view

public:
    Tensor(const std::vector<uint32_t>& shape, Dtype dtype = Dtype::Fp32)
    : data_(std::make_shared<TensorData>(dtype)), shape_(shape) {}
    Tensor() = default;

    // Bind device storage (the engine does this for outputs and temporaries).
    void bindBuffer(PooledBuffer buf, uint32_t baseOffset = 0);

    // Ingest float data, converting fp32 -> this tensor's dtype.
    Tensor& setFloats(const std::vector<float>& inData);
    Tensor& setFloats(const float* inData);

    // Raw typed write, no conversion; sizeof(T) must be the element size.
    template <typename T>
    Tensor& setData(const T* src)
    {
        VAI_ASSERT(validShape() && baseOffset_ == 0);
        VAI_ASSERT(sizeof(T) == bytesPerElement(data_->dtype_) && "setData<T>: sizeof(T) != element size");
        data_->lastSubmission_ = {nullptr, 0};
        data_->hostUploaded_ = false;
        data_->hostData_.resize(numBytes());
        std::memcpy(data_->hostData_.data(), src, numBytes());
        return *this;
    }

    // The same data seen as `dims` (shares the data).
    Tensor reshape(const std::vector<uint32_t>& dims) const;
    // Reinterpret the bound buffer as `dims` from element `baseOffset` (shares the buffer).
    Tensor view(const std::vector<uint32_t>& dims, uint32_t baseOffset) const;

    // Host-side layout helpers (tensor.h:202-237): the result owns its bytes.
    Tensor permute(const std::vector<uint32_t>& perm) const;
    std::vector<Tensor> split(const std::vector<uint32_t>& offsets) const;
    Tensor concat(const std::vector<Tensor>& others) const;

    uint64_t byteOffset() const { return uint64_t(baseOffset_) * bytesPerElement(dtype()); }
    const std::vector<uint32_t>& shape() const
    {
        static const std::vector<uint32_t> empty{};
        return data_ ? shape_ : empty;
    }
    bool isShapeOf(const std::vector<uint32_t>& dims) const;   // uint32_t(-1) matches any
    Dtype dtype() const { return data_ ? data_->dtype_ : Dtype::None; }
    size_t numElements() const
    {
        if (!data_ || shape_.empty()) return 0;
        size_t n = 1;
        for (uint32_t d : shape_) n *= d;
        return n;
    }
    size_t numBytes() const { return numElements() * bytesPerElement(dtype()); }
    bool validShape() const
    {
        if (!data_ || shape_.empty()) return false;
        for (uint32_t d : shape_) if (d == 0) return false;
        return true;
    }
    bool hasHostData() const { return data_ && !data_->hostData_.empty(); }
    const void* hostData() const { return hasHostData() ? data_->hostData_.data() : nullptr; }
    bool gpuBufferBound() const { return data_ && data_->buffer_; }
    // Changes on every upload of host data (device pointers can repeat when
    // the pool hands a released buffer out again).
    uint64_t uploadId() const { return data_ ? data_->uploadId_ : 0; }
    uint32_t baseOffset() const { return baseOffset_; }
    // Device address of element 0 of this tensor (the Vulkan BufferRange's role).
    void* devicePtr() const;
    std::pair<NeuralNet*, uint64_t> lastSubmission() const
    {
        return data_ ? data_->lastSubmission_ : std::pair<NeuralNet*, uint64_t>{nullptr, 0};
    }
    bool sameData(const Tensor& o) const { return data_ == o.data_; }

    // Device -> host copy (waits for the net that last wrote it), then a typed pointer.
    Tensor& downloadToHost();
    template <typename T = float>
    const T* getData()
    {
        return reinterpret_cast<const T*>(downloadToHost().data_->hostData_.data());
    }
    // The host copy as fp32, whatever the dtype.
    std::vector<float> toFloats();

    // Host -> device copy into the bound buffer (synchronous).
    void upload(void* stream);
};

}   // namespace vai
