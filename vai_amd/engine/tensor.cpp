// tensor.cpp -- host conversions, layout helpers and host<->device copies of vai::Tensor.
#include "tensor.h"

#include <atomic>

#include <algorithm>
#include <bit>
#include <numeric>

#include "../../include/vai_amd.h"
#include "neural-net.h"

namespace vai {

// F16 -> F32, exact for every code (subnormal halves included).
static inline float halfToFloat(uint16_t h)
{
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {   // subnormal: value m * 2^-24, normalised by hand
            int shift = 0;
            uint32_t mm = m;
            while ((mm & 0x400u) == 0) { mm <<= 1; ++shift; }
            bits = sign | (uint32_t(127 - 15 - shift + 1) << 23) | ((mm & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    return std::bit_cast<float>(bits);
}

// F32 -> F16 with the reference host's rules (tensor.cpp:61-90): RNE, results
// below the smallest normal half flush to signed zero, overflow to inf.
static inline uint16_t floatToHalf(float f)
{
    const uint32_t b = std::bit_cast<uint32_t>(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t expRaw = (b >> 23) & 0xFFu, mant = b & 0x7FFFFFu;
    if (expRaw == 0xFFu) return uint16_t(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int32_t e = int32_t(expRaw) - 112;
    if (e <= 0) return uint16_t(sign);
    uint32_t m10 = mant >> 13;
    const uint32_t rest = mant & 0x1FFFu;
    m10 += (rest > 0x1000u) | ((rest == 0x1000u) & (m10 & 1u));
    uint32_t v = uint32_t(e) * 0x400u + m10;
    if (v >= 0x7C00u) v = 0x7C00u;
    return uint16_t(sign | v);
}

void convertDtype(const void* src, Dtype srcDtype, void* dst, Dtype dstDtype, size_t count)
{
    if (srcDtype == dstDtype) {
        std::memcpy(dst, src, count * bytesPerElement(srcDtype));
        return;
    }
    if (srcDtype == Dtype::Fp32 && dstDtype == Dtype::Fp16) {
        auto s = static_cast<const float*>(src);
        auto d = static_cast<uint16_t*>(dst);
        for (size_t i = 0; i < count; ++i) d[i] = floatToHalf(s[i]);
    } else if (srcDtype == Dtype::Fp16 && dstDtype == Dtype::Fp32) {
        auto s = static_cast<const uint16_t*>(src);
        auto d = static_cast<float*>(dst);
        for (size_t i = 0; i < count; ++i) d[i] = halfToFloat(s[i]);
    } else {
        throw std::runtime_error("convertDtype: unsupported dtype pair");
    }
}

void Tensor::bindBuffer(PooledBuffer buf, uint32_t baseOffset)
{
    require(data_ && baseOffset_ == 0, "bindBuffer: tensor has no data or is a view");
    data_->buffer_ = std::move(buf);
    baseOffset_ = baseOffset;
    require(!data_->buffer_ || byteOffset() + numBytes() <= data_->buffer_.size(), "bindBuffer: buffer too small");
}

Tensor& Tensor::setFloats(const std::vector<float>& inData)
{
    require(inData.size() == numElements(), "setFloats: element count mismatch");
    return setFloats(inData.data());
}

Tensor& Tensor::setFloats(const float* inData)
{
    require(validShape() && baseOffset_ == 0, "setFloats: invalid shape or a view");
    data_->lastSubmission_ = {nullptr, 0};
    data_->hostUploaded_ = false;
    data_->hostData_.resize(numBytes());
    convertDtype(inData, Dtype::Fp32, data_->hostData_.data(), dtype(), numElements());
    return *this;
}

Tensor Tensor::reshape(const std::vector<uint32_t>& dims) const
{
    require(data_ != nullptr, "reshape: empty tensor");
    size_t n = 1;
    for (auto d : dims) n *= d;
    require(n == numElements(), "reshape: element count mismatch");
    Tensor out = *this;
    out.shape_ = dims;
    return out;
}

Tensor Tensor::view(const std::vector<uint32_t>& dims, uint32_t baseOffset) const
{
    require(data_ != nullptr, "view: empty tensor");
    Tensor out = *this;
    out.shape_ = dims;
    out.baseOffset_ = baseOffset;
    require(!data_->buffer_ || out.byteOffset() + out.numBytes() <= data_->buffer_.size(), "view: out of range");
    return out;
}

bool Tensor::isShapeOf(const std::vector<uint32_t>& dims) const
{
    if (!data_ || shape_.size() != dims.size()) return false;
    for (size_t i = 0; i < dims.size(); ++i)
        if (dims[i] != uint32_t(-1) && dims[i] != shape_[i]) return false;
    return true;
}

Tensor Tensor::permute(const std::vector<uint32_t>& perm) const
{
    require(hasHostData(), "permute: needs host data");
    const size_t rank = shape_.size();
    require(perm.size() == rank, "permute: rank mismatch");
    std::vector<uint32_t> dst(rank);
    for (size_t i = 0; i < rank; ++i) {
        require(perm[i] < rank, "permute: bad axis");
        dst[i] = shape_[perm[i]];
    }
    std::vector<size_t> ss(rank, 1), ds(rank, 1);
    for (int i = int(rank) - 2; i >= 0; --i) {
        ss[i] = ss[i + 1] * shape_[i + 1];
        ds[i] = ds[i + 1] * dst[i + 1];
    }
    const size_t n = numElements(), es = bytesPerElement(dtype());
    HostBuffer out(n * es);
    std::vector<uint32_t> idx(rank);
    for (size_t lin = 0; lin < n; ++lin) {
        size_t rem = lin, dl = 0;
        for (size_t i = 0; i < rank; ++i) { idx[i] = uint32_t(rem / ss[i]); rem %= ss[i]; }
        for (size_t i = 0; i < rank; ++i) dl += size_t(idx[perm[i]]) * ds[i];
        std::memcpy(&out[dl * es], &data_->hostData_[lin * es], es);
    }
    Tensor t(dst, dtype());
    t.data_->hostData_ = std::move(out);
    return t;
}

std::vector<Tensor> Tensor::split(const std::vector<uint32_t>& offsets) const
{
    require(hasHostData() && !shape_.empty(), "split: needs host data");
    std::vector<uint32_t> bounds = offsets;
    bounds.push_back(shape_[0]);
    const size_t stride = numElements() / shape_[0] * bytesPerElement(dtype());
    std::vector<Tensor> parts;
    uint32_t begin = 0;
    for (uint32_t end : bounds) {
        require(begin < end && end <= shape_[0], "split: offsets must ascend inside the leading axis");
        std::vector<uint32_t> sh = shape_;
        sh[0] = end - begin;
        Tensor t(sh, dtype());
        t.data_->hostData_.assign(data_->hostData_.begin() + begin * stride, data_->hostData_.begin() + end * stride);
        parts.push_back(std::move(t));
        begin = end;
    }
    return parts;
}

Tensor Tensor::concat(const std::vector<Tensor>& others) const
{
    require(hasHostData() && !shape_.empty(), "concat: needs host data");
    std::vector<uint32_t> sh = shape_;
    HostBuffer out(data_->hostData_);
    for (const Tensor& o : others) {
        require(o.hasHostData() && o.dtype() == dtype() && o.shape_.size() == shape_.size(), "concat: mismatch");
        for (size_t d = 1; d < shape_.size(); ++d) require(o.shape_[d] == shape_[d], "concat: trailing dims differ");
        sh[0] += o.shape_[0];
        out.insert(out.end(), o.data_->hostData_.begin(), o.data_->hostData_.end());
    }
    Tensor t(sh, dtype());
    t.data_->hostData_ = std::move(out);
    return t;
}

void* Tensor::devicePtr() const
{
    require(gpuBufferBound(), "devicePtr: no device buffer bound");
    return static_cast<char*>(data_->buffer_.ptr()) + byteOffset();
}

void Tensor::upload(void* stream)
{
    require(hasHostData() && gpuBufferBound(), "upload: needs host data and a device buffer");
    const vai_status st = vai_memcpy_h2d(devicePtr(), data_->hostData_.data(), numBytes(), (vai_stream_t)stream);
    require(st == VAI_OK, std::string("upload: ") + vai_status_string(st));
    data_->hostUploaded_ = true;
    static std::atomic<uint64_t> uploads{0};
    data_->uploadId_ = ++uploads;
}

Tensor& Tensor::downloadToHost()
{
    require(data_ != nullptr, "downloadToHost: empty tensor");
    if (!gpuBufferBound()) {
        require(hasHostData(), "downloadToHost: tensor has neither host nor device data");
        return *this;
    }
    if (data_->lastSubmission_.first) data_->lastSubmission_.first->sync();
    data_->hostData_.resize(numBytes());
    const vai_status st = vai_memcpy_d2h(data_->hostData_.data(), devicePtr(), numBytes(), nullptr);
    require(st == VAI_OK, std::string("downloadToHost: ") + vai_status_string(st));
    return *this;
}

std::vector<float> Tensor::toFloats()
{
    downloadToHost();
    std::vector<float> out(numElements());
    convertDtype(data_->hostData_.data(), dtype(), out.data(), Dtype::Fp32, numElements());
    return out;
}

}   // namespace vai
