// buffer-pool.h -- size-bucketed reuse of hipMalloc'd device buffers: the
// reference's BufferPool / PooledBuffer (/root/reference/vai/engine/
// buffer-pool.h:20-153) with HBM allocations in place of Vulkan buffers.
// Requests round up to a power of two (>= 256 B) so buffers recycle across
// shapes; a PooledBuffer is move-only and returns its buffer on release.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace vai {

class BufferPool;

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t size = 0;          // capacity in bytes
};

class PooledBuffer
{
    std::shared_ptr<BufferPool> pool_;
    DeviceBuffer buf_;

public:
    PooledBuffer() = default;
    PooledBuffer(std::shared_ptr<BufferPool> pool, DeviceBuffer buf) : pool_(std::move(pool)), buf_(buf) {}
    PooledBuffer(const PooledBuffer&) = delete;
    PooledBuffer& operator=(const PooledBuffer&) = delete;
    PooledBuffer(PooledBuffer&& o) noexcept : pool_(std::move(o.pool_)), buf_(o.buf_) { o.buf_ = {}; }
    PooledBuffer& operator=(PooledBuffer&& o) noexcept
    {
        if (this != &o) {
            release();
            pool_ = std::move(o.pool_);
            buf_ = o.buf_;
            o.buf_ = {};
        }
        return *this;
    }
    ~PooledBuffer() { release(); }

    void release();
    explicit operator bool() const { return buf_.ptr != nullptr; }
    void* ptr() const { return buf_.ptr; }
    size_t size() const { return buf_.size; }
};

class BufferPool : public std::enable_shared_from_this<BufferPool>
{
    std::mutex mu_;
    std::map<size_t, std::vector<void*>> free_;   // capacity -> free buffers
    size_t live_bytes_ = 0, cached_bytes_ = 0;
    uint32_t logLevel_ = 0;

public:
    explicit BufferPool(uint32_t logLevel = 0) : logLevel_(logLevel) {}
    ~BufferPool();

    static size_t bucket(size_t bytes);
    // A buffer of at least `bytes`; throws std::runtime_error when HBM is exhausted.
    PooledBuffer requestBuffer(size_t bytes);
    void giveBack(DeviceBuffer buf);
    // hipFree every cached (unused) buffer.
    void trim();
    size_t liveBytes() const { return live_bytes_; }
    size_t cachedBytes() const { return cached_bytes_; }
};

std::shared_ptr<BufferPool> defaultBufferPool();

}   // namespace vai
