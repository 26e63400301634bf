// buffer-pool.cpp -- hipMalloc-backed BufferPool.
#include "buffer-pool.h"

#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../include/vai_amd.h"

namespace vai {

void PooledBuffer::release()
{
    if (buf_.ptr && pool_) pool_->giveBack(buf_);
    buf_ = {};
    pool_.reset();
}

size_t BufferPool::bucket(size_t bytes)
{
    size_t b = 256;
    while (b < bytes) b <<= 1;
    return b;
}

PooledBuffer BufferPool::requestBuffer(size_t bytes)
{
    const size_t cap = bucket(bytes ? bytes : 1);
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = free_.find(cap);
        if (it != free_.end() && !it->second.empty()) {
            void* p = it->second.back();
            it->second.pop_back();
            cached_bytes_ -= cap;
            live_bytes_ += cap;
            if (logLevel_ >= 2) std::fprintf(stderr, "[BufferPool] reuse %zu B\n", cap);
            return PooledBuffer(shared_from_this(), {p, cap});
        }
    }
    void* p = nullptr;
    vai_status st = vai_malloc(&p, cap);
    if (st != VAI_OK) {
        trim();
        st = vai_malloc(&p, cap);
        if (st != VAI_OK)
            throw std::runtime_error(std::string("BufferPool: hipMalloc of ") + std::to_string(cap) +
                                     " bytes failed: " + vai_status_string(st));
    }
    {
        std::lock_guard<std::mutex> lk(mu_);
        live_bytes_ += cap;
    }
    if (logLevel_ >= 1) std::fprintf(stderr, "[BufferPool] new %zu B\n", cap);
    return PooledBuffer(shared_from_this(), {p, cap});
}

void BufferPool::giveBack(DeviceBuffer buf)
{
    std::lock_guard<std::mutex> lk(mu_);
    free_[buf.size].push_back(buf.ptr);
    live_bytes_ -= buf.size;
    cached_bytes_ += buf.size;
}

void BufferPool::trim()
{
    std::lock_guard<std::mutex> lk(mu_);
    for (auto& [cap, v] : free_)
        for (void* p : v) vai_free(p);
    free_.clear();
    cached_bytes_ = 0;
}

BufferPool::~BufferPool() { trim(); }

std::shared_ptr<BufferPool> defaultBufferPool()
{
    // Never destroyed: freeing device memory from a static destructor could
    // run after the HIP runtime has shut down.
    static auto* pool = new std::shared_ptr<BufferPool>(std::make_shared<BufferPool>());
    return *pool;
}

}   // namespace vai
