// MemoryPool.hpp -- caching allocator for tensor storage and GEMM workspaces.
//
// Same contract as the reference's MemoryPool (include/MemoryPool.hpp:24-127):
// allocate/free by (bytes, device), power-of-two size bins, blocks cached
// until empty_cache(), mutex-protected.  Device blocks come from hipMalloc on
// the tensor's device; host blocks are 64-byte aligned heap memory (so CPU
// tensors work on machines without a GPU).  Split-K partials and im2col
// buffers are taken from here, so once warm no GEMM call allocates.
//
// Reservation (graph capture): blocks handed out while a Reservation is active
// on the calling thread are not recycled when freed; they go back to the cache
// only when the Reservation is destroyed.  A captured HIP graph keeps using
// the addresses it recorded, so those blocks must not be given to other
// tensors while the graph can still be replayed.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>
#include <new>
#include <unordered_map>
#include <utility>
#include <vector>

#include "Defines.hpp"
#include "GpuUtils.hpp"

class MemoryPool {
public:
    static MemoryPool& get() {
        static MemoryPool pool;
        return pool;
    }

    class Reservation {
    public:
        Reservation() = default;
        ~Reservation() { MemoryPool::get().end_reservation(*this); }
        Reservation(const Reservation&) = delete;
        Reservation& operator=(const Reservation&) = delete;
        void start() { active() = this; }
        void stop() {
            if (active() == this) active() = nullptr;
        }
        size_t blocks() const { return blocks_.size(); }
        // Whether a Reservation is pinning this thread's allocations now.
        static bool active_on_this_thread() { return active() != nullptr; }
        size_t fresh_allocations() const { return fresh_; }  // blocks that needed a new malloc

    private:
        friend class MemoryPool;
        static Reservation*& active() {
            thread_local Reservation* r = nullptr;
            return r;
        }
        std::vector<void*> blocks_;
        size_t fresh_ = 0;
    };

    void* allocate(size_t bytes, Device device) {
        if (bytes == 0) return nullptr;
        const size_t b = bin(bytes);
        Reservation* r = Reservation::active();
        {
            std::lock_guard<std::mutex> lk(mu_);
            auto& fl = cache(device)[b];
            if (!fl.empty()) {
                void* p = fl.back();
                fl.pop_back();
                if (r) reserve_locked(r, p, b, device);
                return p;
            }
        }
        if (r) ++r->fresh_;
        void* p = fresh(b, device);
        if (r) {
            std::lock_guard<std::mutex> lk(mu_);
            reserve_locked(r, p, b, device);
        }
        return p;
    }

    void free(void* p, size_t bytes, Device device) {
        if (!p || bytes == 0) return;
        std::lock_guard<std::mutex> lk(mu_);
        auto it = reserved_.find(p);
        if (it != reserved_.end()) {  // held for a captured graph: recycled later
            it->second.freed = true;
            return;
        }
        cache(device)[bin(bytes)].push_back(p);
    }

    // Returns every cached block to the system (device memory: hipFree).
    void empty_cache() {
        release(Device(DeviceType::CPU));
        for (int i = 0; i < kMaxGpus; ++i) release(Device(DeviceType::CUDA, (uint8_t)i));
    }

    size_t cached_blocks(Device device) {
        std::lock_guard<std::mutex> lk(mu_);
        size_t n = 0;
        for (auto& kv : cache(device)) n += kv.second.size();
        return n;
    }

    static size_t bin(size_t bytes) {
        size_t b = 256;
        while (b < bytes) b <<= 1;
        return b;
    }

private:
    struct Held {
        size_t bin;
        Device device;
        bool freed;
    };

    void reserve_locked(Reservation* r, void* p, size_t b, Device device) {
        r->blocks_.push_back(p);
        reserved_[p] = Held{b, device, false};
    }

    void end_reservation(Reservation& r) {
        r.stop();
        std::lock_guard<std::mutex> lk(mu_);
        for (void* p : r.blocks_) {
            auto it = reserved_.find(p);
            if (it == reserved_.end()) continue;
            if (it->second.freed) cache(it->second.device)[it->second.bin].push_back(p);
            reserved_.erase(it);   // still owned by a live tensor: its free() caches it
        }
        r.blocks_.clear();
    }

    void* fresh(size_t b, Device device) {
        if (device.is_gpu()) {
            int prev = 0;
            GPU_CHECK(hipGetDevice(&prev));
            if (prev != device.index) GPU_CHECK(hipSetDevice(device.index));
            void* p = nullptr;
            hipError_t e = hipMalloc(&p, b);
            if (e != hipSuccess) {  // release cached blocks once and retry
                release(device);
                e = hipMalloc(&p, b);
            }
            if (prev != device.index) (void)hipSetDevice(prev);
            if (e != hipSuccess) mt_detail::hip_fail(e, __FILE__, __LINE__);
            return p;
        }
        void* p = std::aligned_alloc(64, b);
        if (!p) throw std::bad_alloc();
        return p;
    }

    static constexpr int kMaxGpus = 16;
    using Bins = std::unordered_map<size_t, std::vector<void*>>;

    MemoryPool() = default;
    ~MemoryPool() = default;  // blocks are kept until process exit, as the reference does

    Bins& cache(Device d) {
        if (!d.is_gpu()) return host_;
        if (d.index >= kMaxGpus) throw std::invalid_argument("MemoryPool: device index out of range");
        return gpu_[d.index];
    }

    void release(Device d) {
        std::vector<void*> blocks;
        {
            std::lock_guard<std::mutex> lk(mu_);
            for (auto& kv : cache(d)) {
                blocks.insert(blocks.end(), kv.second.begin(), kv.second.end());
                kv.second.clear();
            }
        }
        for (void* p : blocks) {
            if (d.is_gpu()) (void)hipFree(p);
            else std::free(p);
        }
    }

    std::mutex mu_;
    Bins host_;
    Bins gpu_[kMaxGpus];
    std::unordered_map<void*, Held> reserved_;   // blocks of live Reservations
};
