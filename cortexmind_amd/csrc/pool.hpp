// Stream-ordered caching allocator for device memory: the core, independent
// of the device API so that its bookkeeping can be tested on the host.
//
// Replaces the reference's ForgeChunk (source/CortexMind/framework/Memory/
// forge.cuh:30-90, forge.cu:13-122): one fixed 128 MiB cudaMalloc carved
// first-fit, which is never seeded (allocate returns nullptr until reset(),
// forge.cu:13-22) and cannot hold one [8192, 8192] fp32 tensor.  Here:
//  * requests round up to a size class: powers of two from 512 B to 1 MiB,
//    then multiples of 2 MiB, so a freed block is reused by any request of
//    its class without splitting or coalescing;
//  * a block belongs to the stream it was allocated on.  A freed block goes
//    back to that stream's free list and is reused only by allocations on
//    the same stream, whose queue order already places the new use after
//    every use before the free; using a block on another stream needs the
//    caller's own synchronisation, as with any stream-ordered allocator;
//  * when the device allocation fails, the cached blocks are returned to
//    the device (after a device sync) and the allocation is retried once;
//  * blocks of 64 GiB and above are not cached (returned on free).
// Sized for a 288 GB HBM3E part: no pool limit of its own; the device's
// capacity is the limit.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace cxm {

struct PoolStats {
    size_t bytes_in_use;   // sum of size classes of live blocks
    size_t bytes_cached;   // sum of size classes of freed, cached blocks
    size_t peak_in_use;
    uint64_t allocs;       // successful allocations
    uint64_t hits;         // of which served from the cache
    uint64_t frees;
    uint64_t device_allocs;  // allocations that reached the device API
};

inline size_t pool_size_class(size_t bytes) {
    constexpr size_t kMin = 512, kSmall = size_t(1) << 20, kLarge = size_t(2) << 20;
    if (bytes <= kMin) return kMin;
    if (bytes <= kSmall) {
        size_t c = kMin;
        while (c < bytes) c <<= 1;
        return c;
    }
    return (bytes + kLarge - 1) / kLarge * kLarge;
}

// Backend: static int alloc(void **p, size_t bytes) (0 = ok, else error);
// static void release(void *p); static int sync() (waits for all device work).
template <class Backend>
class CachingPool {
public:
    using Stream = const void *;

    int allocate(void **out, size_t bytes, int device, Stream stream) {
        if (!out || bytes == 0) return -1;
        *out = nullptr;
        const size_t cls = pool_size_class(bytes);
        std::lock_guard<std::mutex> lk(mu_);
        auto it = free_.find(Key{device, stream, cls});
        if (it != free_.end() && !it->second.empty()) {
            void *p = it->second.back();
            it->second.pop_back();
            stats_.bytes_cached -= cls;
            ++stats_.hits;
            return track(p, cls, device, stream, out);
        }
        void *p = nullptr;
        int rc = Backend::alloc(&p, cls);
        if (rc != 0) {
            // give the cache back to the device and try once more
            rc = release_locked();
            if (rc != 0) return rc;
            rc = Backend::alloc(&p, cls);
            if (rc != 0) return rc;
        }
        ++stats_.device_allocs;
        return track(p, cls, device, stream, out);
    }

    // 0, or -1 for a pointer this pool did not hand out (or freed twice).
    int deallocate(void *p) {
        if (!p) return 0;
        std::lock_guard<std::mutex> lk(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) return -1;
        const Live b = it->second;
        live_.erase(it);
        stats_.bytes_in_use -= b.cls;
        ++stats_.frees;
        if (b.cls >= (size_t(64) << 30)) {
            Backend::release(p);
            return 0;
        }
        free_[Key{b.device, b.stream, b.cls}].push_back(p);
        stats_.bytes_cached += b.cls;
        return 0;
    }

    // Returns every cached block to the device (after waiting for all work).
    int release_cached() {
        std::lock_guard<std::mutex> lk(mu_);
        return release_locked();
    }

    // Forgets the blocks cached for a stream that is being destroyed: they
    // are returned to the device (after a sync).
    int drop_stream(Stream stream) {
        std::lock_guard<std::mutex> lk(mu_);
        bool any = false;
        for (auto &kv : free_)
            if (kv.first.stream == stream && !kv.second.empty()) any = true;
        if (!any) return 0;
        int rc = Backend::sync();
        if (rc != 0) return rc;
        for (auto it = free_.begin(); it != free_.end();) {
            if (it->first.stream == stream) {
                for (void *p : it->second) {
                    Backend::release(p);
                    stats_.bytes_cached -= it->first.cls;
                }
                it = free_.erase(it);
            } else {
                ++it;
            }
        }
        return 0;
    }

    PoolStats stats() {
        std::lock_guard<std::mutex> lk(mu_);
        return stats_;
    }

    // Size class of a live block (0 if unknown).
    size_t block_size(const void *p) {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = live_.find(const_cast<void *>(p));
        return it == live_.end() ? 0 : it->second.cls;
    }

private:
    struct Key {
        int device;
        Stream stream;
        size_t cls;
        bool operator<(const Key &o) const {
            if (device != o.device) return device < o.device;
            if (stream != o.stream) return stream < o.stream;
            return cls < o.cls;
        }
    };
    struct Live {
        size_t cls;
        int device;
        Stream stream;
    };

    int track(void *p, size_t cls, int device, Stream stream, void **out) {
        live_[p] = Live{cls, device, stream};
        stats_.bytes_in_use += cls;
        if (stats_.bytes_in_use > stats_.peak_in_use) stats_.peak_in_use = stats_.bytes_in_use;
        ++stats_.allocs;
        *out = p;
        return 0;
    }

    int release_locked() {
        if (stats_.bytes_cached == 0) return 0;
        int rc = Backend::sync();
        if (rc != 0) return rc;
        for (auto &kv : free_)
            for (void *p : kv.second) Backend::release(p);
        free_.clear();
        stats_.bytes_cached = 0;
        return 0;
    }

    std::mutex mu_;
    std::map<Key, std::vector<void *>> free_;
    std::unordered_map<void *, Live> live_;
    PoolStats stats_{};
};

}  // namespace cxm
