// C ABI of the stream-ordered caching allocator (pool.hpp) over hipMalloc.
#include "cxm_common.hpp"
#include "pool.hpp"

namespace cxm {
namespace {

struct HipBackend {
    static int alloc(void **p, size_t bytes) {
        const hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();  // clear the sticky out-of-memory status before a retry
            return static_cast<int>(e);
        }
        return 0;
    }
    static void release(void *p) { (void)hipFree(p); }
    static int sync() { return static_cast<int>(hipDeviceSynchronize()); }
};

CachingPool<HipBackend> &pool() {
    static CachingPool<HipBackend> p;
    return p;
}

}  // namespace

int pool_drop_stream(cxm_stream_t s) { return pool().drop_stream(s); }

}  // namespace cxm

extern "C" {

int cxm_pool_alloc(void **ptr, size_t bytes, cxm_stream_t s) {
    if (!ptr || bytes == 0) return CXM_E_INVALID;
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    const int rc = cxm::pool().allocate(ptr, bytes, dev, s);
    return rc < 0 ? CXM_E_INVALID : rc;
}

int cxm_pool_free(void *ptr) { return cxm::pool().deallocate(ptr) == 0 ? CXM_OK : CXM_E_INVALID; }

int cxm_pool_release(void) { return cxm::pool().release_cached(); }

int cxm_pool_stats(cxm_pool_stats_t *out) {
    if (!out) return CXM_E_INVALID;
    const cxm::PoolStats s = cxm::pool().stats();
    out->bytes_in_use = s.bytes_in_use;
    out->bytes_cached = s.bytes_cached;
    out->peak_in_use = s.peak_in_use;
    out->allocs = s.allocs;
    out->hits = s.hits;
    out->frees = s.frees;
    out->device_allocs = s.device_allocs;
    return CXM_OK;
}

}  // extern "C"
