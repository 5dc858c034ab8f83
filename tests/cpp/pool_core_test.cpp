// Host test of the caching pool's bookkeeping (cortexmind_amd/csrc/pool.hpp)
// over a host-memory backend: size classes, same-stream reuse, no reuse
// across streams, foreign and double frees, stats, the release-and-retry
// path on an out-of-memory backend, and stream teardown.  Prints ALL OK and
// returns 0 when every check passes.
#include <cstdio>
#include <cstdlib>
#include <map>

#include "../../cortexmind_amd/csrc/pool.hpp"

namespace {

// Host memory with a byte limit, standing in for the device.
struct HostBackend {
    static size_t limit, in_use;
    static int syncs, allocs, releases;
    static std::map<void *, size_t> sizes;
    static int alloc(void **p, size_t bytes) {
        if (in_use + bytes > limit) return 2;  // out of memory
        *p = std::malloc(bytes);
        if (!*p) return 2;
        sizes[*p] = bytes;
        in_use += bytes;
        ++allocs;
        return 0;
    }
    static void release(void *p) {
        in_use -= sizes[p];
        sizes.erase(p);
        ++releases;
        std::free(p);
    }
    static int sync() {
        ++syncs;
        return 0;
    }
};
size_t HostBackend::limit = size_t(1) << 40, HostBackend::in_use = 0;
int HostBackend::syncs = 0, HostBackend::allocs = 0, HostBackend::releases = 0;
std::map<void *, size_t> HostBackend::sizes;

int failures = 0;
#define EXPECT(c, ...)                          \
    do {                                        \
        if (!(c)) {                             \
            std::printf("FAIL %d: ", __LINE__); \
            std::printf(__VA_ARGS__);           \
            std::printf("\n");                  \
            ++failures;                         \
        }                                       \
    } while (0)

}  // namespace

int main() {
    using cxm::pool_size_class;
    EXPECT(pool_size_class(1) == 512, "class(1)");
    EXPECT(pool_size_class(512) == 512, "class(512)");
    EXPECT(pool_size_class(513) == 1024, "class(513)");
    EXPECT(pool_size_class(1000000) == (size_t(1) << 20), "class(1e6)");
    EXPECT(pool_size_class((size_t(1) << 20) + 1) == (size_t(2) << 20), "class(1MiB+1)");
    EXPECT(pool_size_class(size_t(5) << 20) == (size_t(6) << 20), "class(5MiB)");
    EXPECT(pool_size_class(size_t(256) << 20) == (size_t(256) << 20), "class(256MiB)");

    cxm::CachingPool<HostBackend> pool;
    const void *s1 = reinterpret_cast<const void *>(0x10), *s2 = reinterpret_cast<const void *>(0x20);
    void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr;
    EXPECT(pool.allocate(&a, 1000, 0, s1) == 0 && a, "alloc a");
    EXPECT(pool.block_size(a) == 1024, "a class");
    EXPECT(pool.deallocate(a) == 0, "free a");
    EXPECT(pool.deallocate(a) == -1, "double free rejected");
    int x = 0;
    EXPECT(pool.deallocate(&x) == -1, "foreign pointer rejected");
    EXPECT(pool.allocate(&b, 700, 0, s1) == 0 && b == a, "same class, same stream: reused");
    EXPECT(pool.allocate(&c, 1024, 0, s2) == 0 && c != a, "other stream: not reused");
    pool.deallocate(b);
    EXPECT(pool.allocate(&d, 600, 0, s2) == 0 && d != a, "block cached for s1 is not handed to s2");
    cxm::PoolStats st = pool.stats();
    EXPECT(st.allocs == 4 && st.hits == 1 && st.frees == 2, "counts %llu %llu %llu",
           (unsigned long long)st.allocs, (unsigned long long)st.hits, (unsigned long long)st.frees);
    EXPECT(st.bytes_in_use == 2048 && st.bytes_cached == 1024, "bytes %zu %zu", st.bytes_in_use, st.bytes_cached);
    EXPECT(st.peak_in_use == 2048, "peak %zu", st.peak_in_use);
    EXPECT(st.device_allocs == 3, "device allocs %llu", (unsigned long long)st.device_allocs);

    // out of memory: the cache is given back (one sync) and the allocation retried
    pool.deallocate(c);
    pool.deallocate(d);
    EXPECT(pool.stats().bytes_cached == 3072, "cached before oom %zu", pool.stats().bytes_cached);
    const int releases0 = HostBackend::releases, syncs0 = HostBackend::syncs;
    HostBackend::limit = HostBackend::in_use + 1024;  // a 4 KiB block fits only once the 3 KiB cache is gone
    void *big = nullptr;
    EXPECT(pool.allocate(&big, 4096, 0, s1) == 0 && big, "retry after releasing the cache succeeds");
    EXPECT(HostBackend::releases == releases0 + 3, "three cached blocks released (%d)", HostBackend::releases - releases0);
    EXPECT(HostBackend::syncs == syncs0 + 1, "one sync before releasing");
    EXPECT(pool.stats().bytes_cached == 0, "cache empty after release");
    void *huge = nullptr;
    EXPECT(pool.allocate(&huge, size_t(1) << 30, 0, s1) == 2 && !huge, "still out of memory: the error comes back");
    HostBackend::limit = size_t(1) << 40;

    // release with nothing cached does not sync
    const int syncs1 = HostBackend::syncs;
    EXPECT(pool.release_cached() == 0 && HostBackend::syncs == syncs1, "no-op release");

    // stream teardown returns that stream's cache only
    void *e1 = nullptr, *e2 = nullptr;
    pool.allocate(&e1, 512, 0, s1);
    pool.allocate(&e2, 512, 0, s2);
    pool.deallocate(e1);
    pool.deallocate(e2);
    EXPECT(pool.drop_stream(s1) == 0, "drop s1");
    void *e3 = nullptr, *e4 = nullptr;
    pool.allocate(&e4, 512, 0, s2);
    EXPECT(e4 == e2, "s2's cache survives s1's teardown");
    pool.allocate(&e3, 512, 0, s1);
    EXPECT(pool.stats().bytes_cached == 0, "nothing left cached");

    // devices are kept apart
    void *g0 = nullptr, *g1 = nullptr;
    pool.allocate(&g0, 2048, 0, s1);
    pool.deallocate(g0);
    pool.allocate(&g1, 2048, 1, s1);
    EXPECT(g1 != g0, "device 1 does not reuse device 0's block");

    for (void *p : {a, big, e3, e4, g1}) pool.deallocate(p);
    pool.release_cached();
    EXPECT(HostBackend::in_use == 0, "every block returned (%zu bytes left)", HostBackend::in_use);
    if (failures == 0) std::printf("ALL OK\n");
    return failures == 0 ? 0 : 1;
}
