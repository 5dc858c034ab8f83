// Device, memory, stream and event entry points of the C ABI, plus the
// per-(device, stream) workspace the multi-pass kernels use and the
// exchange region of the single-pass long-row softmax.
//
// Replaces the reference's device pool and copies: ForgeChunk
// (source/CortexMind/framework/Memory/forge.cu:13-122, one 128 MiB
// cudaMalloc carved first-fit) and transform (Memory/transform.cu:17-40,
// blocking cudaMemcpy).  Allocation here is a direct hipMalloc: on a
// 288 GB HBM3E part the fixed 128 MiB pool cannot even hold one
// [8192, 8192] fp32 tensor, and hipMalloc already returns 256-byte
// aligned memory that the vector kernels rely on.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "cxm_common.hpp"

namespace {

int st(hipError_t e) { return e == hipSuccess ? CXM_OK : static_cast<int>(e); }

// One device region of a stream's scratch.  `pinned`: handed to a launch
// made under stream capture, so a graph holds its address; it is then never
// freed while the entry lives (a growth retires it instead) and goes back to
// the device only with the stream (cxm_stream_destroy) or at
// cxm_release_workspaces.
struct Region {
    void *p = nullptr;
    size_t size = 0;  // counters (workspace), rows (exchange) or slots (tagged)
    size_t bytes = 0;
    bool pinned = false;
};

struct WsEntry {
    Region ws;       // ticket counters + partials
    size_t ws_counters = 0, ws_scratch = 0;
    Region xc;       // exchange region (never shared with other kernels' scratch)
    Region tg;       // tagged partial slots (never shared either)
    std::vector<void *> retired;  // pinned regions replaced by a growth
};

void free_entry(WsEntry &w) {
    for (Region *r : {&w.ws, &w.xc, &w.tg}) {
        if (r->p) (void)hipFree(r->p);
        *r = Region{};
    }
    for (void *p : w.retired) (void)hipFree(p);
    w.retired.clear();
}

std::atomic<unsigned> g_xwait{1u << 16};
// Tags of the flat reductions' slots, one counter for the whole process: a
// region freed by one stream and handed to another by the allocator can
// hold no slot with a tag a later call uses (until 2^32 calls have passed).
std::atomic<unsigned> g_tag{0};

std::mutex g_ws_mu;
std::map<std::pair<int, cxm_stream_t>, WsEntry> g_ws;

// Whether s is capturing (any capture status but none).
int capturing(cxm_stream_t s, bool *cap) {
    hipStreamCaptureStatus c = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(reinterpret_cast<hipStream_t>(s), &c);
    if (e != hipSuccess) return st(e);
    *cap = c != hipStreamCaptureStatusNone;
    return CXM_OK;
}

// Makes r a zero-filled region of `bytes` (recording `size`), replacing a
// smaller one.  Under capture nothing is allocated, filled or synchronised
// (a hipMemsetAsync would only be recorded into the graph, not run):
// CXM_E_CAPTURE, and the caller makes one eager call of that shape first.
// A replaced region the stream's queued kernels may still use is waited
// for; a pinned one is kept (a captured graph holds its address).
int grow(WsEntry &w, Region &r, size_t size, size_t bytes, bool cap, cxm_stream_t s) {
    if (cap) return CXM_E_CAPTURE;
    hipStream_t hs = reinterpret_cast<hipStream_t>(s);
    if (r.p != nullptr) {
        const hipError_t e = hipStreamSynchronize(hs);
        if (e != hipSuccess) return st(e);
        if (r.pinned) {
            w.retired.push_back(r.p);
        } else {
            const hipError_t f = hipFree(r.p);
            if (f != hipSuccess) return st(f);
        }
        r = Region{};
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return st(e);
    e = hipMemsetAsync(p, 0, bytes, hs);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return st(e);
    }
    r.p = p;
    r.size = size;
    r.bytes = bytes;
    r.pinned = false;
    return CXM_OK;
}

}  // namespace

namespace cxm {

int launch_status() { return st(hipGetLastError()); }

int get_workspace(cxm_stream_t s, size_t counters, size_t scratch_bytes, Workspace *ws) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    bool cap = false;
    int rc = capturing(s, &cap);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.ws.p == nullptr || w.ws_counters < counters || w.ws_scratch < scratch_bytes) {
        size_t nc = counters < 1024 ? 1024 : counters;
        size_t sb = scratch_bytes < (size_t(8) << 20) ? (size_t(8) << 20) : scratch_bytes;
        if (w.ws_counters > nc) nc = w.ws_counters;
        if (w.ws_scratch > sb) sb = w.ws_scratch;
        const size_t cw = nc * cxm::kCtr;  // words; a multiple of 64 keeps the scratch 256-byte aligned
        // only the counters need zeros; the fill covers the region's start
        rc = grow(w, w.ws, nc, cw * sizeof(unsigned) + sb, cap, s);
        if (rc) return rc;
        w.ws_counters = nc;
        w.ws_scratch = sb;
    }
    if (cap) w.ws.pinned = true;
    ws->counters = static_cast<unsigned *>(w.ws.p);
    ws->counters_n = w.ws_counters;
    ws->scratch = static_cast<unsigned *>(w.ws.p) + w.ws_counters * cxm::kCtr;
    ws->scratch_bytes = w.ws_scratch;
    return CXM_OK;
}

int get_exchange(cxm_stream_t s, size_t rows, Exchange *x) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    bool cap = false;
    int rc = capturing(s, &cap);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.xc.p == nullptr || w.xc.size < rows) {
        size_t nr = rows < 64 ? 64 : rows;
        if (w.xc.size > nr) nr = w.xc.size;
        // all-zero: epoch 0, tickets 0, every slot tagged 0
        const size_t bytes = nr * (kCtr * sizeof(unsigned) + kXMaxSegs * 2 * sizeof(unsigned long long));
        rc = grow(w, w.xc, nr, bytes, cap, s);
        if (rc) return rc;
    }
    if (cap) w.xc.pinned = true;
    x->hdr = static_cast<unsigned *>(w.xc.p);
    x->slots = reinterpret_cast<unsigned long long *>(static_cast<unsigned *>(w.xc.p) + w.xc.size * kCtr);
    return CXM_OK;
}

int get_tagged(cxm_stream_t s, size_t n, TaggedSlots *t) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    bool cap = false;
    int rc = capturing(s, &cap);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.tg.p == nullptr || w.tg.size < n) {
        size_t nn = n < 4096 ? 4096 : n;
        if (w.tg.size > nn) nn = w.tg.size;
        // all-zero: every slot tagged 0, a tag no call uses
        rc = grow(w, w.tg, nn, nn * sizeof(unsigned long long), cap, s);
        if (rc) return rc;
    }
    if (cap) w.tg.pinned = true;
    t->slots = static_cast<unsigned long long *>(w.tg.p);
    t->n = w.tg.size;
    t->epoch = next_tag();
    t->clear = cap ? 1 : 0;
    return CXM_OK;
}

unsigned next_tag() {
    unsigned v = g_tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
    while (v == 0u || v == ~0u)  // 0 marks an empty slot; ~0 is tag 0's miss mark
        v = g_tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
    return v;
}

int device_layout(DevLayout *out) {
    static std::atomic<int> cus[64], xccs[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    if (dev < 0 || dev >= 64) return CXM_E_TOO_LARGE;
    int c = cus[dev].load(std::memory_order_acquire), x = xccs[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return st(e);
        e = hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev);
        if (e != hipSuccess || x < 1) x = 1;
        xccs[dev].store(x, std::memory_order_relaxed);
        cus[dev].store(c, std::memory_order_release);
    }
    out->cus = c;
    out->xccs = x;
    return CXM_OK;
}

int workspace_query(cxm_stream_t s, int which, void **base, size_t *bytes, int *pinned) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws.find({dev, s});
    const Region none{};
    const Region &r = it == g_ws.end() ? none : which == 0 ? it->second.ws : which == 1 ? it->second.xc : it->second.tg;
    *base = r.p;
    *bytes = r.bytes;
    *pinned = r.pinned ? 1 : 0;
    return CXM_OK;
}

unsigned exchange_wait_limit() { return g_xwait.load(std::memory_order_relaxed); }

}  // namespace cxm

extern "C" {

const char *cxm_error_string(int status) {
    switch (status) {
        case CXM_OK: return "success";
        case CXM_E_INVALID: return "invalid argument (null pointer, bad size or enum)";
        case CXM_E_TOO_LARGE: return "size beyond the kernel's index range";
        case CXM_E_NO_DEVICE: return "no gfx950 device";
        case CXM_E_CAPTURE:
            return "stream is capturing and the call needs scratch the stream does not have yet "
                   "(make one eager call of that shape on the stream before capture)";
        default:
            if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
            return "unknown cxm status";
    }
}

int cxm_device_count(int *count) {
    if (!count) return CXM_E_INVALID;
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) return CXM_E_NO_DEVICE;
    return st(e);
}

int cxm_set_device(int device) { return st(hipSetDevice(device)); }

int cxm_device_info(char *name, size_t name_len, int *cu_count, char *arch, size_t arch_len) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return st(e);
    if (name && name_len) {
        std::strncpy(name, p.name, name_len - 1);
        name[name_len - 1] = '\0';
    }
    if (arch && arch_len) {
        std::strncpy(arch, p.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    if (cu_count) *cu_count = p.multiProcessorCount;
    return CXM_OK;
}

int cxm_device_sync(void) { return st(hipDeviceSynchronize()); }

int cxm_dev_malloc(void **ptr, size_t bytes) {
    if (!ptr || bytes == 0) return CXM_E_INVALID;
    *ptr = nullptr;
    return st(hipMalloc(ptr, bytes));
}

int cxm_dev_free(void *ptr) {
    if (!ptr) return CXM_OK;
    return st(hipFree(ptr));
}

int cxm_memcpy_h2d(void *dst, const void *src, size_t bytes, cxm_stream_t s) {
    if (bytes == 0) return CXM_OK;
    if (!dst || !src) return CXM_E_INVALID;
    return st(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, reinterpret_cast<hipStream_t>(s)));
}

int cxm_memcpy_d2h(void *dst, const void *src, size_t bytes, cxm_stream_t s) {
    if (bytes == 0) return CXM_OK;
    if (!dst || !src) return CXM_E_INVALID;
    hipStream_t hs = reinterpret_cast<hipStream_t>(s);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, hs);
    if (e != hipSuccess) return st(e);
    return st(hipStreamSynchronize(hs));
}

int cxm_memcpy_d2d(void *dst, const void *src, size_t bytes, cxm_stream_t s) {
    if (bytes == 0) return CXM_OK;
    if (!dst || !src) return CXM_E_INVALID;
    return st(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, reinterpret_cast<hipStream_t>(s)));
}

int cxm_memset(void *dst, int byte_value, size_t bytes, cxm_stream_t s) {
    if (bytes == 0) return CXM_OK;
    if (!dst) return CXM_E_INVALID;
    return st(hipMemsetAsync(dst, byte_value, bytes, reinterpret_cast<hipStream_t>(s)));
}

int cxm_stream_create(cxm_stream_t *s) {
    if (!s) return CXM_E_INVALID;
    hipStream_t hs = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&hs, hipStreamNonBlocking);
    *s = reinterpret_cast<cxm_stream_t>(hs);
    return st(e);
}

int cxm_stream_sync(cxm_stream_t s) { return st(hipStreamSynchronize(reinterpret_cast<hipStream_t>(s))); }

int cxm_stream_destroy(cxm_stream_t s) {
    if (!s) return CXM_E_INVALID;
    // cached pool blocks of this stream go back to the device: a new stream
    // may reuse the handle value
    (void)cxm::pool_drop_stream(s);
    {
        // Drop this stream's workspaces before the handle can be reused.
        std::lock_guard<std::mutex> lk(g_ws_mu);
        for (auto it = g_ws.begin(); it != g_ws.end();) {
            if (it->first.second == s) {
                (void)hipStreamSynchronize(reinterpret_cast<hipStream_t>(s));
                free_entry(it->second);
                it = g_ws.erase(it);
            } else {
                ++it;
            }
        }
    }
    return st(hipStreamDestroy(reinterpret_cast<hipStream_t>(s)));
}

int cxm_event_create(cxm_event_t *e) {
    if (!e) return CXM_E_INVALID;
    hipEvent_t he = nullptr;
    hipError_t r = hipEventCreate(&he);
    *e = reinterpret_cast<cxm_event_t>(he);
    return st(r);
}

int cxm_event_record(cxm_event_t e, cxm_stream_t s) {
    if (!e) return CXM_E_INVALID;
    return st(hipEventRecord(reinterpret_cast<hipEvent_t>(e), reinterpret_cast<hipStream_t>(s)));
}

int cxm_event_sync(cxm_event_t e) {
    if (!e) return CXM_E_INVALID;
    return st(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e)));
}

int cxm_event_elapsed_ms(float *ms, cxm_event_t start, cxm_event_t stop) {
    if (!ms || !start || !stop) return CXM_E_INVALID;
    return st(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                  reinterpret_cast<hipEvent_t>(stop)));
}

int cxm_event_destroy(cxm_event_t e) {
    if (!e) return CXM_E_INVALID;
    return st(hipEventDestroy(reinterpret_cast<hipEvent_t>(e)));
}

int cxm_workspace_query(cxm_stream_t s, int which, void **base, size_t *bytes, int *pinned) {
    if (!base || !bytes || !pinned || which < 0 || which > 2) return CXM_E_INVALID;
    return cxm::workspace_query(s, which, base, bytes, pinned);
}

int cxm_exchange_wait_limit(unsigned polls, unsigned *previous) {
    const unsigned old = g_xwait.exchange(polls);
    if (previous) *previous = old;
    return CXM_OK;
}

int cxm_release_workspaces(void) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    int rc = CXM_OK;
    int cur = 0;
    (void)hipGetDevice(&cur);
    for (auto &kv : g_ws) {
        (void)hipSetDevice(kv.first.first);
        const hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(kv.first.second));
        if (e != hipSuccess && rc == CXM_OK) rc = st(e);
        if (e == hipSuccess) free_entry(kv.second);
    }
    g_ws.clear();
    (void)hipSetDevice(cur);
    return rc;
}

}  // extern "C"
