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

#include "cxm_common.hpp"

namespace {

int st(hipError_t e) { return e == hipSuccess ? CXM_OK : static_cast<int>(e); }

struct WsEntry {
    void *base = nullptr;
    size_t counters = 0;
    size_t scratch_bytes = 0;
    void *xbase = nullptr;  // exchange region (never shared with other kernels' scratch)
    size_t xrows = 0;
    void *tbase = nullptr;  // tagged partial slots (never shared either)
    size_t tslots = 0;
    unsigned tepoch = 0;    // tag of the last call that used them
};

void free_entry(WsEntry &w) {
    if (w.base) (void)hipFree(w.base);
    if (w.xbase) (void)hipFree(w.xbase);
    if (w.tbase) (void)hipFree(w.tbase);
    w.base = w.xbase = w.tbase = nullptr;
}

std::atomic<unsigned> g_xwait{1u << 16};

std::mutex g_ws_mu;
std::map<std::pair<int, cxm_stream_t>, WsEntry> g_ws;

}  // namespace

namespace cxm {

int launch_status() { return st(hipGetLastError()); }

int get_workspace(cxm_stream_t s, size_t counters, size_t scratch_bytes, Workspace *ws) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.base == nullptr || w.counters < counters || w.scratch_bytes < scratch_bytes) {
        size_t nc = counters < 1024 ? 1024 : counters;
        size_t sb = scratch_bytes < (size_t(8) << 20) ? (size_t(8) << 20) : scratch_bytes;
        if (w.counters > nc) nc = w.counters;
        if (w.scratch_bytes > sb) sb = w.scratch_bytes;
        const size_t cw = nc * cxm::kCtr;  // words; a multiple of 64 keeps the scratch 256-byte aligned
        if (w.base != nullptr) {
            // Kernels queued on this stream may still use the old region.
            e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(s));
            if (e != hipSuccess) return st(e);
            e = hipFree(w.base);
            w.base = nullptr;
            if (e != hipSuccess) return st(e);
        }
        void *p = nullptr;
        e = hipMalloc(&p, cw * sizeof(unsigned) + sb);
        if (e != hipSuccess) return st(e);
        e = hipMemsetAsync(p, 0, cw * sizeof(unsigned), reinterpret_cast<hipStream_t>(s));
        if (e != hipSuccess) {
            (void)hipFree(p);
            return st(e);
        }
        w.base = p;
        w.counters = nc;
        w.scratch_bytes = sb;
    }
    ws->counters = static_cast<unsigned *>(w.base);
    ws->counters_n = w.counters;
    ws->scratch = static_cast<unsigned *>(w.base) + w.counters * cxm::kCtr;
    ws->scratch_bytes = w.scratch_bytes;
    return CXM_OK;
}

int get_exchange(cxm_stream_t s, size_t rows, Exchange *x) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.xbase == nullptr || w.xrows < rows) {
        size_t nr = rows < 64 ? 64 : rows;
        if (w.xrows > nr) nr = w.xrows;
        if (w.xbase != nullptr) {
            e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(s));
            if (e != hipSuccess) return st(e);
            e = hipFree(w.xbase);
            w.xbase = nullptr;
            w.xrows = 0;
            if (e != hipSuccess) return st(e);
        }
        const size_t bytes = nr * (kCtr * sizeof(unsigned) + kXMaxSegs * 2 * sizeof(unsigned long long));
        void *p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return st(e);
        // all-zero: epoch 0, tickets 0, every slot tagged 0
        e = hipMemsetAsync(p, 0, bytes, reinterpret_cast<hipStream_t>(s));
        if (e != hipSuccess) {
            (void)hipFree(p);
            return st(e);
        }
        w.xbase = p;
        w.xrows = nr;
    }
    x->hdr = static_cast<unsigned *>(w.xbase);
    x->slots = reinterpret_cast<unsigned long long *>(static_cast<unsigned *>(w.xbase) + w.xrows * kCtr);
    return CXM_OK;
}

int get_tagged(cxm_stream_t s, size_t n, TaggedSlots *t) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return st(e);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(reinterpret_cast<hipStream_t>(s), &cap);
    if (e != hipSuccess) return st(e);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsEntry &w = g_ws[{dev, s}];
    if (w.tbase == nullptr || w.tslots < n) {
        size_t nn = n < 4096 ? 4096 : n;
        if (w.tslots > nn) nn = w.tslots;
        if (w.tbase != nullptr) {
            e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(s));
            if (e != hipSuccess) return st(e);
            e = hipFree(w.tbase);
            w.tbase = nullptr;
            w.tslots = 0;
            if (e != hipSuccess) return st(e);
        }
        const size_t bytes = nn * sizeof(unsigned long long);
        void *p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return st(e);
        // all-zero: every slot tagged 0, a tag no call uses
        e = hipMemsetAsync(p, 0, bytes, reinterpret_cast<hipStream_t>(s));
        if (e != hipSuccess) {
            (void)hipFree(p);
            return st(e);
        }
        w.tbase = p;
        w.tslots = nn;
    }
    if (++w.tepoch == 0) w.tepoch = 1;
    t->slots = static_cast<unsigned long long *>(w.tbase);
    t->n = w.tslots;
    t->epoch = w.tepoch;
    t->clear = cap != hipStreamCaptureStatusNone ? 1 : 0;
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
        hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(kv.first.second));
        if (e == hipSuccess && kv.second.base) e = hipFree(kv.second.base);
        if (e == hipSuccess && kv.second.xbase) e = hipFree(kv.second.xbase);
        if (e == hipSuccess && kv.second.tbase) e = hipFree(kv.second.tbase);
        if (e != hipSuccess && rc == CXM_OK) rc = st(e);
    }
    g_ws.clear();
    (void)hipSetDevice(cur);
    return rc;
}

}  // extern "C"
