// Device scratch memory of the kernels that need more than their inputs and
// outputs: split-K partial tiles, gathered expert rows and their tile list,
// transpose = false partial sums, decode-attention partials.
//
// Two sources:
//  * the library-owned workspace, one buffer per (device, stream).  Calls on
//    one stream are ordered, so they may share its buffer; calls on two
//    streams never share one.  Buffers only grow, and a buffer is never
//    freed while the process runs: a HIP graph captured earlier keeps the
//    address it recorded, so the retired buffer must stay valid for its
//    replays.  Growth is geometric (at least twice the old size), so the
//    retired buffers of a stream hold less than its current one.  No buffer
//    is allocated while the stream is capturing (the caller then takes a
//    plan without scratch, or fails with a message).
//  * a fixed region named by the caller (the allocation-free entry points):
//    never grown; a request beyond its size gets nothing.
//
// Kernels that hand results between workgroups of one launch also need
// arrival counters that start at zero: one small zero-filled buffer per
// (device, stream), separate from the workspace (whose contents other
// kernels overwrite), which every such kernel leaves zeroed when it ends.
#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "eq_common.hpp"

namespace eq {

namespace {

struct OwnedBuffer {
    void* ptr = nullptr;
    size_t cap = 0;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, OwnedBuffer>& owned_buffers() {
    static auto* m = new std::map<std::pair<int, hipStream_t>, OwnedBuffer>();  // lives until exit
    return *m;
}
std::map<std::pair<int, hipStream_t>, unsigned*>& counter_buffers() {
    static auto* m = new std::map<std::pair<int, hipStream_t>, unsigned*>();  // lives until exit
    return *m;
}
std::vector<void*>& retired_buffers() {
    static auto* v = new std::vector<void*>();  // kept alive: graphs may still use them
    return *v;
}

}  // namespace

int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

void* ws_acquire(const WsSource* src, size_t bytes, hipStream_t st) {
    if (bytes == 0) bytes = 256;
    if (src) return bytes <= src->cap ? src->ptr : nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    OwnedBuffer& buf = owned_buffers()[std::make_pair(dev, st)];
    if (buf.cap >= bytes) return buf.ptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    size_t want = bytes;
    if (want < 2 * buf.cap) want = 2 * buf.cap;
    if (want < (size_t(4) << 20)) want = size_t(4) << 20;
    want = (want + 255) & ~size_t(255);
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();  // a failed allocation is reported by the caller, not by the next launch check
        return nullptr;
    }
    if (buf.ptr) retired_buffers().push_back(buf.ptr);
    buf.ptr = p;
    buf.cap = want;
    return p;
}

unsigned* ws_counters(const WsSource* src, hipStream_t st) {
    if (src) return src->counters;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    unsigned*& c = counter_buffers()[std::make_pair(dev, st)];
    if (c) return c;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, size_t(kWsCounters) * sizeof(unsigned)) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    // zeroed once, in stream order before any kernel of `st` counts in it;
    // every kernel leaves its counters at zero again
    if (hipMemsetAsync(p, 0, size_t(kWsCounters) * sizeof(unsigned), st) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p);
        return nullptr;
    }
    c = static_cast<unsigned*>(p);
    return c;
}

}  // namespace eq
