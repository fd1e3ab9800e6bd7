// lq_runtime.hip -- errors, device caching allocator, copies, streams and events.
//
// Stands in for the parts of Lucid's engine the quantized path touches on the device
// side: storage allocation (lucid/_C/core/Allocator.h), device selection and the
// synchronisation the bench harness brackets timings with (lucid/metal/__init__.py:56).
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "lq_internal.h"

namespace lq {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_hip(hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return set_error(e == hipErrorOutOfMemory ? LQ_ERR_NOMEM : LQ_ERR_HIP, m);
}

// ---------------------------------------------------------------------- allocator
// Per-device caching allocator.  Freed blocks go back to a size-ordered free list and
// are reused by later requests of up to twice their size; nothing is returned to HIP
// until lq_empty_cache.  Blocks are reused in host call order, so work that shares a
// block must run on one stream (the library's usage model: one stream per thread).
namespace {
struct Block {
    size_t size;
    int device;
};
struct Allocator {
    std::mutex mu;
    std::unordered_map<void*, Block> live;
    std::map<int, std::multimap<size_t, void*>> free_lists;
    size_t allocated = 0;
    size_t cached = 0;
};
Allocator& alloc() {
    static Allocator* a = new Allocator();  // never destroyed: outlives static teardown
    return *a;
}
size_t round_size(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes <= (1u << 20)) return (bytes + 511) & ~size_t(511);
    return (bytes + (2u << 20) - 1) & ~size_t((2u << 20) - 1);
}
}  // namespace

}  // namespace lq

using namespace lq;

extern "C" {

int lq_abi_version(void) { return LQ_ABI_VERSION; }

const char* lq_last_error(void) { return g_last_error.c_str(); }

const char* lq_backend_name(void) { return "hip-gfx950"; }

int lq_device_count(int* count) {
    LQ_REQUIRE(count, "lq_device_count: NULL count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        n = 0;  // no device / no driver is not an error here
    }
    *count = n;
    return LQ_OK;
}

int lq_set_device(int device) {
    LQ_HIP(hipSetDevice(device));
    return LQ_OK;
}

int lq_get_device(int* device) {
    LQ_REQUIRE(device, "lq_get_device: NULL device");
    LQ_HIP(hipGetDevice(device));
    return LQ_OK;
}

int lq_malloc(void** d_ptr, size_t bytes) {
    LQ_REQUIRE(d_ptr, "lq_malloc: NULL out pointer");
    int dev = 0;
    LQ_HIP(hipGetDevice(&dev));
    size_t sz = round_size(bytes);
    Allocator& a = alloc();
    {
        std::lock_guard<std::mutex> g(a.mu);
        auto& fl = a.free_lists[dev];
        auto it = fl.lower_bound(sz);
        if (it != fl.end() && it->first <= 2 * sz) {
            void* p = it->second;
            size_t got = it->first;
            fl.erase(it);
            a.live[p] = Block{got, dev};
            a.cached -= got;
            a.allocated += got;
            *d_ptr = p;
            return LQ_OK;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
        // Release the cache once and retry before giving up.
        (void)hipGetLastError();
        lq_empty_cache();
        e = hipMalloc(&p, sz);
        if (e != hipSuccess) return check_hip(e, "lq_malloc: hipMalloc");
    }
    std::lock_guard<std::mutex> g(a.mu);
    a.live[p] = Block{sz, dev};
    a.allocated += sz;
    *d_ptr = p;
    return LQ_OK;
}

int lq_free(void* d_ptr) {
    if (!d_ptr) return LQ_OK;
    Allocator& a = alloc();
    std::lock_guard<std::mutex> g(a.mu);
    auto it = a.live.find(d_ptr);
    if (it == a.live.end()) return set_error(LQ_ERR_INVALID, "lq_free: pointer not from lq_malloc");
    Block b = it->second;
    a.live.erase(it);
    a.allocated -= b.size;
    a.cached += b.size;
    a.free_lists[b.device].emplace(b.size, d_ptr);
    return LQ_OK;
}

int lq_empty_cache(void) {
    Allocator& a = alloc();
    std::vector<std::pair<int, void*>> victims;
    {
        std::lock_guard<std::mutex> g(a.mu);
        for (auto& kv : a.free_lists)
            for (auto& e : kv.second) victims.emplace_back(kv.first, e.second);
        a.free_lists.clear();
        a.cached = 0;
    }
    if (victims.empty()) return LQ_OK;
    int cur = 0;
    LQ_HIP(hipGetDevice(&cur));
    for (auto& v : victims) {
        LQ_HIP(hipSetDevice(v.first));
        LQ_HIP(hipFree(v.second));
    }
    LQ_HIP(hipSetDevice(cur));
    return LQ_OK;
}

int lq_memory_stats(size_t* allocated, size_t* cached) {
    Allocator& a = alloc();
    std::lock_guard<std::mutex> g(a.mu);
    if (allocated) *allocated = a.allocated;
    if (cached) *cached = a.cached;
    return LQ_OK;
}

int lq_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, void* stream) {
    if (bytes == 0) return LQ_OK;
    LQ_REQUIRE(d_dst && h_src, "lq_memcpy_h2d: NULL pointer");
    LQ_HIP(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    LQ_HIP(hipStreamSynchronize(as_stream(stream)));  // pageable source: complete before return
    return LQ_OK;
}

int lq_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, void* stream) {
    if (bytes == 0) return LQ_OK;
    LQ_REQUIRE(h_dst && d_src, "lq_memcpy_d2h: NULL pointer");
    LQ_HIP(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    LQ_HIP(hipStreamSynchronize(as_stream(stream)));
    return LQ_OK;
}

int lq_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes, void* stream) {
    if (bytes == 0) return LQ_OK;
    LQ_REQUIRE(d_dst && d_src, "lq_memcpy_d2d: NULL pointer");
    LQ_HIP(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return LQ_OK;
}

}  // extern "C"

__global__ void lq_fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, size_t count) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < count; i += stride) dst[i] = value;
}

extern "C" {

int lq_fill_u32(void* d_dst, uint32_t value, size_t count, void* stream) {
    if (count == 0) return LQ_OK;
    LQ_REQUIRE(d_dst, "lq_fill_u32: NULL pointer");
    size_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(lq_fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       (uint32_t*)d_dst, value, count);
    return launch_status("lq_fill_u32");
}

int lq_stream_create(void** stream) {
    LQ_REQUIRE(stream, "lq_stream_create: NULL out pointer");
    hipStream_t s;
    LQ_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = (void*)s;
    return LQ_OK;
}

int lq_stream_destroy(void* stream) {
    if (!stream) return LQ_OK;
    LQ_HIP(hipStreamDestroy(as_stream(stream)));
    return LQ_OK;
}

int lq_stream_synchronize(void* stream) {
    LQ_HIP(hipStreamSynchronize(as_stream(stream)));
    return LQ_OK;
}

int lq_device_synchronize(void) {
    LQ_HIP(hipDeviceSynchronize());
    return LQ_OK;
}

int lq_event_create(void** event) {
    LQ_REQUIRE(event, "lq_event_create: NULL out pointer");
    hipEvent_t e;
    LQ_HIP(hipEventCreate(&e));
    *event = (void*)e;
    return LQ_OK;
}

int lq_event_destroy(void* event) {
    if (!event) return LQ_OK;
    LQ_HIP(hipEventDestroy((hipEvent_t)event));
    return LQ_OK;
}

int lq_event_record(void* event, void* stream) {
    LQ_REQUIRE(event, "lq_event_record: NULL event");
    LQ_HIP(hipEventRecord((hipEvent_t)event, as_stream(stream)));
    return LQ_OK;
}

int lq_event_synchronize(void* event) {
    LQ_REQUIRE(event, "lq_event_synchronize: NULL event");
    LQ_HIP(hipEventSynchronize((hipEvent_t)event));
    return LQ_OK;
}

int lq_event_elapsed_ms(float* ms, void* start, void* stop) {
    LQ_REQUIRE(ms && start && stop, "lq_event_elapsed_ms: NULL argument");
    LQ_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return LQ_OK;
}

int lq_graph_begin_capture(void* stream) {
    LQ_REQUIRE(stream, "lq_graph_begin_capture: capture needs a created stream, not the null stream");
    LQ_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return LQ_OK;
}

int lq_graph_end_capture(void* stream, void** graph_exec) {
    LQ_REQUIRE(stream && graph_exec, "lq_graph_end_capture: NULL argument");
    hipGraph_t g = nullptr;
    LQ_HIP(hipStreamEndCapture((hipStream_t)stream, &g));
    hipGraphExec_t e = nullptr;
    const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);  // the executable graph keeps what it needs
    if (err != hipSuccess) return check_hip(err, "hipGraphInstantiate");
    *graph_exec = (void*)e;
    return LQ_OK;
}

int lq_graph_launch(void* graph_exec, void* stream) {
    LQ_REQUIRE(graph_exec, "lq_graph_launch: NULL graph");
    LQ_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
    return LQ_OK;
}

int lq_graph_destroy(void* graph_exec) {
    if (graph_exec) LQ_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    return LQ_OK;
}

}  // extern "C"
