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

#include "lq_block_cache.h"
#include "lq_internal.h"

namespace lq {

static thread_local std::string g_last_error;
static thread_local const char* g_last_path = "";

void note_path(const char* path) { g_last_path = path; }

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static int counts[kMaxDevices];  // 0 = not queried yet; racing first queries store the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    if (dev >= kMaxDevices) {
        int n = 0;
        return hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    int n = __atomic_load_n(&counts[dev], __ATOMIC_RELAXED);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    __atomic_store_n(&counts[dev], n, __ATOMIC_RELAXED);
    return n;
}

int check_hip(hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return set_error(e == hipErrorOutOfMemory ? LQ_ERR_NOMEM : LQ_ERR_HIP, m);
}

// ---------------------------------------------------------------------- allocator
// Per-device caching allocator over lq_block_cache.h: freed blocks are reused by later
// requests of up to twice their size, on the stream they were freed on at once and on any
// other stream once a HIP event recorded at the free has completed.  Nothing is returned to
// HIP until lq_empty_cache.
namespace {
// Events are pooled: a free records one, the reuse (or lq_empty_cache) hands it back.
std::mutex g_event_mu;
std::vector<hipEvent_t> g_event_pool;

void* record_marker(void* stream) {
    hipStream_t st = as_stream(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;  // under capture: keep the block bound to this stream
    }
    hipEvent_t e = nullptr;
    {
        std::lock_guard<std::mutex> g(g_event_mu);
        if (!g_event_pool.empty()) {
            e = g_event_pool.back();
            g_event_pool.pop_back();
        }
    }
    if (!e && hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipEventRecord(e, st) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipEventDestroy(e);
        return nullptr;
    }
    return e;
}

bool marker_done(void* marker) {
    const hipError_t r = hipEventQuery(reinterpret_cast<hipEvent_t>(marker));
    if (r == hipSuccess) return true;
    (void)hipGetLastError();  // hipErrorNotReady is not a sticky error
    return false;
}

void release_marker(void* marker) {
    std::lock_guard<std::mutex> g(g_event_mu);
    g_event_pool.push_back(reinterpret_cast<hipEvent_t>(marker));
}

BlockCache& cache() {
    static BlockCache* c = new BlockCache(MarkerOps{record_marker, marker_done, release_marker});  // never destroyed
    return *c;
}
}  // namespace

}  // namespace lq

using namespace lq;

extern "C" {

int lq_abi_version(void) { return LQ_ABI_VERSION; }

const char* lq_last_error(void) { return g_last_error.c_str(); }

const char* lq_last_path(void) { return g_last_path; }

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

int lq_malloc_async(void** d_ptr, size_t bytes, void* stream) {
    LQ_REQUIRE(d_ptr, "lq_malloc: NULL out pointer");
    int dev = 0;
    LQ_HIP(hipGetDevice(&dev));
    const size_t sz = BlockCache::round_size(bytes);
    if (void* p = cache().take(dev, sz, stream)) {
        *d_ptr = p;
        return LQ_OK;
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
    cache().add_live(p, dev, sz);
    *d_ptr = p;
    return LQ_OK;
}

int lq_malloc(void** d_ptr, size_t bytes) { return lq_malloc_async(d_ptr, bytes, nullptr); }

int lq_free_async(void* d_ptr, void* stream) {
    if (!d_ptr) return LQ_OK;
    if (!cache().put(d_ptr, stream)) return set_error(LQ_ERR_INVALID, "lq_free: pointer not from lq_malloc");
    return LQ_OK;
}

int lq_free(void* d_ptr) { return lq_free_async(d_ptr, nullptr); }

int lq_record_stream(void* d_ptr, void* stream) {
    LQ_REQUIRE(d_ptr, "lq_record_stream: NULL pointer");
    if (!cache().record_use(d_ptr, stream)) return set_error(LQ_ERR_INVALID, "lq_record_stream: pointer not from lq_malloc");
    return LQ_OK;
}

int lq_empty_cache(void) {
    const auto victims = cache().drain();
    if (!victims.empty()) {
        int cur = 0;
        LQ_HIP(hipGetDevice(&cur));
        for (auto& v : victims) {
            LQ_HIP(hipSetDevice(v.first));
            LQ_HIP(hipFree(v.second));  // hipFree waits for the device's pending work
        }
        LQ_HIP(hipSetDevice(cur));
    }
    std::vector<hipEvent_t> events;
    {
        std::lock_guard<std::mutex> g(g_event_mu);
        events.swap(g_event_pool);
    }
    for (hipEvent_t ev : events) (void)hipEventDestroy(ev);
    return LQ_OK;
}

int lq_memory_stats(size_t* allocated, size_t* cached) {
    cache().stats(allocated, cached);
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

// The streaming-read floor: every 16-byte chunk of src loaded once (4 per thread, 64 B
// apart in a wave's 1 KB-per-load pattern), XOR-folded, and written only if it equals a value
// the caller chooses never to match -- so the loads stay and nothing is stored.
constexpr int RF_THREADS = 256, RF_PER = 4;
typedef uint32_t rf_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(RF_THREADS) void lq_read_floor_kernel(const rf_u32x4* __restrict__ src, size_t n16,
                                                                    uint32_t never, uint32_t* sink) {
    const size_t base = (size_t)blockIdx.x * RF_THREADS * RF_PER + threadIdx.x;
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < RF_PER; ++u) {
        const size_t i = base + (size_t)u * RF_THREADS;
        if (i < n16) {
            const rf_u32x4 v = __builtin_nontemporal_load(src + i);
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (acc == never) sink[threadIdx.x] = acc;
}

namespace lq {
// A captured graph and its executable form, owned together by an lq_graph_* handle.
struct CapturedGraph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};
}  // namespace lq

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

int lq_read_floor(const void* d_src, size_t bytes, uint32_t never, uint32_t* d_sink, void* stream) {
    if (bytes == 0) return LQ_OK;
    LQ_REQUIRE(d_src && d_sink, "lq_read_floor: NULL pointer");
    LQ_REQUIRE(bytes % 16 == 0 && ((uintptr_t)d_src & 15) == 0,
               "lq_read_floor: bytes and the source address must be multiples of 16");
    const size_t n16 = bytes / 16, per = (size_t)RF_THREADS * RF_PER;
    const size_t blocks = (n16 + per - 1) / per;
    LQ_REQUIRE(blocks <= 0x7fffffff, "lq_read_floor: too many bytes for one launch");
    hipLaunchKernelGGL(lq_read_floor_kernel, dim3((unsigned)blocks), dim3(RF_THREADS), 0, as_stream(stream),
                       (const rf_u32x4*)d_src, n16, never, d_sink);
    return launch_status("lq_read_floor");
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
    // blocks that recorded a use on this stream must not record an event on it once it is
    // gone: wait for its work, then drop it from their records
    LQ_HIP(hipStreamSynchronize(as_stream(stream)));
    cache().forget_stream(stream);
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
    if (err != hipSuccess) {
        (void)hipGraphDestroy(g);
        return check_hip(err, "hipGraphInstantiate");
    }
    // The handle owns both graphs: the captured one stays alive for as long as its
    // executable form (a tool that maps an executable graph's nodes back to the captured
    // graph at launch, such as a tracing profiler, reads it), and both go in
    // lq_graph_destroy.
    *graph_exec = new CapturedGraph{g, e};
    return LQ_OK;
}

int lq_graph_launch(void* graph_exec, void* stream) {
    LQ_REQUIRE(graph_exec, "lq_graph_launch: NULL graph");
    LQ_HIP(hipGraphLaunch(static_cast<CapturedGraph*>(graph_exec)->exec, (hipStream_t)stream));
    return LQ_OK;
}

int lq_graph_destroy(void* graph_exec) {
    if (!graph_exec) return LQ_OK;
    CapturedGraph* cg = static_cast<CapturedGraph*>(graph_exec);
    const hipError_t e1 = hipGraphExecDestroy(cg->exec);
    const hipError_t e2 = hipGraphDestroy(cg->graph);
    delete cg;
    LQ_HIP(e1);
    LQ_HIP(e2);
    return LQ_OK;
}

}  // extern "C"
