// runtime.hip -- device, stream, memory and event entry points of the C launch ABI.
//
// Replaces the reference's GPUManager (Mods/GPUManager.h:26-58, GPUManager.h:540-594):
// instead of one MTLDevice with a thread-local command buffer / encoder, one HIP device with
// one stream per host thread.  Launches are asynchronous; mx_hip_sync() is the
// commit-and-wait (GPUManager.h:558-562) and, unlike the reference, checks for errors.
#include "common.hpp"

#include <atomic>
#include <mutex>
#include <unordered_map>
#include <thread>

namespace mx {

namespace {
thread_local std::string t_last_error;
std::atomic<int> g_device{-1};
std::mutex g_streams_mu;
std::unordered_map<std::thread::id, hipStream_t> g_streams;
}  // namespace

void set_error(const std::string& msg) { t_last_error = msg; }

int fail(int status, const std::string& msg) {
    t_last_error = msg;
    return status;
}

int hip_fail(hipError_t err, const char* what) {
    t_last_error = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
    return MX_ERR_HIP;
}

// Each host thread gets its own stream, created lazily with default priority, as the
// reference gives each thread its own command buffer (GPUManager.h:57-58).
static int thread_stream(hipStream_t* out) {
    int dev = g_device.load();
    if (dev < 0) return fail(MX_ERR_NOT_INITIALIZED, "mx_hip_init() was not called");
    std::lock_guard<std::mutex> lk(g_streams_mu);
    auto it = g_streams.find(std::this_thread::get_id());
    if (it != g_streams.end()) { *out = it->second; return MX_OK; }
    MX_HIP(hipSetDevice(dev));
    hipStream_t s = nullptr;
    MX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    g_streams.emplace(std::this_thread::get_id(), s);
    *out = s;
    return MX_OK;
}

bool resolve_stream(void* in, hipStream_t* out) {
    if (in) { *out = (hipStream_t)in; return g_device.load() >= 0 || (fail(MX_ERR_NOT_INITIALIZED, "mx_hip_init() was not called"), false); }
    return thread_stream(out) == MX_OK;
}

// Device allocations made through the ABI (mx_hip_alloc) and frees, counted so a caller can
// check that a phase allocated nothing (the reference's "no buffer is built during EXECUTE",
// .agents/MemoryManagement.md:335).  No kernel entry point allocates.
namespace {
std::atomic<uint64_t> g_allocs{0}, g_frees{0};
}  // namespace

// Looks up this device's address of the fixed scratch of mx_launch_reduce_noalloc (reduce.hip),
// once per device, with the device current.
int reduce_noalloc_setup(int device);

}  // namespace mx

using namespace mx;

extern "C" {

const char* mx_last_error(void) { return t_last_error.c_str(); }

const char* mx_version(void) { return "matrix_amd 0.1 (gfx950)"; }

int mx_hip_device_count(int* count) {
    if (!count) return fail(MX_ERR_INVALID_ARG, "mx_hip_device_count: null pointer");
    MX_HIP(hipGetDeviceCount(count));
    return MX_OK;
}

int mx_hip_init(int device) {
    int n = 0;
    MX_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return fail(MX_ERR_INVALID_ARG, "mx_hip_init: device " + std::to_string(device) +
                                            " out of range (" + std::to_string(n) + " devices)");
    MX_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    MX_HIP(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail(MX_ERR_UNSUPPORTED, "mx_hip_init: kernels are built for gfx950, device is " + arch);
    const int rc = reduce_noalloc_setup(device);
    if (rc != MX_OK) return rc;
    g_device.store(device);
    return MX_OK;
}

int mx_hip_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_streams_mu);
    int rc = MX_OK;
    for (auto& kv : g_streams) {
        hipError_t e = hipStreamSynchronize(kv.second);
        if (e != hipSuccess && rc == MX_OK) rc = hip_fail(e, "hipStreamSynchronize");
        (void)hipStreamDestroy(kv.second);
    }
    g_streams.clear();
    g_device.store(-1);
    return rc;
}

int mx_hip_alloc(size_t bytes, void** dptr) {
    if (!dptr) return fail(MX_ERR_INVALID_ARG, "mx_hip_alloc: null out pointer");
    if (g_device.load() < 0) return fail(MX_ERR_NOT_INITIALIZED, "mx_hip_init() was not called");
    *dptr = nullptr;
    if (bytes == 0) return MX_OK;
    MX_HIP(hipMalloc(dptr, bytes));
    g_allocs.fetch_add(1, std::memory_order_relaxed);
    return MX_OK;
}

int mx_hip_free(void* dptr) {
    if (!dptr) return MX_OK;
    MX_HIP(hipFree(dptr));
    g_frees.fetch_add(1, std::memory_order_relaxed);
    return MX_OK;
}

int mx_hip_alloc_stats(uint64_t* allocs, uint64_t* frees) {
    if (!allocs || !frees) return fail(MX_ERR_INVALID_ARG, "mx_hip_alloc_stats: null pointer");
    *allocs = g_allocs.load(std::memory_order_relaxed);
    *frees = g_frees.load(std::memory_order_relaxed);
    return MX_OK;
}

static int copy_impl(void* dst, const void* src, size_t bytes, void* stream, hipMemcpyKind kind) {
    if (bytes == 0) return MX_OK;
    if (!dst || !src) return fail(MX_ERR_INVALID_ARG, "mx_hip copy: null pointer");
    hipStream_t s;
    if (!resolve_stream(stream, &s)) return MX_ERR_NOT_INITIALIZED;
    MX_HIP(hipMemcpyAsync(dst, src, bytes, kind, s));
    // Host buffers are pageable: finish the copy before handing them back to the caller.
    if (kind != hipMemcpyDeviceToDevice) MX_HIP(hipStreamSynchronize(s));
    return MX_OK;
}

int mx_hip_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy_impl(dst, src, bytes, stream, hipMemcpyHostToDevice);
}
int mx_hip_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return copy_impl(dst, src, bytes, stream, hipMemcpyDeviceToHost);
}
int mx_hip_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy_impl(dst, src, bytes, stream, hipMemcpyDeviceToDevice);
}

int mx_hip_memset(void* dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return MX_OK;
    if (!dst) return fail(MX_ERR_INVALID_ARG, "mx_hip_memset: null pointer");
    hipStream_t s;
    if (!resolve_stream(stream, &s)) return MX_ERR_NOT_INITIALIZED;
    MX_HIP(hipMemsetAsync(dst, value, bytes, s));
    return MX_OK;
}

int mx_hip_stream_for_thread(void** stream) {
    if (!stream) return fail(MX_ERR_INVALID_ARG, "mx_hip_stream_for_thread: null pointer");
    hipStream_t s;
    int rc = thread_stream(&s);
    if (rc != MX_OK) return rc;
    *stream = (void*)s;
    return MX_OK;
}

// Extra streams for callers that run independent nodes concurrently (no counterpart in the
// reference, whose encoder is one in-order queue per thread).  Default priority, non-blocking.
int mx_hip_stream_create(void** stream) {
    if (!stream) return fail(MX_ERR_INVALID_ARG, "mx_hip_stream_create: null pointer");
    if (g_device.load() < 0) return fail(MX_ERR_NOT_INITIALIZED, "mx_hip_init() was not called");
    hipStream_t s = nullptr;
    MX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = (void*)s;
    return MX_OK;
}

int mx_hip_stream_destroy(void* stream) {
    if (!stream) return MX_OK;
    MX_HIP(hipStreamDestroy((hipStream_t)stream));
    return MX_OK;
}

int mx_hip_stream_wait_event(void* stream, void* event) {
    if (!event) return fail(MX_ERR_INVALID_ARG, "mx_hip_stream_wait_event: null event");
    hipStream_t s;
    if (!resolve_stream(stream, &s)) return MX_ERR_NOT_INITIALIZED;
    MX_HIP(hipStreamWaitEvent(s, (hipEvent_t)event, 0));
    return MX_OK;
}

int mx_hip_sync(void* stream) {
    hipStream_t s;
    if (!resolve_stream(stream, &s)) return MX_ERR_NOT_INITIALIZED;
    MX_HIP(hipStreamSynchronize(s));
    MX_HIP(hipGetLastError());
    return MX_OK;
}

int mx_hip_event_create(void** event) {
    if (!event) return fail(MX_ERR_INVALID_ARG, "mx_hip_event_create: null pointer");
    hipEvent_t e;
    MX_HIP(hipEventCreate(&e));
    *event = (void*)e;
    return MX_OK;
}

int mx_hip_event_destroy(void* event) {
    if (!event) return MX_OK;
    MX_HIP(hipEventDestroy((hipEvent_t)event));
    return MX_OK;
}

int mx_hip_event_record(void* event, void* stream) {
    if (!event) return fail(MX_ERR_INVALID_ARG, "mx_hip_event_record: null event");
    hipStream_t s;
    if (!resolve_stream(stream, &s)) return MX_ERR_NOT_INITIALIZED;
    MX_HIP(hipEventRecord((hipEvent_t)event, s));
    return MX_OK;
}

int mx_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (!start || !stop || !ms) return fail(MX_ERR_INVALID_ARG, "mx_hip_event_elapsed_ms: null pointer");
    MX_HIP(hipEventSynchronize((hipEvent_t)stop));
    MX_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return MX_OK;
}

}  // extern "C"
