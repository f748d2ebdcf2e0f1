// runtime.hip - the thin C-ABI over the HIP runtime (include/snx_hip.h) and
// the library's thread-local error text.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "snx_hip.h"
#include "sneppx_qlinear.h"
#include "../snx_internal.h"
#include "../ws_registry.h"

namespace {
thread_local char g_err[512];

int check(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    snx_set_error("%s: %s", what, hipGetErrorString(e));
    return -1;
}

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// zero fill of a new zeroed workspace (a kernel, not a memset, so that a
// caller capturing the stream into a graph records an ordinary kernel node)
__global__ void __launch_bounds__(256) k_fill_zero_u32(uint32_t* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}
}  // namespace

// The library's internal scratch (split-K partials, prepared activations,
// gathers) comes from per-thread workspaces keyed by (device, stream, slot):
// ws_registry.h holds the rules (no sharing between threads, stream-ordered
// growth, buffers of ended threads adopted by later ones).  Here it gets the
// device side: the stream-ordered pool, and a fill kernel for zeroed
// buffers.
namespace {
void* ws_alloc(size_t bytes, void* stream, bool zeroed) {
    void* p = nullptr;
    if (snx_hip_malloc_async(&p, bytes, stream)) return nullptr;
    if (zeroed) {
        const size_t n = bytes / 4;
        k_fill_zero_u32<<<(unsigned)(n / 256 < 1024 ? (n + 255) / 256 : 1024), 256, 0, S(stream)>>>(
            static_cast<uint32_t*>(p), n);
        if (snx_launch_check("k_fill_zero_u32")) {
            (void)hipFreeAsync(p, S(stream));
            return nullptr;
        }
    }
    return p;
}

void ws_release(void* p, void* stream) { (void)hipFreeAsync(p, S(stream)); }

void* workspace(size_t bytes, int slot, void* stream, bool zeroed) {
    static std::once_flag once;
    std::call_once(once, [] { snx_ws::init(ws_alloc, ws_release); });
    int dev = 0;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    return snx_ws::get(dev, stream, slot, bytes, zeroed);
}
}  // namespace

extern "C" {

void snx_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

void snx_clear_error(void) { g_err[0] = 0; }

const char* SNEPPX_qlinear_last_error(void) { return g_err; }

int snx_launch_check(const char* kernel) {
    return check(hipGetLastError(), kernel);
}

int snx_hip_device_count(int* count) {
    if (!count) return -1;
    return check(hipGetDeviceCount(count), "hipGetDeviceCount");
}

int snx_hip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return -1;
    *ptr = nullptr;
    if (bytes == 0) bytes = 1;
    return check(hipMalloc(ptr, bytes), "hipMalloc");
}

int snx_hip_free(void* ptr) { return ptr ? check(hipFree(ptr), "hipFree") : 0; }

// The library's workspaces come from the device's default stream-ordered
// pool.  With the pool's default release threshold (0) its memory goes back
// to the driver at every synchronisation, so each call would map fresh
// memory; keeping it (threshold = max) makes a workspace allocation a cheap
// pool operation.  Set once per device.
static int keep_pool_memory() {
    static std::atomic<uint64_t> done{0};   // bit d: device d configured
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    const uint64_t bit = 1ull << dev;
    if (done.load(std::memory_order_acquire) & bit) return 0;
    hipMemPool_t pool;
    if (hipDeviceGetDefaultMemPool(&pool, dev) == hipSuccess) {
        uint64_t keep = UINT64_MAX;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
    }
    done.fetch_or(bit, std::memory_order_acq_rel);
    return 0;
}

int snx_hip_malloc_async(void** ptr, size_t bytes, void* stream) {
    if (!ptr) return -1;
    *ptr = nullptr;
    if (bytes == 0) bytes = 1;
    keep_pool_memory();
    return check(hipMallocAsync(ptr, bytes, S(stream)), "hipMallocAsync");
}

int snx_hip_free_async(void* ptr, void* stream) {
    return ptr ? check(hipFreeAsync(ptr, S(stream)), "hipFreeAsync") : 0;
}

void* snx_workspace(size_t bytes, int slot, void* stream) { return workspace(bytes, slot, stream, false); }

// As snx_workspace, with a new buffer zero-filled (stream-ordered) when it is
// taken; for data the caller's kernels return to zero before they end (the
// split GEMM's arrival counters).
void* snx_workspace_zeroed(size_t bytes, int slot, void* stream) { return workspace(bytes, slot, stream, true); }

// Frees (stream-ordered) this thread's workspaces on `stream` and those that
// ended threads left on it, for a caller about to destroy that stream.
void snx_release_workspaces(void* stream) { snx_ws::release_stream(stream); }

int SNEPPX_qlinear_release_workspaces(SNEPPXStream stream) {
    snx_ws::release_stream(stream);
    return 0;
}

// Workspaces currently held (by live threads and left by ended ones).
long snx_workspace_count(void) { return snx_ws::live(); }

int snx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(stream)), "hipMemcpyAsync(H2D)");
}

int snx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(stream)), "hipMemcpyAsync(D2H)");
}

int snx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(stream)), "hipMemcpyAsync(D2D)");
}

int snx_hip_stream_create(void** stream) {
    if (!stream) return -1;
    hipStream_t s = nullptr;
    if (check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return -1;
    *stream = s;
    return 0;
}

int snx_hip_stream_destroy(void* stream) {
    return stream ? check(hipStreamDestroy(S(stream)), "hipStreamDestroy") : 0;
}

int snx_hip_stream_sync(void* stream) { return check(hipStreamSynchronize(S(stream)), "hipStreamSynchronize"); }

int snx_hip_device_sync(void) { return check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int snx_hip_event_create(void** event) {
    if (!event) return -1;
    hipEvent_t e = nullptr;
    if (check(hipEventCreate(&e), "hipEventCreate")) return -1;
    *event = e;
    return 0;
}

int snx_hip_event_destroy(void* event) {
    return event ? check(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy") : 0;
}

int snx_hip_event_record(void* event, void* stream) {
    return check(hipEventRecord(reinterpret_cast<hipEvent_t>(event), S(stream)), "hipEventRecord");
}

int snx_hip_event_sync(void* event) {
    return check(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
}

int snx_hip_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms) return -1;
    return check(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                     reinterpret_cast<hipEvent_t>(stop)), "hipEventElapsedTime");
}

int snx_hip_device_info(char* arch, size_t arch_len, int* cu_count, int* clock_khz) {
    int dev = 0;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return -1;
    hipDeviceProp_t p;
    if (check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties")) return -1;
    if (arch && arch_len) {
        strncpy(arch, p.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (cu_count) *cu_count = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    return 0;
}

int snx_hip_stream_begin_capture(void* stream) {
    return check(hipStreamBeginCapture(S(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

int snx_hip_stream_end_capture(void* stream, void** graph_exec) {
    if (!graph_exec) return -1;
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    if (check(hipStreamEndCapture(S(stream), &g), "hipStreamEndCapture")) return -1;
    hipGraphExec_t e = nullptr;
    const int rc = check(hipGraphInstantiate(&e, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc) return -1;
    *graph_exec = e;
    return 0;
}

int snx_hip_graph_launch(void* graph_exec, void* stream) {
    return check(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), S(stream)), "hipGraphLaunch");
}

int snx_hip_graph_destroy(void* graph_exec) {
    return graph_exec ? check(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)),
                              "hipGraphExecDestroy")
                      : 0;
}

}  // extern "C"
