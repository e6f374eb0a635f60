// The host runtime of the HIP backend: device selection, one library stream,
// device memory, pinned host staging, events, graph capture, and the device
// error word that kernels report bad input through.
//
// It plays the part of the reference's runtime plumbing around each generated
// kernel (runtime.py:167-301 loads a library, owns the arena and calls each
// kernel; pool.c is the executor the kernels run on). Here the executor is
// one HIP stream: every kernel entry point enqueues on it and returns, and
// nc_sync() is where the host waits and where a kernel's failure code (the
// reference's loopir.Fail, loopir.py:280-285) comes back.
#include "nc_common.h"

#include <stdio.h>
#include <string.h>

namespace {

int g_device = -1;
hipStream_t g_stream = nullptr;
int32_t *g_error = nullptr;          // device word: 0, or the first failure code
char g_message[512] = "";

int32_t record(hipError_t e, const char *what) {
    if (e == hipSuccess) return NC_OK;
    snprintf(g_message, sizeof g_message, "%s: %s", what, hipGetErrorString(e));
    return NC_LAUNCH_FAILED;
}

}  // namespace

namespace nc {
hipStream_t stream() { return g_stream; }
int device() { return g_device; }
int32_t *error_word() { return g_error; }
int32_t launched(const char *what) { return record(hipGetLastError(), what); }
void set_message(const char *text) { snprintf(g_message, sizeof g_message, "%s", text); }
}  // namespace nc

NC_EXPORT const char *nc_last_error(void) { return g_message; }

NC_EXPORT int32_t nc_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

NC_EXPORT int32_t nc_init(int32_t device) {
    if (g_device == device && g_stream) return NC_OK;
    if (g_device >= 0) {
        nc::set_message("nc_init: the library is already bound to another device");
        return NC_BAD_ARGS;
    }
    int32_t rc = record(hipSetDevice(device), "hipSetDevice");
    if (rc) return rc;
    rc = record(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc) return rc;
    rc = record(hipMalloc(&g_error, 256), "hipMalloc(error word)");
    if (rc) return rc;
    rc = record(hipMemset(g_error, 0, 256), "hipMemset(error word)");
    if (rc) return rc;
    rc = nc::attention_scratch_init(device);      // the no-allocation entry point's workspace address
    if (rc) return rc;
    g_device = device;
    return record(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

NC_EXPORT int32_t nc_device_info(char *name, int64_t name_len, int64_t *compute_units,
                                 int64_t *lds_bytes, int64_t *hbm_bytes, int64_t *clock_khz) {
    hipDeviceProp_t p;
    int32_t rc = record(hipGetDeviceProperties(&p, g_device < 0 ? 0 : g_device), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", p.gcnArchName);
    if (compute_units) *compute_units = p.multiProcessorCount;
    if (lds_bytes) *lds_bytes = (int64_t)p.maxSharedMemoryPerMultiProcessor;
    if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
    if (clock_khz) *clock_khz = p.clockRate;
    return NC_OK;
}

#ifndef NC_LIBRARY_DIGEST
#define NC_LIBRARY_DIGEST "unversioned"
#endif

// A hash of the library's sources and build flags (made by the build).
NC_EXPORT const char *nc_library_digest(void) { return NC_LIBRARY_DIGEST; }

// The HIP runtime and driver versions (hipRuntimeGetVersion, hipDriverGetVersion):
// part of the key under which tuned schedules are cached.
NC_EXPORT int32_t nc_runtime_version(int64_t *runtime, int64_t *driver) {
    int r = 0, d = 0;
    int32_t rc = record(hipRuntimeGetVersion(&r), "hipRuntimeGetVersion");
    if (rc) return rc;
    rc = record(hipDriverGetVersion(&d), "hipDriverGetVersion");
    if (rc) return rc;
    if (runtime) *runtime = r;
    if (driver) *driver = d;
    return NC_OK;
}

NC_EXPORT void *nc_malloc(int64_t bytes) {
    void *p = nullptr;
    if (bytes <= 0) bytes = 1;
    if (record(hipMalloc(&p, (size_t)bytes), "hipMalloc")) return nullptr;
    return p;
}

NC_EXPORT int32_t nc_free(void *p) { return p ? record(hipFree(p), "hipFree") : NC_OK; }

NC_EXPORT void *nc_host_malloc(int64_t bytes) {
    void *p = nullptr;
    if (bytes <= 0) bytes = 1;
    if (record(hipHostMalloc(&p, (size_t)bytes, hipHostMallocDefault), "hipHostMalloc")) return nullptr;
    return p;
}

NC_EXPORT int32_t nc_host_free(void *p) { return p ? record(hipHostFree(p), "hipHostFree") : NC_OK; }

// Copies are ordered on the library stream. The synchronous forms wait for
// the copy (and everything before it) to finish.
NC_EXPORT int32_t nc_memcpy_h2d(void *dst, const void *src, int64_t n) {
    int32_t rc = record(hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyHostToDevice, g_stream), "hipMemcpyAsync(h2d)");
    return rc ? rc : record(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

NC_EXPORT int32_t nc_memcpy_d2h(void *dst, const void *src, int64_t n) {
    int32_t rc = record(hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyDeviceToHost, g_stream), "hipMemcpyAsync(d2h)");
    return rc ? rc : record(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

NC_EXPORT int32_t nc_memcpy_h2d_async(void *dst, const void *src, int64_t n) {
    return record(hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyHostToDevice, g_stream), "hipMemcpyAsync(h2d)");
}

NC_EXPORT int32_t nc_memcpy_d2h_async(void *dst, const void *src, int64_t n) {
    return record(hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyDeviceToHost, g_stream), "hipMemcpyAsync(d2h)");
}

NC_EXPORT int32_t nc_memcpy_d2d(void *dst, const void *src, int64_t n) {
    return record(hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyDeviceToDevice, g_stream), "hipMemcpyAsync(d2d)");
}

// height rows of width bytes, each with its own pitch on either side (the KV
// cache's [layer, head] blocks): kind 1 host to device, 2 device to host.
// Ordered on the library stream; waits.
NC_EXPORT int32_t nc_memcpy_rows(void *dst, int64_t dst_pitch, const void *src, int64_t src_pitch, int64_t width,
                                 int64_t height, int32_t kind) {
    if (!dst || !src || width < 0 || height < 0 || width > dst_pitch || width > src_pitch || (kind != 1 && kind != 2)) {
        nc::set_message("nc_memcpy_rows: bad arguments");
        return NC_BAD_ARGS;
    }
    if (width == 0 || height == 0) return NC_OK;
    const hipMemcpyKind direction = kind == 1 ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    int32_t rc = record(hipMemcpy2DAsync(dst, (size_t)dst_pitch, src, (size_t)src_pitch, (size_t)width,
                                         (size_t)height, direction, g_stream), "hipMemcpy2DAsync");
    return rc ? rc : record(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

// Wait for the stream. Returns the first kernel failure code recorded since
// the last call (and clears it), NC_LAUNCH_FAILED on a runtime error, or 0.
NC_EXPORT int32_t nc_sync(void) {
    int32_t rc = record(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
    if (rc) return rc;
    int32_t code = 0;
    rc = record(hipMemcpy(&code, g_error, sizeof code, hipMemcpyDeviceToHost), "hipMemcpy(error word)");
    if (rc) return rc;
    if (code) {
        snprintf(g_message, sizeof g_message, "a kernel reported failure code %d", code);
        rc = record(hipMemset(g_error, 0, sizeof code), "hipMemset(error word)");
        if (rc) return rc;
    }
    return code;
}

NC_EXPORT void *nc_stream_handle(void) { return (void *)g_stream; }
NC_EXPORT void *nc_error_word(void) { return (void *)g_error; }

// -- events: kernel timing on the library stream ----------------------------

NC_EXPORT void *nc_event_create(void) {
    hipEvent_t e = nullptr;
    if (record(hipEventCreate(&e), "hipEventCreate")) return nullptr;
    return (void *)e;
}

NC_EXPORT int32_t nc_event_record(void *e) { return record(hipEventRecord((hipEvent_t)e, g_stream), "hipEventRecord"); }

NC_EXPORT int32_t nc_event_elapsed_ms(void *start, void *stop, float *ms) {
    int32_t rc = record(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize");
    return rc ? rc : record(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime");
}

NC_EXPORT int32_t nc_event_destroy(void *e) { return record(hipEventDestroy((hipEvent_t)e), "hipEventDestroy"); }

// -- graphs: a step's launches captured once and replayed --------------------

NC_EXPORT int32_t nc_capture_begin(void) {
    return record(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

// Ends capture and instantiates; *out receives the executable graph.
NC_EXPORT int32_t nc_capture_end(void **out) {
    hipGraph_t graph = nullptr;
    int32_t rc = record(hipStreamEndCapture(g_stream, &graph), "hipStreamEndCapture");
    if (rc) return rc;
    hipGraphExec_t exec = nullptr;
    rc = record(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    hipGraphDestroy(graph);
    if (rc) return rc;
    *out = (void *)exec;
    return NC_OK;
}

NC_EXPORT int32_t nc_graph_launch(void *exec) {
    return record(hipGraphLaunch((hipGraphExec_t)exec, g_stream), "hipGraphLaunch");
}

NC_EXPORT int32_t nc_graph_destroy(void *exec) {
    return record(hipGraphExecDestroy((hipGraphExec_t)exec), "hipGraphExecDestroy");
}
