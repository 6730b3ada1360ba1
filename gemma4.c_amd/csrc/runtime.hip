// runtime.hip -- library state: device, stream, errors, allocation helpers.
#include <stdarg.h>
#include <string.h>

#include "g4_internal.h"

namespace {
hipStream_t g_stream = nullptr;   // null = the device's default stream
int g_device = -1;
int g_cus = 0;
thread_local char g_err[512] = "";
}  // namespace

hipStream_t g4_stream() { return g_stream; }
int g4_num_cus() { return g_cus > 0 ? g_cus : 256; }

int g4_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int g4_hip_status(hipError_t e) {
    if (e == hipSuccess) return G4_OK;
    return g4_fail(G4_ERR_HIP, "HIP error %d: %s", (int)e, hipGetErrorString(e));
}

int g4_check_launch(const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return G4_OK;
    return g4_fail(G4_ERR_HIP, "launch of %s failed: %s", kernel, hipGetErrorString(e));
}

extern "C" const char* g4_last_error(void) { return g_err; }

extern "C" int g4_init(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return g4_fail(G4_ERR_NODEV, "no HIP device available");
    G4_CHECK_ARG(device >= 0 && device < n, "g4_init: device %d out of range (%d devices)", device, n);
    G4_HIP(hipSetDevice(device));
    g_device = device;
    hipDeviceProp_t p;
    G4_HIP(hipGetDeviceProperties(&p, device));
    g_cus = p.multiProcessorCount;
    return g4_attn_scratch_setup(device);
}

extern "C" int g4_device_info(int* cus, char* arch, int arch_len) {
    if (g_device < 0) return g4_fail(G4_ERR_STATE, "g4_device_info: g4_init not called");
    hipDeviceProp_t p;
    G4_HIP(hipGetDeviceProperties(&p, g_device));
    if (cus) *cus = p.multiProcessorCount;
    if (arch && arch_len > 0) snprintf(arch, (size_t)arch_len, "%s", p.gcnArchName);
    return G4_OK;
}

extern "C" int g4_set_stream(void* stream) {
    g_stream = (hipStream_t)stream;
    return G4_OK;
}
extern "C" void* g4_get_stream(void) { return (void*)g_stream; }

extern "C" int g4_sync(void) { return g4_hip_status(hipStreamSynchronize(g_stream)); }

extern "C" int g4_malloc(void** p, size_t bytes) {
    G4_CHECK_ARG(p, "g4_malloc: null out pointer");
    *p = nullptr;
    if (bytes == 0) return G4_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();   // an allocation failure is not a later launch's error
        return g4_fail(G4_ERR_NOMEM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    return G4_OK;
}
extern "C" int g4_free(void* p) {
    if (!p) return G4_OK;
    return g4_hip_status(hipFree(p));
}
extern "C" int g4_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    G4_CHECK_ARG(dst && src, "g4_memcpy_h2d: null pointer");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    return g4_hip_status(hipStreamSynchronize(g_stream));
}
extern "C" int g4_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    G4_CHECK_ARG(dst && src, "g4_memcpy_d2h: null pointer");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    return g4_hip_status(hipStreamSynchronize(g_stream));
}

// ---- timing helpers (HIP events on the library stream) -----------------------
extern "C" int g4_event_create(void** ev) {
    G4_CHECK_ARG(ev, "g4_event_create: null pointer");
    return g4_hip_status(hipEventCreate((hipEvent_t*)ev));
}
extern "C" int g4_event_destroy(void* ev) { return g4_hip_status(hipEventDestroy((hipEvent_t)ev)); }
extern "C" int g4_event_record(void* ev) { return g4_hip_status(hipEventRecord((hipEvent_t)ev, g_stream)); }
extern "C" int g4_event_elapsed_ms(void* start, void* stop, float* ms) {
    G4_CHECK_ARG(ms, "g4_event_elapsed_ms: null pointer");
    G4_HIP(hipEventSynchronize((hipEvent_t)stop));
    return g4_hip_status(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

extern "C" int g4_memcpy_h2d_async(void* dst, const void* src, size_t bytes) {
    G4_CHECK_ARG(dst && src, "g4_memcpy_h2d_async: null pointer");
    return g4_hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
}
extern "C" int g4_memcpy_d2h_async(void* dst, const void* src, size_t bytes) {
    G4_CHECK_ARG(dst && src, "g4_memcpy_d2h_async: null pointer");
    return g4_hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
}
extern "C" int g4_memcpy_d2d_async(void* dst, const void* src, size_t bytes) {
    G4_CHECK_ARG(dst && src, "g4_memcpy_d2d_async: null pointer");
    return g4_hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
}

// synchronous fill of device memory (set-up only; never inside a captured graph)
extern "C" int g4_memset(void* p, int value, size_t bytes) {
    G4_CHECK_ARG(p || !bytes, "g4_memset: null pointer");
    if (!bytes) return G4_OK;
    G4_HIP(hipMemsetAsync(p, value, bytes, g_stream));
    return g4_hip_status(hipStreamSynchronize(g_stream));
}
extern "C" int g4_host_alloc(void** p, size_t bytes) {
    G4_CHECK_ARG(p && bytes, "g4_host_alloc: bad arguments");
    return g4_hip_status(hipHostMalloc(p, bytes, hipHostMallocDefault));
}
extern "C" int g4_host_free(void* p) { return p ? g4_hip_status(hipHostFree(p)) : G4_OK; }

// ---- streams and graphs: a decode step is captured once and replayed ---------
extern "C" int g4_stream_create(void** s) {
    G4_CHECK_ARG(s, "g4_stream_create: null pointer");
    return g4_hip_status(hipStreamCreateWithFlags((hipStream_t*)s, hipStreamNonBlocking));
}
extern "C" int g4_stream_destroy(void* s) { return s ? g4_hip_status(hipStreamDestroy((hipStream_t)s)) : G4_OK; }

extern "C" int g4_graph_begin(void) {
    if (!g_stream) return g4_fail(G4_ERR_STATE, "g4_graph_begin: capture needs a created stream (g4_set_stream)");
    return g4_hip_status(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
}
extern "C" int g4_graph_end(void** exec) {
    G4_CHECK_ARG(exec, "g4_graph_end: null pointer");
    hipGraph_t g = nullptr;
    G4_HIP(hipStreamEndCapture(g_stream, &g));
    hipGraphExec_t e = nullptr;
    int rc = g4_hip_status(hipGraphInstantiate(&e, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *exec = (void*)e;
    return G4_OK;
}
extern "C" int g4_graph_launch(void* exec) {
    G4_CHECK_ARG(exec, "g4_graph_launch: null graph");
    return g4_hip_status(hipGraphLaunch((hipGraphExec_t)exec, g_stream));
}
extern "C" int g4_graph_destroy(void* exec) {
    return exec ? g4_hip_status(hipGraphExecDestroy((hipGraphExec_t)exec)) : G4_OK;
}
