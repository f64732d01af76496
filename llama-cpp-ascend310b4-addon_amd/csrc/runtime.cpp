// runtime.cpp -- error reporting and device plumbing of the C ABI.
#include "mi_common.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace mi {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char *what) {
    set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return (int)e;
}

}  // namespace mi

using mi::hip_fail;

#define HIP_RET(expr, what)                            \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

extern "C" {

const char *mi_last_error(void) { return mi::g_err; }

int mi_device_count(int *count) {
    if (!count) return MI_ERR_ARG;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        mi::set_error("hipGetDeviceCount: %s", hipGetErrorString(e));
        return MI_ERR_NODEVICE;
    }
    *count = n;
    return n > 0 ? MI_OK : MI_ERR_NODEVICE;
}

int mi_set_device(int device) {
    HIP_RET(hipSetDevice(device), "hipSetDevice");
    return MI_OK;
}

int mi_device_name(int device, char *buf, size_t len) {
    hipDeviceProp_t p;
    HIP_RET(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
    snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return MI_OK;
}

int mi_malloc(void **ptr, size_t bytes) {
    if (!ptr) return MI_ERR_ARG;
    HIP_RET(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
    return MI_OK;
}

int mi_free(void *ptr) {
    HIP_RET(hipFree(ptr), "hipFree");
    return MI_OK;
}

int mi_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    HIP_RET(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync H2D");
    HIP_RET(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return MI_OK;
}

int mi_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    HIP_RET(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync D2H");
    HIP_RET(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return MI_OK;
}

int mi_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
    HIP_RET(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync D2D");
    return MI_OK;
}

int mi_memset(void *dst, int value, size_t bytes, void *stream) {
    HIP_RET(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream), "hipMemsetAsync");
    return MI_OK;
}

int mi_stream_create(void **stream) {
    hipStream_t s;
    HIP_RET(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = (void *)s;
    return MI_OK;
}

int mi_stream_destroy(void *stream) {
    HIP_RET(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    return MI_OK;
}

int mi_stream_sync(void *stream) {
    HIP_RET(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return MI_OK;
}

int mi_device_sync(void) {
    HIP_RET(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return MI_OK;
}

int mi_event_create(void **event) {
    hipEvent_t e;
    HIP_RET(hipEventCreate(&e), "hipEventCreate");
    *event = (void *)e;
    return MI_OK;
}

int mi_event_destroy(void *event) {
    HIP_RET(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
    return MI_OK;
}

int mi_event_record(void *event, void *stream) {
    HIP_RET(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
    return MI_OK;
}

int mi_event_elapsed_ms(float *ms, void *start, void *stop) {
    HIP_RET(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize");
    HIP_RET(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime");
    return MI_OK;
}

int mi_graph_capture_begin(void *stream) {
    HIP_RET(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return MI_OK;
}

int mi_graph_capture_end(void *stream, void **graph_exec) {
    hipGraph_t g = nullptr;
    HIP_RET(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph_exec = (void *)ge;
    return MI_OK;
}

int mi_graph_launch(void *graph_exec, void *stream) {
    HIP_RET(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream), "hipGraphLaunch");
    return MI_OK;
}

int mi_graph_destroy(void *graph_exec) {
    HIP_RET(hipGraphExecDestroy((hipGraphExec_t)graph_exec), "hipGraphExecDestroy");
    return MI_OK;
}

}  // extern "C"
