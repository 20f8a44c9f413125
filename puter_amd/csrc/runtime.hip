// Runtime side of the C ABI: error reporting, device selection, memory and
// streams.  Replaces the reference's CUDA bridge context/runtime
// (device/cuda/internal/bridge/context.c, runtime.c) with plain HIP calls; the
// memory entry points back the tensor.Backend Upload/Download/Close of a cgo
// `device/hip` package (reference memory backend: device/cuda/backend.go:101-234).
#include <cstdarg>

#include "common.hpp"

namespace puter {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PUTER_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return PUTER_OK;
}

static int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return PUTER_OK;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
        return fail(PUTER_ERR_UNAVAILABLE, "%s: %s", what, hipGetErrorString(e));
    return fail(PUTER_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace puter

using namespace puter;

extern "C" {

const char *puter_hip_last_error(void) { return g_last_error; }

int puter_hip_version(void) { return 1; }

int puter_hip_device_count(int *count) {
    if (!count) return fail(PUTER_ERR_NIL, "device_count: nil out pointer");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) {
        *count = 0;
        return hip_status(e, "hipGetDeviceCount");
    }
    return PUTER_OK;
}

int puter_hip_set_device(int device) { return hip_status(hipSetDevice(device), "hipSetDevice"); }

int puter_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return fail(PUTER_ERR_NIL, "malloc: nil out pointer");
    *ptr = nullptr;
    if (bytes == 0) return PUTER_OK;
    return hip_status(hipMalloc(ptr, bytes), "hipMalloc");
}

int puter_hip_free(void *ptr) {
    if (!ptr) return PUTER_OK;
    return hip_status(hipFree(ptr), "hipFree");
}

int puter_hip_memcpy_htod(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return PUTER_OK;
    if (!dst || !src) return fail(PUTER_ERR_NIL, "memcpy_htod: nil buffer");
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
                      "hipMemcpyAsync(HtoD)");
}

int puter_hip_memcpy_dtoh(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return PUTER_OK;
    if (!dst || !src) return fail(PUTER_ERR_NIL, "memcpy_dtoh: nil buffer");
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                      "hipMemcpyAsync(DtoH)");
}

int puter_hip_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return PUTER_OK;
    if (!dst || !src) return fail(PUTER_ERR_NIL, "memcpy_dtod: nil buffer");
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)),
                      "hipMemcpyAsync(DtoD)");
}

int puter_hip_stream_create(void **stream) {
    if (!stream) return fail(PUTER_ERR_NIL, "stream_create: nil out pointer");
    hipStream_t s = nullptr;
    int rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return rc;
}

int puter_hip_stream_destroy(void *stream) {
    if (!stream) return PUTER_OK;
    return hip_status(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}

int puter_hip_stream_synchronize(void *stream) {
    return hip_status(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

}  // extern "C"
