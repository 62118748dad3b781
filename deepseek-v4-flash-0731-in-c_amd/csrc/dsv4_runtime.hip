// dsv4_runtime.hip - error reporting and small device-memory helpers of the
// C ABI (the host C layer and the Python tests use these instead of linking
// the HIP runtime themselves).
#include <stdarg.h>
#include <stdio.h>

#include "dsv4_gpu_internal.h"

static thread_local char g_err[512];

extern "C" {

int dsv4g_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int dsv4g_check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return dsv4g_fail(DSV4G_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

const char *dsv4g_last_error(void) { return g_err; }

const char *dsv4g_version(void) { return "dsv4-moe-gfx950 " DSV4G_VERSION; }

int dsv4g_device_count(int *count) {
  DSV4G_HIP(hipGetDeviceCount(count));
  return 0;
}

int dsv4g_malloc(void **ptr, size_t bytes) {
  *ptr = NULL;
  DSV4G_HIP(hipMalloc(ptr, bytes ? bytes : 1));
  return 0;
}

int dsv4g_free(void *ptr) {
  if (ptr) DSV4G_HIP(hipFree(ptr));
  return 0;
}

int dsv4g_host_malloc(void **ptr, size_t bytes) {
  *ptr = NULL;
  DSV4G_HIP(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault));
  return 0;
}

int dsv4g_host_free(void *ptr) {
  if (ptr) DSV4G_HIP(hipHostFree(ptr));
  return 0;
}

int dsv4g_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream) {
  DSV4G_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
  return 0;
}

int dsv4g_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
  DSV4G_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
  return 0;
}

int dsv4g_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
  DSV4G_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
  DSV4G_HIP(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

int dsv4g_stream_sync(void *stream) {
  DSV4G_HIP(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

}  // extern "C"
