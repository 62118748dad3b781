// dsv4_gpu_internal.h - definitions shared by the HIP translation units of
// libdsv4_gpu.so (not part of the public C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "dsv4_gpu.h"

// FP4 exact GEMV: float2 LDS entries per workgroup (rows per tile =
// FP4_LDS_ENTRIES / next_pow2(in / 32), at most 256).
#define FP4_LDS_ENTRIES 4096
// FP8 exact GEMV: rows per workgroup tile and widest supported input.
#define FP8_TR 16
#define FP8_MAX_IN 8192

// Arguments of the exact FP4/FP8 GEMV kernels. Matrix m (0/1) is picked by
// blockIdx.z, token vector b by blockIdx.y (strides in elements).
struct GemvArgs {
  float *y[2];
  const uint8_t *W[2];
  const uint8_t *S[2];
  const float *qx;
  const float *qscale;
  size_t y_stride, qx_stride, qs_stride;
  int in, rows, round_out;
  // paired FP4 tiles with the SwiGLU epilogue (swi_y set): swi_y[r] =
  // bf16(swiglu(gate[r], up[r]) * swi_w) instead of the two rows
  float *swi_y;
  const float *swi_w;  // device pointer to the route weight (null: 1)
  float swi_limit;
  int np;  // FP4 passes per tile (0: chosen by the launcher)
};

// Largest expert count of the router kernels.
#define ROUTER_MAX_EXPERTS 1024

extern "C" {
int dsv4g_layer_ok(const DSV4GLayer *L, const char *who);
int dsv4g_fail(int code, const char *fmt, ...);
int dsv4g_check_launch(const char *what);
int dsv4g_launch_gemv_fp4(const GemvArgs *a, int nvec, int nmat, void *stream);
int dsv4g_launch_gemv_fp8(const GemvArgs *a, int nvec, int nmat, void *stream);
unsigned *dsv4g_decode_status_word(void *workspace);
}

#define DSV4G_TRY(expr)            \
  do {                             \
    int _rc = (expr);              \
    if (_rc) return _rc;           \
  } while (0)

#define DSV4G_HIP(expr)                                                          \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess)                                                        \
      return dsv4g_fail(DSV4G_EHIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)
