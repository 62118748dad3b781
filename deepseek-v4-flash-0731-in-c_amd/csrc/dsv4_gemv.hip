// dsv4_gemv.hip - decode-side kernels of the quantized MoE expert path for
// gfx950: activation FP8 quantisation, FP4/FP8 block-scaled GEMVs whose
// results are bit-identical to the reference's scalar loop order, the BF16
// router GEMV, the float-scale public GEMVs, dequantisers and the
// synthetic-checkpoint quantisers.
// The bit-exact GEMV row tiles are in dsv4_tiles.h.
#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"
#include "dsv4_tiles.h"

using namespace dsv4;

namespace dsv4 {

// ============================================================ activation ==
// One wave per 128-element group (src/dsv4/dsv4_model.c:5580-5606).
// grid = (ceil(n/128), nvec); x/qx rows are n apart, qscale rows ceil(n/128).
__global__ __launch_bounds__(64) void k_quant_fp8_act(float *__restrict__ qx,
                                                      float *__restrict__ qscale,
                                                      const float *__restrict__ x,
                                                      int n) {
  const int g = blockIdx.x, lane = threadIdx.x;
  const size_t row = blockIdx.y;
  const float *xr = x + row * (size_t)n;
  float *qr = qx + row * (size_t)n;
  const int base = g * 128;
  const int i0 = base + lane, i1 = base + 64 + lane;
  const float a = i0 < n ? xr[i0] : 0.0f;
  const float b = i1 < n ? xr[i1] : 0.0f;
  const float amax = wave_max(fmaxf(fabsf(a), fabsf(b)));
  const float scale = act_scale(amax);
  const float inv = 1.0f / scale;
  if (lane == 0) qscale[row * (size_t)((n + 127) / 128) + g] = scale;
  if (i0 < n) qr[i0] = quant_e4m3(a, inv);
  if (i1 < n) qr[i1] = quant_e4m3(b, inv);
}

// ============================================================== dequant ==
// FP4: out[r][c] = e2m1(W[r][c]) * e8m0(S[r][c/32]) (exact product).
__global__ void k_dequant_fp4(float *__restrict__ out, const uint8_t *__restrict__ W,
                              const uint8_t *__restrict__ S, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  const int pcols = (cols + 1) / 2, gcols = (cols + 31) / 32;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / cols, c = i % cols;
    const uint32_t b = W[r * pcols + (c >> 1)];
    const uint32_t nib = (c & 1) ? (b >> 4) : (b & 15u);
    out[i] = e2m1_decode(nib) * e8m0(S[r * gcols + c / 32]);
  }
}

// FP8: out[r][c] = e4m3(W[r][c]) * e8m0(S[r/128][c/128]).
__global__ void k_dequant_fp8(float *__restrict__ out, const uint8_t *__restrict__ W,
                              const uint8_t *__restrict__ S, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  const int cb = (cols + 127) / 128;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / cols, c = i % cols;
    out[i] = e4m3_decode(W[i]) * e8m0(S[(r / 128) * cb + c / 128]);
  }
}

// Hardware-convert probes: the GEMVs decode with the gfx950 MX/OCP converts;
// these write their results for every code so the tests can pin them to the
// reference decode.
__global__ void k_probe_converts(float *__restrict__ fp4_out, float *__restrict__ fp8_out) {
  const uint32_t t = threadIdx.x;  // 0..255
  const uint32_t word = t | (t << 8) | (t << 16) | (t << 24);
  const float2 a = fp4x2<0>(word);
  fp4_out[2 * t] = a.x;
  fp4_out[2 * t + 1] = a.y;
  const float2 b = fp8x2<false>(word);
  fp8_out[t] = b.x;
}

// grid = (ceil(rows / tr), nvec, nmat). blockIdx.y selects a token vector
// (batch), blockIdx.z selects matrix 0/1 (pair).
__global__ __launch_bounds__(256) void k_gemv_fp4(GemvArgs a) {
  __shared__ float2 ps[FP4_LDS_ENTRIES + 256];
  const int m = blockIdx.z, b = blockIdx.y;
  const Fp4Geom q = fp4_geom(a.in);
  fp4_rows_exact(a.y[m] + (size_t)b * a.y_stride, a.qx + (size_t)b * a.qx_stride,
                 a.qscale + (size_t)b * a.qs_stride, a.W[m], a.S[m], a.in, a.rows,
                 blockIdx.x * q.tr, ps);
}

__global__ __launch_bounds__(256) void k_gemv_fp8(GemvArgs a) {
  __shared__ __align__(16) float xs[FP8_MAX_IN / 128 * 132];
  __shared__ float2 ps[FP8_TR * (FP8_MAX_IN / 128 + 1)];
  const int m = blockIdx.z, b = blockIdx.y;
  fp8_rows_exact(a.y[m] + (size_t)b * a.y_stride, a.qx + (size_t)b * a.qx_stride,
                 a.qscale + (size_t)b * a.qs_stride, a.W[m], a.S[m], a.in, a.rows,
                 blockIdx.x * FP8_TR, a.round_out, xs, ps);
}

// ======================================================== BF16 GEMV =====
// y[r] = the reference's column-order chain acc = fmaf(bf16(W[r][c]), x[c],
// acc) (src/dsv4/dsv4_model.c:298-303; its 8-row AVX2 path runs the same
// chain per row): one lane per (row, token), the row read 16 bytes at a
// time, x shared by the wave (one line per load). Bit-exact; the cost is
// one dependent fmaf per column.
__global__ __launch_bounds__(64) void k_gemv_bf16(float *__restrict__ y,
                                                  const float *__restrict__ x,
                                                  const uint16_t *__restrict__ W, int in,
                                                  int out, int round_out, size_t y_stride,
                                                  size_t x_stride) {
  const int row = blockIdx.x * 64 + threadIdx.x;
  const int b = blockIdx.y;
  if (row >= out) return;
  const float *xb = x + (size_t)b * x_stride;
  const uint16_t *wr = W + (size_t)row * in;
  float acc = 0.0f;
  int c = 0;
  if ((in & 7) == 0) {
    for (; c < in; c += 8) {
      const uint4 w = *reinterpret_cast<const uint4 *>(wr + c);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc = fmaf(u2f(wd[d] << 16), xb[c + 2 * d], acc);
        acc = fmaf(u2f(wd[d] & 0xFFFF0000u), xb[c + 2 * d + 1], acc);
      }
    }
  }
  for (; c < in; ++c) acc = fmaf(bf16_to_f32(wr[c]), xb[c], acc);
  y[(size_t)b * y_stride + row] = round_out ? bf16_round(acc) : acc;
}

// ============================================= public float-scale GEMVs ===
// dsv4_gemv_fp8 / dsv4_gemv_fp8_tbl (src/dsv4/dsv4_ops.c:176-239) and
// dsv4_gemv_fp4 (src/dsv4/dsv4_ops.c:249-284): one sequential chain per row,
// unfused (the reference builds with -ffp-contract=off), here one lane per
// row with the same expression and column order. Bit-exact.
// mode 0 (dsv4_gemv_fp8): acc += w * (x * s); mode 1 (_tbl): acc += (w * x) * s.
__global__ __launch_bounds__(64) void k_gemv_fp8_float(float *__restrict__ y,
                                                       const float *__restrict__ x,
                                                       const uint8_t *__restrict__ W,
                                                       const float *__restrict__ wscale, int in,
                                                       int rows, int block, int mode) {
  const int row = blockIdx.x * 64 + threadIdx.x;
  if (row >= rows) return;
  const int cblocks = (in + block - 1) / block;
  const float *srow = wscale + (size_t)(row / block) * cblocks;
  const uint8_t *wr = W + (size_t)row * in;
  float acc = 0.0f;
  for (int c = 0; c < in; ++c) {
    const float w = e4m3_decode(wr[c]);
    const float s = srow[c / block];
    acc += mode == 0 ? w * (x[c] * s) : (w * x[c]) * s;
  }
  y[row] = acc;
}

// acc += (w * (qx * qs)) * ws, columns in order
__global__ __launch_bounds__(64) void k_gemv_fp4_float(float *__restrict__ y,
                                                       const float *__restrict__ qx,
                                                       const float *__restrict__ qscale,
                                                       const uint8_t *__restrict__ W,
                                                       const float *__restrict__ wscale, int in,
                                                       int rows, int group) {
  const int row = blockIdx.x * 64 + threadIdx.x;
  if (row >= rows) return;
  const size_t pcols = (size_t)(in + 1) / 2, gcols = (size_t)(in + group - 1) / group;
  const uint8_t *wr = W + (size_t)row * pcols;
  const float *ws = wscale + (size_t)row * gcols;
  float acc = 0.0f;
  for (int c = 0; c < in; ++c) {
    const uint32_t b = wr[c >> 1];
    const float w = e2m1_decode((c & 1) ? (b >> 4) : (b & 15u));
    const float xd = qx[c] * qscale[c / 128];
    acc += (w * xd) * ws[c / group];
  }
  y[row] = acc;
}

// ================================================ synthetic quantisers ===
// Build checkpoints in the reference formats from fp32 weights. The rules
// are the reference's activation rules applied to weights: E8M0 scale
// 2^ceil(log2(amax/6)) per 32 (FP4, nearest E2M1 with ties to the even code,
// src/dsv4/dsv4_model.c:1420-1447) or 2^ceil(log2(amax/448)) per 128x128
// block (FP8), or the fp32 absmax/448 block scale of the public FP8 GEMV.
__device__ __forceinline__ uint32_t fp4_code(float q) {
  const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float a = fabsf(q);
  int best = 0;
  float bd = a;
  for (int k = 0; k < 8; ++k) {
    const float d = fabsf(a - mag[k]);
    if (d < bd) {
      bd = d;
      best = k;
    } else if (d == bd && (k & 1) == 0) {
      best = k;
    }
  }
  return (uint32_t)best | (q < 0.0f ? 8u : 0u);
}

__device__ __forceinline__ int pow2_ceil_exp(float r) {
  int e;
  const float m = frexpf(r, &e);
  if (m == 0.5f) e--;
  return e;
}

// One thread per (row, 32-group).
__global__ void k_quant_fp4_rows(uint8_t *__restrict__ packed, uint8_t *__restrict__ scales,
                                 const float *__restrict__ w, int rows, int cols) {
  const int gcols = cols / 32;
  const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (idx >= (size_t)rows * gcols) return;
  const size_t r = idx / gcols, g = idx % gcols;
  const float *wr = w + r * cols + g * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(wr[i]));
  const float floor_amax = 6.0f * 0x1p-126f;
  if (amax < floor_amax) amax = floor_amax;
  const int e = pow2_ceil_exp(amax * (1.0f / 6.0f));
  scales[idx] = (uint8_t)(e + 127);
  const float inv = 1.0f / ldexpf(1.0f, e);
  uint8_t *pr = packed + r * (cols / 2) + g * 16;
  for (int i = 0; i < 16; ++i) {
    float q0 = wr[2 * i] * inv, q1 = wr[2 * i + 1] * inv;
    q0 = fminf(fmaxf(q0, -6.0f), 6.0f);
    q1 = fminf(fmaxf(q1, -6.0f), 6.0f);
    pr[i] = (uint8_t)(fp4_code(q0) | (fp4_code(q1) << 4));
  }
}

// One workgroup per 128x128 block. mode 0: E8M0 scale codes (uint8);
// mode 1: fp32 absmax/448 scales.
__global__ __launch_bounds__(256) void k_quant_fp8_blocks(uint8_t *__restrict__ codes,
                                                          void *__restrict__ scales,
                                                          const float *__restrict__ w,
                                                          int rows, int cols, int mode) {
  __shared__ float red[4];
  const int cb = (cols + 127) / 128;
  const int br = blockIdx.x / cb, bc = blockIdx.x % cb;
  const int r0 = br * 128, c0 = bc * 128;
  const int r1 = min(r0 + 128, rows), c1 = min(c0 + 128, cols);
  float amax = 0.0f;
  for (int i = threadIdx.x; i < 128 * 128; i += 256) {
    const int r = r0 + i / 128, c = c0 + i % 128;
    if (r < r1 && c < c1) amax = fmaxf(amax, fabsf(w[(size_t)r * cols + c]));
  }
  amax = wave_max(amax);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float inv;
  bool divide = false;
  float s = 1.0f;
  if (mode == 0) {
    const float a = amax < 1e-4f ? 1e-4f : amax;
    const int e = pow2_ceil_exp(a * (1.0f / 448.0f));
    if (threadIdx.x == 0) reinterpret_cast<uint8_t *>(scales)[blockIdx.x] = (uint8_t)(e + 127);
    inv = 1.0f / ldexpf(1.0f, e);
  } else {
    s = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (threadIdx.x == 0) reinterpret_cast<float *>(scales)[blockIdx.x] = s;
    inv = 0.0f;
    divide = true;
  }
  for (int i = threadIdx.x; i < 128 * 128; i += 256) {
    const int r = r0 + i / 128, c = c0 + i % 128;
    if (r < r1 && c < c1) {
      const float v = w[(size_t)r * cols + c];
      float q = divide ? v / s : v * inv;
      if (q > 448.0f) q = 448.0f;
      else if (q < -448.0f) q = -448.0f;
      codes[(size_t)r * cols + c] = (uint8_t)e4m3_code(round_e4m3(q));
    }
  }
}

}  // namespace dsv4

// ============================================================ C-ABI =====
using namespace dsv4;

extern "C" {

int dsv4g_quant_fp8_act(float *qx, float *qscale, const float *x, int n, int nvec,
                        void *stream) {
  if (n <= 0 || nvec <= 0) return dsv4g_fail(DSV4G_EINVAL, "quant_fp8_act: bad size");
  dim3 grid((n + 127) / 128, nvec);
  hipLaunchKernelGGL(k_quant_fp8_act, grid, dim3(64), 0, (hipStream_t)stream, qx, qscale,
                     x, n);
  return dsv4g_check_launch("quant_fp8_act");
}

int dsv4g_dequant_fp4(float *out, const uint8_t *W, const uint8_t *S, int rows, int cols,
                      void *stream) {
  hipLaunchKernelGGL(k_dequant_fp4, dim3(1024), dim3(256), 0, (hipStream_t)stream, out, W,
                     S, rows, cols);
  return dsv4g_check_launch("dequant_fp4");
}

int dsv4g_dequant_fp8(float *out, const uint8_t *W, const uint8_t *S, int rows, int cols,
                      void *stream) {
  hipLaunchKernelGGL(k_dequant_fp8, dim3(1024), dim3(256), 0, (hipStream_t)stream, out, W,
                     S, rows, cols);
  return dsv4g_check_launch("dequant_fp8");
}

int dsv4g_probe_converts(float *fp4_out, float *fp8_out, void *stream) {
  hipLaunchKernelGGL(k_probe_converts, dim3(1), dim3(256), 0, (hipStream_t)stream, fp4_out,
                     fp8_out);
  return dsv4g_check_launch("probe_converts");
}

static int fp4_shape_ok(int in, const char *who) {
  if (in <= 0 || in % 32 != 0 || in > 32 * 256) {
    return dsv4g_fail(DSV4G_EINVAL, "%s: FP4 input width %d must be a positive multiple of "
                                    "32 and at most 8192", who, in);
  }
  return 0;
}

static int fp8_shape_ok(int in, const char *who) {
  if (in <= 0 || in % 16 != 0 || in > FP8_MAX_IN) {
    return dsv4g_fail(DSV4G_EINVAL, "%s: FP8 input width %d must be a positive multiple of "
                                    "16 and at most %d", who, in, FP8_MAX_IN);
  }
  return 0;
}

int dsv4g_launch_gemv_fp4(const GemvArgs *a, int nvec, int nmat, void *stream) {
  if (fp4_shape_ok(a->in, "gemv_fp4")) return DSV4G_EINVAL;
  if (a->rows <= 0 || nvec <= 0) return dsv4g_fail(DSV4G_EINVAL, "gemv_fp4: bad size");
  int G = a->in / 32, gp = 1;
  while (gp < G) gp <<= 1;
  int tr = FP4_LDS_ENTRIES / gp;
  if (tr > 256) tr = 256;
  dim3 grid((a->rows + tr - 1) / tr, nvec, nmat);
  hipLaunchKernelGGL(k_gemv_fp4, grid, dim3(256), 0, (hipStream_t)stream, *a);
  return dsv4g_check_launch("gemv_fp4");
}

int dsv4g_launch_gemv_fp8(const GemvArgs *a, int nvec, int nmat, void *stream) {
  if (fp8_shape_ok(a->in, "gemv_fp8")) return DSV4G_EINVAL;
  if (a->rows <= 0 || nvec <= 0) return dsv4g_fail(DSV4G_EINVAL, "gemv_fp8: bad size");
  dim3 grid((a->rows + FP8_TR - 1) / FP8_TR, nvec, nmat);
  hipLaunchKernelGGL(k_gemv_fp8, grid, dim3(256), 0, (hipStream_t)stream, *a);
  return dsv4g_check_launch("gemv_fp8");
}

int dsv4g_gemv_fp4_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *S, int in, int rows, void *stream) {
  GemvArgs a = {};
  a.y[0] = y;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W;
  a.S[0] = S;
  a.in = in;
  a.rows = rows;
  a.round_out = 1;
  return dsv4g_launch_gemv_fp4(&a, 1, 1, stream);
}

int dsv4g_gemv_fp4_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int rows, void *stream) {
  GemvArgs a = {};
  a.y[0] = y0;
  a.y[1] = y1;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W0;
  a.S[0] = S0;
  a.W[1] = W1;
  a.S[1] = S1;
  a.in = in;
  a.rows = rows;
  a.round_out = 1;
  return dsv4g_launch_gemv_fp4(&a, 1, 2, stream);
}

int dsv4g_gemv_fp4_batch_q(float *y, const float *qx, const float *qscale, int batch,
                           const uint8_t *W, const uint8_t *S, int in, int rows,
                           void *stream) {
  GemvArgs a = {};
  a.y[0] = y;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W;
  a.S[0] = S;
  a.in = in;
  a.rows = rows;
  a.round_out = 1;
  a.y_stride = rows;
  a.qx_stride = in;
  a.qs_stride = (in + 127) / 128;
  return dsv4g_launch_gemv_fp4(&a, batch, 1, stream);
}

int dsv4g_gemv_fp8_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *S, int in, int out, int round_out, void *stream) {
  GemvArgs a = {};
  a.y[0] = y;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W;
  a.S[0] = S;
  a.in = in;
  a.rows = out;
  a.round_out = round_out;
  return dsv4g_launch_gemv_fp8(&a, 1, 1, stream);
}

int dsv4g_gemv_fp8_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int out, void *stream) {
  GemvArgs a = {};
  a.y[0] = y0;
  a.y[1] = y1;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W0;
  a.S[0] = S0;
  a.W[1] = W1;
  a.S[1] = S1;
  a.in = in;
  a.rows = out;
  a.round_out = 1;
  return dsv4g_launch_gemv_fp8(&a, 1, 2, stream);
}

int dsv4g_gemv_fp8_batch_q(float *y, const float *qx, const float *qscale, int batch,
                           const uint8_t *W, const uint8_t *S, int in, int out,
                           int round_out, void *stream) {
  GemvArgs a = {};
  a.y[0] = y;
  a.qx = qx;
  a.qscale = qscale;
  a.W[0] = W;
  a.S[0] = S;
  a.in = in;
  a.rows = out;
  a.round_out = round_out;
  a.y_stride = out;
  a.qx_stride = in;
  a.qs_stride = (in + 127) / 128;
  return dsv4g_launch_gemv_fp8(&a, batch, 1, stream);
}

int dsv4g_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                    int round_out, int batch, void *stream) {
  if (in <= 0 || out <= 0 || batch <= 0) return dsv4g_fail(DSV4G_EINVAL, "gemv_bf16: bad size");
  dim3 grid((out + 63) / 64, batch);
  hipLaunchKernelGGL(k_gemv_bf16, grid, dim3(64), 0, (hipStream_t)stream, y, x, W, in, out,
                     round_out, (size_t)out, (size_t)in);
  return dsv4g_check_launch("gemv_bf16");
}

int dsv4g_gemv_fp8_float(float *y, const float *x, const uint8_t *W, const float *wscale,
                         int in, int rows, int block, int mode, void *stream) {
  if (in <= 0 || rows <= 0 || block <= 0)
    return dsv4g_fail(DSV4G_EINVAL, "gemv_fp8_float: bad size");
  hipLaunchKernelGGL(k_gemv_fp8_float, dim3((rows + 63) / 64), dim3(64), 0,
                     (hipStream_t)stream, y, x, W, wscale, in, rows, block, mode);
  return dsv4g_check_launch("gemv_fp8_float");
}

int dsv4g_gemv_fp4_float(float *y, const float *qx, const float *qscale, const uint8_t *W,
                         const float *wscale, int in, int rows, int group, void *stream) {
  if (in <= 0 || rows <= 0 || group <= 0)
    return dsv4g_fail(DSV4G_EINVAL, "gemv_fp4_float: bad size");
  hipLaunchKernelGGL(k_gemv_fp4_float, dim3((rows + 63) / 64), dim3(64), 0,
                     (hipStream_t)stream, y, qx, qscale, W, wscale, in, rows, group);
  return dsv4g_check_launch("gemv_fp4_float");
}

int dsv4g_quant_fp4_rows(uint8_t *packed, uint8_t *scales, const float *w, int rows, int cols,
                         void *stream) {
  if (rows <= 0 || cols <= 0 || cols % 32)
    return dsv4g_fail(DSV4G_EINVAL, "quant_fp4_rows: cols must be a multiple of 32");
  const size_t n = (size_t)rows * (cols / 32);
  hipLaunchKernelGGL(k_quant_fp4_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, packed, scales, w, rows, cols);
  return dsv4g_check_launch("quant_fp4_rows");
}

int dsv4g_quant_fp8_blocks(uint8_t *codes, void *scales, const float *w, int rows, int cols,
                           int mode, void *stream) {
  if (rows <= 0 || cols <= 0) return dsv4g_fail(DSV4G_EINVAL, "quant_fp8_blocks: bad size");
  const int nb = ((rows + 127) / 128) * ((cols + 127) / 128);
  hipLaunchKernelGGL(k_quant_fp8_blocks, dim3(nb), dim3(256), 0, (hipStream_t)stream, codes,
                     scales, w, rows, cols, mode);
  return dsv4g_check_launch("quant_fp8_blocks");
}

}  // extern "C"
