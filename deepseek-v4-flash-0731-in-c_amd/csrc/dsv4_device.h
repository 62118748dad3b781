// dsv4_device.h - gfx950 device helpers shared by the MoE expert-path kernels.
//
// Everything here reproduces a fixed numeric rule of the reference engine
// bit-for-bit; the citation on each helper names the rule. All HIP sources are
// compiled with -ffp-contract=off, so an fmaf()/fma() below is the only fused
// operation, and fp32 division/sqrt are IEEE correctly rounded (hipcc default).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DSV4_LIBM_FN __device__ __forceinline__
#define DSV4_LIBM_TABLE static __constant__ const
#include "dsv4_libm.h"

namespace dsv4 {

// Loads and stores through global-address-space pointers: a generic pointer
// gives a FLAT operation, and while one is in flight the compiler can only
// wait for every load of the wave (it cannot order FLAT against other loads),
// so a pending generic load ahead of a weight stream serialises the stream.
template <typename T>
__device__ __forceinline__ T ldg(const T *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
template <typename T>
__device__ __forceinline__ void stg(T *p, T v) {
  *(__attribute__((address_space(1))) T *)p = v;
}

// A wave-uniform pointer made visibly uniform (scalar registers), so that a
// buffer descriptor built from it needs no per-lane waterfall loop.
template <typename T>
__device__ __forceinline__ T *uptr(T *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Raw buffer over [p, p + bytes) (gfx9 descriptor word 3). A load at or past
// `bytes` returns zeros without a memory access, so a tile's edge needs no
// branch around its loads: branch-free loads keep the compiler's vmcnt waits
// progressive (the first result is consumed while later loads stream in).
// The base must be wave-uniform.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc buf_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(BufRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t buf_load4(BufRsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ float buf_loadf(BufRsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// BF16 round-to-nearest-even by integer bias, no NaN special case
// (src/dsv4/dsv4_ops.c:35-44 with the widening of dsv4_internal.h:248-254).
__device__ __forceinline__ float bf16_round(float f) {
  uint32_t u = f2u(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u2f(u & 0xFFFF0000u);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return u2f((uint32_t)h << 16);
}

// E8M0 scale 2^(code-127); code 255 is NaN (src/dsv4/dsv4_ops.c:63-67).
// Code 0 is the fp32 subnormal 2^-127, built from bits so no FTZ applies.
__device__ __forceinline__ float e8m0(uint32_t code) {
  if (code == 255u) return __builtin_nanf("");
  return code == 0u ? u2f(0x00400000u) : u2f(code << 23);
}

// OCP E4M3FN decode (src/dsv4/dsv4_ops.c:47-61): exponent field 0 is
// man*2^-9, S.1111.111 is NaN, else (8+man)*2^(exp-10).
__device__ __forceinline__ float e4m3_decode(uint32_t code) {
  const uint32_t e = (code >> 3) & 15u, m = code & 7u;
  float mag;
  if (e == 0u)
    mag = (float)m * (1.0f / 512.0f);
  else if (e == 15u && m == 7u)
    mag = __builtin_nanf("");
  else
    mag = u2f(((e + 120u) << 23) | (m << 20));
  return (code & 0x80u) ? -mag : mag;
}

// E2M1 nibble (src/dsv4/dsv4_model.c:971-974): bit 3 is the sign.
__device__ __forceinline__ float e2m1_decode(uint32_t nib) {
  const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float v = mag[nib & 7u];
  return (nib & 8u) ? -v : v;
}

// Two FP4 nibbles of byte BYTE of w as fp32 (x = low nibble = even column).
// Hardware MX convert with scale 1.0 is exact.
template <int BYTE>
__device__ __forceinline__ float2 fp4x2(uint32_t w) {
  auto v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, BYTE);
  return make_float2(v[0], v[1]);
}

// Two OCP E4M3 codes (bytes 0,1 or 2,3 of w) as fp32.
template <bool HI>
__device__ __forceinline__ float2 fp8x2(uint32_t w) {
  auto v = __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
  return make_float2(v[0], v[1]);
}

// Nearest E4M3 grid value, ties to even (src/dsv4/dsv4_ops.c:81-109): the
// reference's frexp form, kept for magnitudes above 448 and NaN (its
// overflow and infinity quirks). rintf is round-half-even, identical to the
// reference's floor-based helper for the magnitudes used here (< 16).
__device__ __forceinline__ float round_e4m3_frexp(float v) {
  if (v == 0.0f) return 0.0f;
  const float s = v < 0.0f ? -1.0f : 1.0f;
  const float a = fabsf(v);
  int e;
  float m = frexpf(a, &e);
  if (e >= -5) {
    float mr = rintf(m * 16.0f) / 16.0f;
    if (mr >= 1.0f) {
      mr = 0.5f;
      e++;
    }
    if (e - 1 > 8) return s * 448.0f;
    return s * mr * ldexpf(1.0f, e);
  }
  return s * (rintf(a * 512.0f) / 512.0f);
}

// The same for |v| <= 448 by bit operations, with the grid value's E4M3 code:
// at or above 2^-6 (an E4M3 normal) the fp32 significand is rounded to
// 3 bits, ties to even, by adding 0x7FFFF plus the kept lowest bit at bit 20
// (a carry moves to the exponent, as the reference's mr >= 1 step does), and
// the code is the kept bits rebiased (exponent 127 - 7); below it the value
// is rint(|v| 512) / 512 and the code that integer (8 is the smallest normal,
// code 0x08). The sign is copied, so a negative value that rounds to zero
// gives -0 as the reference's s * 0 does; v = +-0 gives +0 (code 0).
// Checked against the reference's dsv4_round_e4m3 for every float with
// |v| <= 448, both signs, values and decoded codes.
__device__ __forceinline__ float round_e4m3_small(float v, uint32_t &code) {
  const uint32_t u = f2u(v), a = u & 0x7FFFFFFFu;
  uint32_t r, c;
  if (a >= 0x3C800000u) {  // 2^-6
    r = (a + 0x7FFFFu + ((a >> 20) & 1u)) & 0xFFF00000u;
    c = (r >> 20) - (120u << 3);
  } else {
    const float q = rintf(u2f(a) * 512.0f);
    r = f2u(q * (1.0f / 512.0f));
    c = (uint32_t)q;
  }
  if (a == 0u) {
    code = 0u;
    return 0.0f;
  }
  code = c | ((u >> 24) & 0x80u);
  return u2f(r | (u & 0x80000000u));
}

__device__ __forceinline__ float round_e4m3(float v) {
  if (!(fabsf(v) <= 448.0f)) return round_e4m3_frexp(v);
  uint32_t c;
  return round_e4m3_small(v, c);
}

// 2^ceil(log2(max(amax,1e-4)/448)) (src/dsv4/dsv4_model.c:5590-5596): for a
// normal r = 1.f 2^E the reference's frexp gives e = E + 1, less one when
// f = 0, so the scale is r itself when its mantissa is zero and 2^(E+1)
// otherwise (checked against the reference over every amax below 2^-11 and
// above 2^125 and a dense sample between). r is normal for every finite
// amax >= 1e-4; infinity and NaN take the frexp form.
__device__ __forceinline__ float act_scale(float amax) {
  if (amax < 1e-4f) amax = 1e-4f;
  const float r = amax * (1.0f / 448.0f);
  const uint32_t ur = f2u(r);
  if (ur >= 0x7F800000u) {
    int e;
    const float m = frexpf(r, &e);
    if (m == 0.5f) e--;
    return ldexpf(1.0f, e);
  }
  const uint32_t ex = ur & 0x7F800000u;
  return u2f((ur & 0x007FFFFFu) ? ex + 0x00800000u : ex);
}

// q = round_e4m3(clamp(x * inv, +-448)) (src/dsv4/dsv4_model.c:5598-5604).
// A NaN x stays NaN through the clamp and takes the frexp form.
__device__ __forceinline__ float quant_e4m3(float x, float inv) {
  float q = x * inv;
  if (q > 448.0f) q = 448.0f;
  else if (q < -448.0f) q = -448.0f;
  return round_e4m3(q);
}

// E4M3 code of a grid value produced by round_e4m3 (exact).
__device__ __forceinline__ uint32_t e4m3_code(float v) {
  const uint32_t sign = (f2u(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  if (a < 0.015625f) return sign | (uint32_t)(a * 512.0f);  // subnormal, incl. 0
  const uint32_t b = f2u(a);
  const uint32_t ef = ((b >> 23) & 0xFFu) - 120u;  // fp32 exp -> E4M3 field
  return sign | (ef << 3) | ((b >> 20) & 7u);
}

// quant_e4m3 with the value's E4M3 code (a NaN x: NaN, coded by e4m3_code).
__device__ __forceinline__ float quant_e4m3_code(float x, float inv, uint32_t &code) {
  float q = x * inv;
  if (q > 448.0f) q = 448.0f;
  else if (q < -448.0f) q = -448.0f;
  if (!(fabsf(q) <= 448.0f)) {
    const float g = round_e4m3_frexp(q);
    code = e4m3_code(g);
    return g;
  }
  return round_e4m3_small(q, code);
}

// ---- glibc 2.35 libm, restated bit-exactly (dsv4_libm.h) ------------------
__device__ __forceinline__ float libm_expf(float x) { return dsv4_libm_expf(x); }
__device__ __forceinline__ float libm_log1pf_nonneg(float x) {
  return dsv4_libm_log1pf_nonneg(x);
}

// The expf table staged in LDS by threads 0-31 (the caller synchronises):
// kernels that evaluate expf under heavy HBM traffic read it there instead
// of paying a global-memory round trip per call.
__device__ __forceinline__ void libm_stage_table(uint64_t *tab) {
  if (threadIdx.x < 32) tab[threadIdx.x] = dsv4_libm_exp2_tab[threadIdx.x];
}
// The same in two steps, for kernels with weight loads in flight: an
// unconditional load into a register (a branch around it would make the
// compiler wait for every earlier load), stored once the weights are used.
__device__ __forceinline__ uint64_t libm_table_load() {
  return dsv4_libm_exp2_tab[threadIdx.x % 32];
}
__device__ __forceinline__ void libm_table_store(uint64_t *tab, uint64_t v) {
  if (threadIdx.x < 32) tab[threadIdx.x] = v;
}

// sqrt(softplus(z)) (src/dsv4/dsv4_model.c:5827-5831).
__device__ __forceinline__ float sqrt_softplus(float z, const uint64_t *tab) {
  if (z > 20.0f) return sqrtf(z);
  return sqrtf(libm_log1pf_nonneg(dsv4_libm_expf_t(z, tab)));
}
__device__ __forceinline__ float sqrt_softplus(float z) {
  return sqrt_softplus(z, dsv4_libm_exp2_tab);
}

// SwiGLU element (src/dsv4/dsv4_model.c:6264-6268): up clamped to
// [-limit, limit], gate clamped above only, t = silu(g) * u, rounded to fp32.
__device__ __forceinline__ float swiglu_t(float g, float u, float limit, const uint64_t *tab) {
  if (u > limit) u = limit;
  else if (u < -limit) u = -limit;
  if (g > limit) g = limit;
  const float silu = g / (1.0f + dsv4_libm_expf_t(-g, tab));
  return silu * u;
}

__device__ __forceinline__ float swiglu_t(float g, float u, float limit) {
  return swiglu_t(g, u, limit, dsv4_libm_exp2_tab);
}

// Wave-wide reductions (wave64).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// The same reductions through DPP row shifts and row broadcasts (register
// moves, no LDS round trip), for latency-critical single-wave code. The
// windows overlap, which max/min tolerate; lane 63 ends with the result,
// which readlane makes uniform.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v, float idv) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(idv), __float_as_int(v), CTRL,
                                                    ROW_MASK, BANK_MASK, false));
}
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ int dpp_i(int v, int idv) {
  return __builtin_amdgcn_update_dpp(idv, v, CTRL, ROW_MASK, BANK_MASK, false);
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  const float id = -__builtin_inff();
  v = fmaxf(v, dpp_f<0x111, 0xf, 0xf>(v, id));  // row_shr:1
  v = fmaxf(v, dpp_f<0x112, 0xf, 0xf>(v, id));  // row_shr:2
  v = fmaxf(v, dpp_f<0x113, 0xf, 0xf>(v, id));  // row_shr:3
  v = fmaxf(v, dpp_f<0x114, 0xf, 0xe>(v, id));  // row_shr:4
  v = fmaxf(v, dpp_f<0x118, 0xf, 0xc>(v, id));  // row_shr:8
  v = fmaxf(v, dpp_f<0x142, 0xa, 0xf>(v, id));  // row_bcast:15
  v = fmaxf(v, dpp_f<0x143, 0xc, 0xf>(v, id));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ int wave_min_dpp(int v) {
  const int id = 0x7fffffff;
  v = min(v, dpp_i<0x111, 0xf, 0xf>(v, id));
  v = min(v, dpp_i<0x112, 0xf, 0xf>(v, id));
  v = min(v, dpp_i<0x113, 0xf, 0xf>(v, id));
  v = min(v, dpp_i<0x114, 0xf, 0xe>(v, id));
  v = min(v, dpp_i<0x118, 0xf, 0xc>(v, id));
  v = min(v, dpp_i<0x142, 0xa, 0xf>(v, id));
  v = min(v, dpp_i<0x143, 0xc, 0xf>(v, id));
  return __builtin_amdgcn_readlane(v, 63);
}

// gamma_n = n u / (1 - n u), u = 2^-24: the classic bound on the rounding
// error of any n-term summation order.
__device__ __forceinline__ float gamma_n(int n) {
  const double nu = (double)n * 0x1p-24;
  return (float)(nu / (1.0 - nu));
}

// Candidate threshold kth - delta of the approximate router. Overflowing
// logits give kth = +inf with delta = +inf (or a NaN bound): the difference
// is NaN, every ">= thr" test would fail and no expert would be a candidate.
// Then every expert is one (-inf), which keeps at least min(K, E) candidates
// per token, a superset of the exact top-k.
__device__ __forceinline__ float cand_threshold(float kth, float delta) {
  const float thr = kth - delta;
  return thr == thr ? thr : -__builtin_inff();
}

// ---------------------------------------------------- exact chains ----
// One 8-column batch of the exact chain acc = fmaf(g[c], x[c], acc), in
// column order.
__device__ __forceinline__ float chain8(const float4 &ga, const float4 &gb, const float4 &xa,
                                        const float4 &xb, float acc) {
  acc = fmaf(ga.x, xa.x, acc);
  acc = fmaf(ga.y, xa.y, acc);
  acc = fmaf(ga.z, xa.z, acc);
  acc = fmaf(ga.w, xa.w, acc);
  acc = fmaf(gb.x, xb.x, acc);
  acc = fmaf(gb.y, xb.y, acc);
  acc = fmaf(gb.z, xb.z, acc);
  acc = fmaf(gb.w, xb.w, acc);
  return acc;
}

// Chain 8 * NB columns from LDS: g, x at the first column (fp32). The reads
// of the batch two ahead are in flight while a batch is chained; nothing is
// carried across calls (a loop-carried prefetch costs a full LDS drain per
// iteration), so the chain runs at the fma dependency latency.
template <int NB>
__device__ __forceinline__ float chain_cols(const float4 *g, const float4 *x, float acc) {
  float4 g0[4], g1[4], x0[4], x1[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    g0[j] = g[2 * j];
    g1[j] = g[2 * j + 1];
    x0[j] = x[2 * j];
    x1[j] = x[2 * j + 1];
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (j + 2 < NB) {
      g0[(j + 2) % 4] = g[2 * (j + 2)];
      g1[(j + 2) % 4] = g[2 * (j + 2) + 1];
      x0[(j + 2) % 4] = x[2 * (j + 2)];
      x1[(j + 2) % 4] = x[2 * (j + 2) + 1];
    }
    acc = chain8(g0[j % 4], g1[j % 4], x0[j % 4], x1[j % 4], acc);
    // pins the batch in place: its fmas before this point, the next reads
    // after it (otherwise every read is hoisted to the top and the fmas sink)
    asm volatile("" : "+v"(acc)::"memory");
  }
  return acc;
}

// chain_cols with the LDS reads of batch j + LA in flight while batch j is
// chained (ring of LA + 1 batches): for callers whose reads queue behind
// other lanes' (every lane of the wave chaining), where two batches ahead do
// not cover the LDS latency.
template <int NB, int LA>
__device__ __forceinline__ float chain_cols_deep(const float4 *g, const float4 *x, float acc) {
  constexpr int R = LA + 1;
  float4 g0[R], g1[R], x0[R], x1[R];
#pragma unroll
  for (int j = 0; j < LA && j < NB; ++j) {
    g0[j] = g[2 * j];
    g1[j] = g[2 * j + 1];
    x0[j] = x[2 * j];
    x1[j] = x[2 * j + 1];
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (j + LA < NB) {
      g0[(j + LA) % R] = g[2 * (j + LA)];
      g1[(j + LA) % R] = g[2 * (j + LA) + 1];
      x0[(j + LA) % R] = x[2 * (j + LA)];
      x1[(j + LA) % R] = x[2 * (j + LA) + 1];
    }
    acc = chain8(g0[j % R], g1[j % R], x0[j % R], x1[j % R], acc);
    asm volatile("" : "+v"(acc)::"memory");
  }
  return acc;
}

}  // namespace dsv4
