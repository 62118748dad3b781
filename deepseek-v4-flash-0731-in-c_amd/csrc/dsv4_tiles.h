// dsv4_tiles.h - the bit-exact FP4 / FP8 GEMV row tiles shared by the
// standalone GEMV kernels (dsv4_gemv.hip) and the multi-expert MoE launches
// (dsv4_moe.hip).
//
// Bit-exact scheme (FP4 and FP8 alike): the reference accumulates, per output
// row, a partial over each scale group in column order (p = fmaf(w, qx, p))
// and then chains the groups in order (acc = fmaf(p, qscale * ws, acc));
// src/dsv4/dsv4_model.c:651-673, 1049-1074. Here each lane computes one
// (row, group) partial in the same sequential fmaf order, the pair
// (p, qscale*ws) goes through LDS, and one lane per row runs the group chain
// in order. A NaN scale (E8M0 255) skips its group, as in the reference: the
// pair becomes (0, 0), and fmaf(0, 0, acc) == acc because acc starts at +0
// and a round-to-nearest sum is never -0 unless both addends are.
#pragma once

#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"

namespace dsv4 {

// ===================================================== FP4 exact GEMV ====
// One workgroup owns FP4_TR complete rows. Lane t covers group g = t % gp of
// row t / gp in each pass (gp = next power of two >= G, rows per pass
// 256 / gp). G = in / 32 <= 256 and in % 32 == 0.
struct Fp4Geom {
  int G, gp, rpp, tr;
};

__device__ __forceinline__ Fp4Geom fp4_geom(int in) {
  Fp4Geom q;
  q.G = in / 32;
  q.gp = 1;
  while (q.gp < q.G) q.gp <<= 1;
  q.rpp = 256 / q.gp;
  q.tr = FP4_LDS_ENTRIES / q.gp;
  if (q.tr > 256) q.tr = 256;
  return q;
}

// Exact partial of one 32-column group: 32 sequential fmaf in column order.
__device__ __forceinline__ float fp4_group_partial(const uint4 w, const float *xq) {
  float p = 0.0f;
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float2 v;
    v = fp4x2<0>(wd[d]);
    p = fmaf(v.x, xq[8 * d + 0], p);
    p = fmaf(v.y, xq[8 * d + 1], p);
    v = fp4x2<1>(wd[d]);
    p = fmaf(v.x, xq[8 * d + 2], p);
    p = fmaf(v.y, xq[8 * d + 3], p);
    v = fp4x2<2>(wd[d]);
    p = fmaf(v.x, xq[8 * d + 4], p);
    p = fmaf(v.y, xq[8 * d + 5], p);
    v = fp4x2<3>(wd[d]);
    p = fmaf(v.x, xq[8 * d + 6], p);
    p = fmaf(v.y, xq[8 * d + 7], p);
  }
  return p;
}

// Rows [r0, r0 + tr) of y = bf16(W . qx) (FP4, per-32 E8M0 scales).
// ps: LDS scratch of FP4_LDS_ENTRIES + tr float2.
__device__ inline void fp4_rows_exact(float *__restrict__ y, const float *__restrict__ qx,
                               const float *__restrict__ qscale,
                               const uint8_t *__restrict__ W, const uint8_t *__restrict__ S,
                               int in, int rows, int r0, float2 *ps) {
  const Fp4Geom q = fp4_geom(in);
  const int t = threadIdx.x;
  const int g = t % q.gp, rsub = t / q.gp;
  const bool gact = g < q.G;
  const size_t pcols = (size_t)in / 2;
  const int stride = q.G + 1;  // padded LDS row: conflict-free chain reads
  float xq[32];
  float as = 0.0f;
  if (gact) {
    const float4 *xp = reinterpret_cast<const float4 *>(qx + 32 * g);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xp[i];
      xq[4 * i] = v.x;
      xq[4 * i + 1] = v.y;
      xq[4 * i + 2] = v.z;
      xq[4 * i + 3] = v.w;
    }
    as = qscale[g / 4];
  }
  const int npass = q.tr / q.rpp;
  constexpr int U = 4;
  for (int p0 = 0; p0 < npass; p0 += U) {
    uint4 w[U];
    uint32_t code[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int lr = (p0 + u) * q.rpp + rsub;
      const int row = r0 + lr;
      if (gact && p0 + u < npass && row < rows) {
        w[u] = *reinterpret_cast<const uint4 *>(W + (size_t)row * pcols + 16 * g);
        code[u] = S[(size_t)row * q.G + g];
      } else {
        w[u] = make_uint4(0, 0, 0, 0);
        code[u] = 127;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int lr = (p0 + u) * q.rpp + rsub;
      if (gact && p0 + u < npass && r0 + lr < rows) {
        float part = fp4_group_partial(w[u], xq);
        float s = as * e8m0(code[u]);
        if (code[u] == 255u) {  // NaN scale: the reference skips the group
          part = 0.0f;
          s = 0.0f;
        }
        ps[lr * stride + g] = make_float2(part, s);
      }
    }
  }
  __syncthreads();
  if (t < q.tr && r0 + t < rows) {
    const float2 *pr = ps + t * stride;
    float acc = 0.0f;
    for (int gg = 0; gg < q.G; ++gg) {
      const float2 v = pr[gg];
      acc = fmaf(v.x, v.y, acc);
    }
    y[r0 + t] = bf16_round(acc);
  }
}


// ===================================================== FP8 exact GEMV ====
// One workgroup owns FP8_TR rows. Lane t = (row t / 16, block slot t % 16);
// slot j handles 128-column blocks j, j+16, ... Each block partial is a
// 128-long sequential fmaf chain; qx comes from LDS (padded per block).
__device__ inline void fp8_rows_exact(float *__restrict__ y, const float *__restrict__ qx,
                               const float *__restrict__ qscale,
                               const uint8_t *__restrict__ W, const uint8_t *__restrict__ S,
                               int in, int rows, int r0, int round_out, float *xs,
                               float2 *ps) {
  const int t = threadIdx.x;
  const int CB = (in + 127) / 128;
  const int stride = CB + 1;
  // stage qx into LDS, block-padded by 4 floats
  for (int i = t; i < in; i += 256) xs[(i / 128) * 132 + (i % 128)] = qx[i];
  __syncthreads();
  const int lr = t / 16, slot = t % 16;
  const int row = r0 + lr;
  if (row < rows) {
    const uint8_t *wr = W + (size_t)row * in;
    const uint8_t *sr = S + (size_t)(row / 128) * CB;
    for (int cb = slot; cb < CB; cb += 16) {
      const int c0 = cb * 128;
      const int len = in - c0 < 128 ? in - c0 : 128;
      const float *xb = xs + cb * 132;
      float part = 0.0f;
      for (int c = 0; c < len; c += 16) {
        const uint4 w = *reinterpret_cast<const uint4 *>(wr + c0 + c);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float4 xv = *reinterpret_cast<const float4 *>(xb + c + 4 * d);
          float2 v = fp8x2<false>(wd[d]);
          part = fmaf(v.x, xv.x, part);
          part = fmaf(v.y, xv.y, part);
          v = fp8x2<true>(wd[d]);
          part = fmaf(v.x, xv.z, part);
          part = fmaf(v.y, xv.w, part);
        }
      }
      const uint32_t code = sr[cb];
      float s = qscale[cb] * e8m0(code);
      if (code == 255u) {
        part = 0.0f;
        s = 0.0f;
      }
      ps[lr * stride + cb] = make_float2(part, s);
    }
  }
  __syncthreads();
  if (t < FP8_TR && r0 + t < rows) {
    const float2 *pr = ps + t * stride;
    float acc = 0.0f;
    for (int cb = 0; cb < CB; ++cb) {
      const float2 v = pr[cb];
      acc = fmaf(v.x, v.y, acc);
    }
    y[r0 + t] = round_out ? bf16_round(acc) : acc;
  }
}


}  // namespace dsv4
