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

__device__ __host__ __forceinline__ Fp4Geom fp4_geom(int in) {
  Fp4Geom q;
  q.G = in / 32;
  q.gp = 1;
  while (q.gp < q.G) q.gp <<= 1;
  q.rpp = 256 / q.gp;
  q.tr = FP4_LDS_ENTRIES / q.gp;
  if (q.tr > 256) q.tr = 256;
  return q;
}

// The same with at most np passes per tile (np even: a paired tile holds
// np / 2 passes of each matrix), for tiles held in Fp4RegsT<np>.
__device__ __host__ __forceinline__ Fp4Geom fp4_geom_np(int in, int np) {
  Fp4Geom q = fp4_geom(in);
  if (q.tr > np * q.rpp) q.tr = np * q.rpp;
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

// acc = fmaf(p, s, acc) over n (p, s) pairs in order (the group chain of
// one output row). The LDS reads of the next 2 NB pairs are in flight while
// the current 2 NB are chained, so the loop runs at the fma dependency
// latency (NB = 4 holds half the registers of NB = 8). pr: 16-byte aligned.
template <int NB = 8>
__device__ __forceinline__ float pair_chain(const float2 *pr, int n) {
  const float4 *p4 = reinterpret_cast<const float4 *>(pr);
  const int nb = n / (2 * NB);
  float acc = 0.0f;
  float4 cur[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) cur[j] = nb > 0 ? p4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
  for (int b = 0; b < nb; ++b) {
    const int nx = (b + 1 < nb ? b + 1 : b) * NB;
    float4 nxt[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) nxt[j] = p4[nx + j];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc = fmaf(cur[j].x, cur[j].y, acc);
      acc = fmaf(cur[j].z, cur[j].w, acc);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) cur[j] = nxt[j];
  }
  for (int i = nb * 2 * NB; i < n; ++i) {
    const float2 v = pr[i];
    acc = fmaf(v.x, v.y, acc);
  }
  return acc;
}

// Even LDS row stride (in float2) for n pairs: 16-byte aligned rows whose
// 16-byte reads by consecutive lanes fall in distinct banks.
__device__ __host__ __forceinline__ int pair_stride(int n) { return (n | 1) + 1; }

// ============================================ two-step tiles (decode) ====
// The same exact schemes, split so that a kernel issues every weight load
// of its tile before it has the activation vector: *_load fills registers,
// *_finish computes. Register indices are compile-time constants throughout.
// LDS: the pairs take tr * pair_stride(G) float2 (FP4; at most
// FP4_LDS_ENTRIES + 2 * tr), plus 4096 bytes of FP4 scales, or
// FP8_TR * pair_stride(CB) float2 (FP8).

// FP4: all passes of the tile in flight (npass = tr / rpp <= NP; the full
// geometry of fp4_geom has npass <= 16 for every supported width, a caller
// may pass a geometry with fewer rows per tile). The lane's activation slice (group g: 32 E4M3 codes and
// the per-128 scale) is loaded first (fp4_tile_x), so that the first passes
// can start while later weights still stream in; holding codes rather than
// floats keeps the tile within 128 VGPRs (four waves per SIMD).
template <int NP = 16>
struct Fp4RegsT {
  uint4 w[NP];
  uint4 sc;        // this thread's 16 bytes of the tile's E8M0 scales
  uint32_t x8[8];  // E4M3 codes of the activation group, 4 per word
  float as;
};
using Fp4Regs = Fp4RegsT<16>;

// qx8: E4M3 codes of the quantised activation (their values are the grid
// values quant_fp8_act produces, exactly); qscale: per-128 scales. Both in
// global memory (buffer loads); fp4_tile_x_lds reads them from LDS.
template <int NP>
__device__ __forceinline__ void fp4_tile_x(Fp4RegsT<NP> &R, const uint8_t *qx8, const float *qscale,
                                           const Fp4Geom &q) {
  // lanes g >= G read past both buffers: zeros
  const uint32_t g = threadIdx.x % q.gp;
  const BufRsrc rx = buf_rsrc(qx8, 32u * q.G), rs = buf_rsrc(qscale, (uint32_t)q.G);
  const uint4 a = buf_load16(rx, 32u * g);
  const uint4 b = buf_load16(rx, 32u * g + 16u);
  R.x8[0] = a.x;
  R.x8[1] = a.y;
  R.x8[2] = a.z;
  R.x8[3] = a.w;
  R.x8[4] = b.x;
  R.x8[5] = b.y;
  R.x8[6] = b.z;
  R.x8[7] = b.w;
  R.as = buf_loadf(rs, 4u * (g / 4));
  __builtin_amdgcn_sched_barrier(0);  // issued before the weights that follow
}

// The same from LDS (after the weights are issued: no wait on them). Lanes
// g >= G read group G - 1; their partials are never stored.
template <int NP>
__device__ __forceinline__ void fp4_tile_x_lds(Fp4RegsT<NP> &R, const uint8_t *qx8,
                                               const float *qscale, const Fp4Geom &q) {
  const int g = min((int)threadIdx.x % q.gp, q.G - 1);
  const uint4 a = *reinterpret_cast<const uint4 *>(qx8 + 32 * g);
  const uint4 b = *reinterpret_cast<const uint4 *>(qx8 + 32 * g + 16);
  R.x8[0] = a.x;
  R.x8[1] = a.y;
  R.x8[2] = a.z;
  R.x8[3] = a.w;
  R.x8[4] = b.x;
  R.x8[5] = b.y;
  R.x8[6] = b.z;
  R.x8[7] = b.w;
  R.as = qscale[g / 4];
}

__device__ __forceinline__ uint32_t u4_word(const uint4 &v, int d) {
  return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
}

// One nibble pair (byte B of each word) of four independent group chains.
template <int B>
__device__ __forceinline__ void fp4_step4(const uint32_t (&wd)[4], float x0, float x1,
                                          float (&p)[4]) {
  float2 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = fp4x2<B>(wd[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fmaf(v[i].x, x0, p[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fmaf(v[i].y, x1, p[i]);
  // two columns at a time: at most 8 converted weights are live (a
  // pipelined caller holds a second tile in registers meanwhile)
  __builtin_amdgcn_sched_barrier(0);
}

// Partials of passes u0 .. u0 + 3: four 32-long fmaf chains, each in the
// reference's column order, interleaved so the fma latency is hidden.
template <int NP>
__device__ __forceinline__ void fp4_partials4(const Fp4RegsT<NP> &R, int u0, float (&p)[4]) {
  // converted per call on purpose: the scheduling barrier keeps the compiler
  // from hoisting 32 converted floats of every call to the top (registers)
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t *x8 = R.x8;
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = 0.0f;
  // tiles of fewer than four passes repeat their last pass (its extra
  // partials are never stored)
  const int u1 = u0 + 1 < NP ? u0 + 1 : NP - 1, u2 = u0 + 2 < NP ? u0 + 2 : NP - 1;
  const int u3 = u0 + 3 < NP ? u0 + 3 : NP - 1;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t wd[4] = {u4_word(R.w[u0], d), u4_word(R.w[u1], d), u4_word(R.w[u2], d),
                            u4_word(R.w[u3], d)};
    // columns 8d .. 8d + 7: codes in bytes of x8[2d] and x8[2d + 1]
    const float2 x01 = fp8x2<false>(x8[2 * d]), x23 = fp8x2<true>(x8[2 * d]);
    const float2 x45 = fp8x2<false>(x8[2 * d + 1]), x67 = fp8x2<true>(x8[2 * d + 1]);
    fp4_step4<0>(wd, x01.x, x01.y, p);
    fp4_step4<1>(wd, x23.x, x23.y, p);
    fp4_step4<2>(wd, x45.x, x45.y, p);
    fp4_step4<3>(wd, x67.x, x67.y, p);
  }
}

// Weights of rows [r0, r0 + tr) (single matrix) or, paired, of rows
// [r0, r0 + tr/2) of W0 then the same rows of W1 (row lr < half is W0 row
// r0 + lr, lr >= half is W1 row r0 + lr - half; half is npass / 2 whole
// passes, so the matrix of a pass is uniform). The tile's scales (tr * G <= 4096 bytes, row
// lr at lr * G) are fetched first, 16 bytes per thread, for LDS. Every load
// is a buffer load over the tile's existing rows of one matrix (at most 64 KB,
// 32-bit offsets): rows past the matrix, passes past npass and lanes g >= G
// read zeros without touching memory.
// NEAR (paired only): S1 lies after S0 within 2 GiB, so one range covers
// both matrices' scale rows and each scale dword is one load (half the
// registers in flight of the two-range form).
template <int NP, bool NEAR = false>
__device__ __forceinline__ void fp4_load_w(Fp4RegsT<NP> &R, const uint8_t *__restrict__ W0,
                                           const uint8_t *__restrict__ S0,
                                           const uint8_t *__restrict__ W1,
                                           const uint8_t *__restrict__ S1, int in, int rows,
                                           int r0, const Fp4Geom &q, bool pair) {
  const int t = threadIdx.x, g = t % q.gp, rsub = t / q.gp;
  const int npass = q.tr / q.rpp, half = q.tr / 2;
  const uint32_t pcols = (uint32_t)in / 2, G = (uint32_t)q.G;
  const int span = pair ? half : q.tr;  // tile rows of each matrix
  const uint32_t nrow = (uint32_t)max(0, min(span, rows - r0));
  const BufRsrc rs0 = buf_rsrc(S0 + (size_t)r0 * G, nrow * G);
  const BufRsrc rw0 = buf_rsrc(W0 + (size_t)r0 * pcols, nrow * pcols);
  const BufRsrc rs1 = pair ? buf_rsrc(S1 + (size_t)r0 * G, nrow * G) : rs0;
  const BufRsrc rw1 = pair ? buf_rsrc(W1 + (size_t)r0 * pcols, nrow * pcols) : rw0;
  {
    // scales: [W0 rows][W1 rows] when paired (seg bytes each), else the tile's
    // rows of W0; a lane's offset is in range of at most one of the two.
    // Dword loads: the ranges are multiples of 4 bytes, not always of 16.
    const uint32_t o = 16u * (uint32_t)t;
    uint32_t v[4];
    if (NEAR) {
      // one range from W0's tile rows to W1's (dist bytes on): a dword of
      // the first segment reads W0's rows, of the second W1's; padding rows
      // (nrow < half) and lanes past both segments read zeros
      const uint32_t seg = (uint32_t)half * G, nb = nrow * G, dist = (uint32_t)(S1 - S0);
      const BufRsrc rs = buf_rsrc(S0 + (size_t)r0 * G, nb ? dist + nb : 0u);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t od = o + 4u * (uint32_t)d;
        const uint32_t off = od < seg ? (od < nb ? od : 0xFFFFFFF0u)
                                      : (od - seg < nb ? dist + (od - seg) : 0xFFFFFFF0u);
        v[d] = buf_load4(rs, off);
      }
      R.sc = make_uint4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) v[d] = buf_load4(rs0, o + 4u * d);
    if (pair) {
      const uint32_t seg = (uint32_t)half * G;
#pragma unroll
      for (int d = 0; d < 4; ++d) v[d] |= buf_load4(rs1, o + 4u * d - seg);  // o < seg wraps
    }
    R.sc = make_uint4(v[0], v[1], v[2], v[3]);
    }
  }
  const uint32_t gcol = g < q.G ? 16u * (uint32_t)g : 0xFFFFFFF0u;  // g >= G: out of range
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const bool m1 = pair && u >= npass / 2;  // == (lr >= half): half = npass / 2 passes
    const uint32_t lr = (uint32_t)(u * q.rpp + rsub);
    const uint32_t lrow = m1 ? lr - (uint32_t)half : lr;
    R.w[u] = buf_load16(m1 ? rw1 : rw0, gcol == 0xFFFFFFF0u ? gcol : lrow * pcols + gcol);
  }
}

// Partials (group partial, scale) of every tile row into ps, ending with a
// barrier; R is free afterwards. cl: 4096 bytes of LDS for the scales, apart
// from ps. Starts with a barrier: the activation may have been read from LDS
// that ps overlaps.
template <int NP>
__device__ __forceinline__ void fp4_tile_partials(const Fp4RegsT<NP> &R, int rows, int r0,
                                                  const Fp4Geom &q, float2 *ps, uint8_t *cl,
                                                  bool pair) {
  const int t = threadIdx.x, g = t % q.gp, rsub = t / q.gp;
  const bool gact = g < q.G;
  const int npass = q.tr / q.rpp, half = q.tr / 2;
  const int stride = pair_stride(q.G);
  reinterpret_cast<uint4 *>(cl)[t] = R.sc;
  __syncthreads();
#pragma unroll
  for (int u0 = 0; u0 < NP; u0 += 4) {
    if (u0 < npass) {
      float p[4];
      fp4_partials4(R, u0, p);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int u = u0 + i;
        const int lr = u * q.rpp + rsub;
        const int row = r0 + ((pair && lr >= half) ? lr - half : lr);
        if (gact && u < npass && row < rows) {
          const uint32_t code = cl[lr * q.G + g];
          float part = p[i];
          float s = R.as * e8m0(code);
          if (code == 255u) {  // NaN scale: the reference skips the group
            part = 0.0f;
            s = 0.0f;
          }
          ps[lr * stride + g] = make_float2(part, s);
        }
      }
    }
  }
  __syncthreads();
}

// One lane per tile row runs the group chain over ps; returns bf16(acc) for
// lane t < tr (row lr = t), garbage otherwise. NB: pair_chain's read-ahead.
template <int NB = 8>
__device__ __forceinline__ float fp4_tile_chain(const Fp4Geom &q, const float2 *ps) {
  const int t = threadIdx.x;
  float acc = 0.0f;
  if (t < q.tr) acc = pair_chain<NB>(ps + t * pair_stride(q.G), q.G);
  return bf16_round(acc);
}

// Partials, then the chain (fp4_tile_partials, fp4_tile_chain).
template <int NP>
__device__ __forceinline__ float fp4_tile_rows(const Fp4RegsT<NP> &R, int rows, int r0,
                                               const Fp4Geom &q, float2 *ps, uint8_t *cl,
                                               bool pair) {
  fp4_tile_partials(R, rows, r0, q, ps, cl, pair);
  return fp4_tile_chain(q, ps);
}

// Single matrix: y[r0 + t] for the tile's rows.
template <int NP>
__device__ __forceinline__ void fp4_tile_load(Fp4RegsT<NP> &R, const uint8_t *__restrict__ W,
                                              const uint8_t *__restrict__ S, int in, int rows,
                                              int r0, const Fp4Geom &q) {
  fp4_load_w(R, W, S, W, S, in, rows, r0, q, false);
}
template <int NP>
__device__ __forceinline__ void fp4_tile_finish(const Fp4RegsT<NP> &R, float *y, int rows, int r0,
                                                const Fp4Geom &q, float2 *ps, uint8_t *cl) {
  const float v = fp4_tile_rows(R, rows, r0, q, ps, cl, false);
  if (threadIdx.x < q.tr && r0 + (int)threadIdx.x < rows) y[r0 + threadIdx.x] = v;
}

// Paired, with S1 after S0 within 2 GiB (the slots of one expert).
template <int NP>
__device__ __forceinline__ void fp4_pair_load_near(Fp4RegsT<NP> &R, const uint8_t *__restrict__ W0,
                                                   const uint8_t *__restrict__ S0,
                                                   const uint8_t *__restrict__ W1,
                                                   const uint8_t *__restrict__ S1, int in,
                                                   int rows, int r0, const Fp4Geom &q) {
  fp4_load_w<NP, true>(R, W0, S0, W1, S1, in, rows, r0, q, true);
}

// Paired: yl[lr] (LDS) for lr < tr.
template <int NP>
__device__ __forceinline__ void fp4_pair_load(Fp4RegsT<NP> &R, const uint8_t *__restrict__ W0,
                                              const uint8_t *__restrict__ S0,
                                              const uint8_t *__restrict__ W1,
                                              const uint8_t *__restrict__ S1, int in, int rows,
                                              int r0, const Fp4Geom &q) {
  fp4_load_w(R, W0, S0, W1, S1, in, rows, r0, q, true);
}
template <int NP>
__device__ __forceinline__ void fp4_pair_finish(const Fp4RegsT<NP> &R, float *yl, int rows, int r0,
                                                const Fp4Geom &q, float2 *ps, uint8_t *cl) {
  const float v = fp4_tile_rows(R, rows, r0, q, ps, cl, true);
  if (threadIdx.x < q.tr) yl[threadIdx.x] = v;
}

// FP8: lane t = (row r0 + t / 16, block slot t % 16), blocks slot, slot + 16,
// ...; the first two blocks of each lane (inputs up to 4096 wide) are loaded
// ahead, wider inputs load the rest in finish.
struct Fp8Regs {
  uint4 w[16];
  uint32_t sc[2];  // E8M0 codes of the lane's two 128-blocks
};

// Weights (two 128-blocks per lane) and block-scale codes of rows
// [r0, r0 + nr) of W for lane row lr = lr0 + t / 16, as buffer loads: rows
// past the matrix and blocks past the width read zeros.
__device__ __forceinline__ void fp8_load_rows(Fp8Regs &R, const uint8_t *__restrict__ W,
                                              const uint8_t *__restrict__ S, int in, int rows,
                                              int r0, int nr, int lr) {
  const int slot = threadIdx.x % 16;
  const uint32_t CB = (uint32_t)(in + 127) / 128;
  const uint32_t nrow = (uint32_t)max(0, min(nr, rows - r0));
  const BufRsrc rw = buf_rsrc(W + (size_t)r0 * in, nrow * (uint32_t)in);
  const BufRsrc rs = buf_rsrc(S, (uint32_t)((rows + 127) / 128) * CB);
  const uint32_t srow = (uint32_t)((r0 + lr) / 128) * CB;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t cb = (uint32_t)(slot + 16 * j);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t c = cb * 128u + 16u * i;
      R.w[8 * j + i] = buf_load16(rw, cb < CB && c < (uint32_t)in
                                          ? (uint32_t)lr * (uint32_t)in + c
                                          : 0xFFFFFFF0u);
    }
    R.sc[j] = __builtin_amdgcn_raw_buffer_load_b8(
        rs, cb < CB && (uint32_t)lr < nrow ? srow + cb : 0xFFFFFFF0u, 0, 0);
  }
}

__device__ __forceinline__ void fp8_tile_load(Fp8Regs &R, const uint8_t *__restrict__ W,
                                              const uint8_t *__restrict__ S, int in, int rows,
                                              int r0) {
  fp8_load_rows(R, W, S, in, rows, r0, FP8_TR, threadIdx.x / 16);
}

// Sequential partial of one 16-column piece.
__device__ __forceinline__ float fp8_piece(const uint4 w, const float *xb, float part) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float4 xv = *reinterpret_cast<const float4 *>(xb + 4 * d);
    float2 v = fp8x2<false>(wd[d]);
    part = fmaf(v.x, xv.x, part);
    part = fmaf(v.y, xv.y, part);
    v = fp8x2<true>(wd[d]);
    part = fmaf(v.x, xv.z, part);
    part = fmaf(v.y, xv.w, part);
  }
  return part;
}

// Block partials of the lane's row (row < rows) into ps[lr * stride + cb]:
// the two blocks held in R, then, for inputs wider than 4096, the rest
// streamed here. xs: the activation in LDS, padded to 132 floats per
// 128-block; qscale may be LDS or global.
__device__ __forceinline__ void fp8_partials(const Fp8Regs &R, const float *xs,
                                             const float *qscale, const uint8_t *__restrict__ W,
                                             const uint8_t *__restrict__ S, int in, int row,
                                             int lr, float2 *ps) {
  const int slot = threadIdx.x % 16;
  const int CB = (in + 127) / 128, stride = pair_stride(CB);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cb = slot + 16 * j;
    if (cb < CB) {
      const int len = min(128, in - cb * 128);
      const float *xb = xs + cb * 132;
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (16 * i < len) part = fp8_piece(R.w[8 * j + i], xb + 16 * i, part);
      const uint32_t code = R.sc[j];
      float s = qscale[cb] * e8m0(code);
      if (code == 255u) {  // NaN scale: the reference skips the block
        part = 0.0f;
        s = 0.0f;
      }
      ps[lr * stride + cb] = make_float2(part, s);
    }
  }
  const uint8_t *sr = S + (size_t)(row / 128) * CB;
  for (int cb = slot + 32; cb < CB; cb += 16) {
    const int len = min(128, in - cb * 128);
    const uint8_t *wr = W + (size_t)row * in + cb * 128;
    const float *xb = xs + cb * 132;
    float part = 0.0f;
    for (int c = 0; c < len; c += 16)
      part = fp8_piece(*reinterpret_cast<const uint4 *>(wr + c), xb + c, part);
    const uint32_t code = sr[cb];
    float s = qscale[cb] * e8m0(code);
    if (code == 255u) {
      part = 0.0f;
      s = 0.0f;
    }
    ps[lr * stride + cb] = make_float2(part, s);
  }
}

// Rows [r0, r0 + FP8_TR) of y (BF16-rounded if round_out).
__device__ __forceinline__ void fp8_tile_finish(const Fp8Regs &R, float *y, const float *xs,
                                                const float *qscale,
                                                const uint8_t *__restrict__ W,
                                                const uint8_t *__restrict__ S, int in, int rows,
                                                int r0, int round_out, float2 *ps) {
  const int t = threadIdx.x, lr = t / 16, row = r0 + lr;
  const int CB = (in + 127) / 128, stride = pair_stride(CB);
  if (row < rows) fp8_partials(R, xs, qscale, W, S, in, row, lr, ps);
  __syncthreads();
  if (t < FP8_TR && r0 + t < rows) {
    const float acc = pair_chain(ps + t * stride, CB);
    y[r0 + t] = round_out ? bf16_round(acc) : acc;
  }
}

// ---- paired FP8 tiles: the first half of a tile's rows from matrix 0
// (gate), the second half the same rows of matrix 1 (up), so one workgroup
// holds both operands of SwiGLU; yl[lr] receives bf16(acc).
// Lanes t / 16 < 8 (waves 0 and 1) take W0 rows r0 + t / 16, the others W1
// rows r0 + t / 16 - 8 (FP8_TR / 2 = 8 rows of each): the matrix is
// wave-uniform.
__device__ __forceinline__ void fp8_pair_load(Fp8Regs &R, const uint8_t *__restrict__ W0,
                                              const uint8_t *__restrict__ S0,
                                              const uint8_t *__restrict__ W1,
                                              const uint8_t *__restrict__ S1, int in, int rows,
                                              int r0) {
  const bool m1 = __builtin_amdgcn_readfirstlane((int)threadIdx.x / 64) >= 2;
  fp8_load_rows(R, m1 ? W1 : W0, m1 ? S1 : S0, in, rows, r0, FP8_TR / 2,
                (threadIdx.x / 16) & 7);
}

__device__ __forceinline__ void fp8_pair_finish(const Fp8Regs &R, float *yl, const float *xs,
                                                const float *qscale,
                                                const uint8_t *__restrict__ W0,
                                                const uint8_t *__restrict__ S0,
                                                const uint8_t *__restrict__ W1,
                                                const uint8_t *__restrict__ S1, int in, int rows,
                                                int r0, float2 *ps) {
  const int t = threadIdx.x, lr = t / 16, row = r0 + (lr & 7);
  const int CB = (in + 127) / 128, stride = pair_stride(CB);
  if (row < rows) fp8_partials(R, xs, qscale, lr < 8 ? W0 : W1, lr < 8 ? S0 : S1, in, row, lr, ps);
  __syncthreads();
  if (t < FP8_TR && r0 + (t & 7) < rows) {
    const float acc = pair_chain(ps + t * stride, CB);
    yl[t] = bf16_round(acc);
  }
}

// ================================ FP8 tiles staged by direct-to-LDS loads ====
// The same exact FP8 scheme (lane = one 128-column block of one row, its
// partial a sequential fmaf chain in column order, then one lane per row
// chains the blocks), with the tile's weights moved into LDS by
// buffer_load_dwordx4 ... lds instead of registers. A register tile gives
// every lane its own block, 128 contiguous bytes, so each of its loads
// touches 64 different cache lines; here each load instruction moves 1 KB
// of consecutive bytes (coalesced), and the 16-byte pieces are permuted
// within each block on the way so that the compute's block reads are free of
// LDS bank conflicts: piece p of block cb sits at slot (p + cb / 2) mod 8 of
// the block, so the 16 lanes of one read phase (16 consecutive blocks, the
// same piece) hit 16 distinct 16-byte bank groups.
//
// Tile: NR = 32768 / in rows (a power of two), 32 KB; lane t owns row t / CB,
// block t % CB (CB = in / 128). Supported when in is a power of two between
// 1024 and 8192 (fp8s_ok): every wave's 8 KB covers whole rows, and a wave's
// 64 lanes cover whole rows of blocks.
// Paired tiles hold NR / 2 rows of W0 then the same rows of W1.
//
// The loads are issued by inline assembly: the compiler does not see them,
// so it never inserts a wait for them (its own conservative wait before any
// LDS read after a direct-to-LDS load would drain every load in flight), and
// fp8s_wait() waits for all of the calling wave's loads before the barrier
// that publishes the tile.
typedef int DmaRsrc __attribute__((ext_vector_type(4)));

// Raw buffer descriptor in scalar registers (wave-uniform): base, no stride,
// num_records = bytes (reads at or past it return zeros and touch nothing).
__device__ __forceinline__ DmaRsrc dma_rsrc(const void *p, uint32_t bytes) {
  const uint64_t ad = (uint64_t)(uintptr_t)p;
  DmaRsrc r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)ad);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(ad >> 32) & 0xFFFFu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

// 16 bytes per lane from voff of r into LDS [lds + 16 lane] (lds
// wave-uniform). M0 carries the LDS base; one wait state after writing it.
__device__ __forceinline__ void dma_load16(DmaRsrc r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r)
               : "memory");
}

__device__ __forceinline__ void fp8s_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Waits until at most N vector memory operations of the wave are
// outstanding (they complete in order: everything issued before the last N
// has landed).
template <int N>
__device__ __forceinline__ void vm_wait_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __host__ __forceinline__ bool fp8s_ok(int in) {
  return in >= 1024 && in <= 8192 && (in & (in - 1)) == 0;
}
__device__ __host__ __forceinline__ int fp8s_rows(int in) { return 32768 / in; }

// 4 bytes per lane from voff of r into LDS [lds + 4 lane] (lds wave-uniform).
__device__ __forceinline__ void dma_load4(DmaRsrc r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r)
               : "memory");
}

// Issues the load of the scale-code dword holding the calling lane's block
// scale (lane t: tile row t / CB, block t % CB; the tile at rows r0 of W,
// paired: NR / 2 rows of W0, then of W1) into codes[t] (LDS, 4 bytes per
// lane). fp8s_code() extracts the byte once it has landed. The scale array
// of a matrix with CB >= 8 blocks per row is a multiple of 8 bytes, so the
// dword never leaves it.
__device__ __forceinline__ void fp8s_code_dma(uint32_t *codes, const uint8_t *__restrict__ S0,
                                              const uint8_t *__restrict__ S1, int in, int rows,
                                              int r0, bool pair) {
  const int t = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(t / 64);
  const int CB = in / 128, half = fp8s_rows(in) / 2;
  const int lr = t / CB, cb = t % CB;
  // a wave's lanes cover 64 / CB whole rows: one matrix per wave
  const bool m1 = pair && (wv * 64) / CB >= half;
  const int row = r0 + (m1 ? lr - half : lr);
  const DmaRsrc rs = dma_rsrc(m1 ? S1 : S0, (uint32_t)((rows + 127) / 128) * (uint32_t)CB);
  const uint32_t byte = row < rows ? (uint32_t)((row / 128) * CB + cb) : 0xFFFFFFF0u;
  dma_load4(rs, byte & ~3u, lds_addr(codes) + (uint32_t)wv * 256u);
}
__device__ __forceinline__ uint32_t fp8s_code(const uint32_t *codes, int in, int rows, int r0,
                                              bool pair) {
  const int t = threadIdx.x;
  const int CB = in / 128, half = fp8s_rows(in) / 2;
  const int lr = t / CB, cb = t % CB;
  const int row = r0 + ((pair && lr >= half) ? lr - half : lr);
  const uint32_t byte = (uint32_t)((row / 128) * CB + cb);
  return (codes[t] >> (8u * (byte & 3u))) & 0xFFu;
}

// Issues the tile's loads (8 per wave): rows [r0, r0 + NR) of W (or, paired,
// rows [r0, r0 + NR / 2) of W0 and of W1) into tile (32 KB of LDS, 16-byte
// aligned); rows at or past `rows` read zeros.
__device__ __forceinline__ void fp8s_dma(uint8_t *tile, const uint8_t *__restrict__ W0,
                                         const uint8_t *__restrict__ W1, int in, int rows,
                                         int r0, bool pair) {
  const int l = threadIdx.x % 64;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int half = fp8s_rows(in) / 2;
  const int wrows = 8192 / in;  // rows per wave
  const int lr0 = wv * wrows;   // the wave's first tile row
  const bool m1 = pair && lr0 >= half;
  const int mrow = r0 + (m1 ? lr0 - half : lr0);  // its row in the matrix
  const uint8_t *W = m1 ? W1 : W0;
  const int nrow = max(0, min(wrows, rows - mrow));
  const DmaRsrc rw = dma_rsrc(W + (size_t)mrow * in, (uint32_t)(nrow * in));
  const uint32_t base = lds_addr(tile) + (uint32_t)wv * 8192u;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const uint32_t q = (uint32_t)d * 1024u + 16u * (uint32_t)l;  // byte in the wave's 8 KB
    const uint32_t o = q % (uint32_t)in, cb = o / 128u, slot = (o % 128u) / 16u;
    const uint32_t piece = (slot - cb / 2u) & 7u;
    dma_load16(rw, (q / (uint32_t)in) * (uint32_t)in + cb * 128u + 16u * piece,
               base + (uint32_t)d * 1024u);
  }
}

// After fp8s_wait() and a barrier: the lane's block partial from the staged
// tile and the activation xs (LDS, 132 floats per 128-block), paired with
// its scale qscale[cb] * e8m0(code) into ps[lr * stride + cb] (a NaN scale
// skips the block), then a barrier and one lane per row chains the blocks;
// returns the row's fp32 sum for lanes t < NR (rows past `rows` give 0).
__device__ __forceinline__ float fp8s_rows_dot(const uint8_t *tile, const float *xs,
                                               const float *qscale, uint32_t code, int in,
                                               float2 *ps) {
  const int t = threadIdx.x;
  const int CB = in / 128, NR = fp8s_rows(in), stride = pair_stride(CB);
  const int lr = t / CB, cb = t % CB;
  const uint8_t *blk = tile + (size_t)lr * in + cb * 128;
  const float *xb = xs + cb * 132;
  float part = 0.0f;
  // one piece ahead: its weight read is in flight while a piece is chained
  // (the chain is sequential; reading further ahead only costs registers)
  uint4 w = *reinterpret_cast<const uint4 *>(blk + 16 * ((cb / 2) & 7));
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const uint4 wn = *reinterpret_cast<const uint4 *>(blk + 16 * ((p + 1 + cb / 2) & 7));
    part = fp8_piece(w, xb + 16 * p, part);
    w = wn;
    asm volatile("" : "+v"(part)::"memory");  // keeps later pieces' reads below
  }
  float s = qscale[cb] * e8m0(code);
  if (code == 255u) {  // NaN scale: the reference skips the block
    part = 0.0f;
    s = 0.0f;
  }
  ps[lr * stride + cb] = make_float2(part, s);
  __syncthreads();
  return t < NR ? pair_chain(ps + t * stride, CB) : 0.0f;
}

}  // namespace dsv4
