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

// The FP4 GEMVs (dsv4_gemv_fp4_q / _pair_q / _batch_q,
// src/dsv4/dsv4_model.c:967-1380) on the decode layer's register tiles
// (dsv4_tiles.h): one (row, 32-column group) partial per lane as a sequential
// fmaf chain, one lane per row chaining the groups in order; NP
// passes per tile (paired: NP / 2 of each matrix over the same rows), every
// pass issued before the first FMA, NP chosen by the host so that one call
// spans about a thousand workgroups. The token's activation arrives as the
// E4M3 grid values the activation quant produced (floats): its codes are
// exact (e4m3_code) and go to LDS with the per-128 scales, loaded ahead of
// the weights. grid = (tiles, nvec); pair: y[0] / y[1] for W[0] / W[1].
template <int NP>
__global__ __launch_bounds__(256) void k_gemv_fp4_t(GemvArgs a, int pair) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float s_y[256];
  const int tid = threadIdx.x, b = blockIdx.y;
  const Fp4Geom q = fp4_geom_np(a.in, NP);
  const int in = a.in;
  const float *qx = a.qx + (size_t)b * a.qx_stride;
  const float *qs = a.qscale + (size_t)b * a.qs_stride;
  // this thread's activation values (16 at 16 tid, and 4096 further for
  // in > 4096) and per-128 scale (thread i < in / 128: scale i), loaded
  // before the weights (loads complete in order: issued after the weights,
  // they would wait for every weight to land)
  const BufRsrc rx = buf_rsrc(qx, 4u * (uint32_t)in);
  uint4 xv[8];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xv[4 * k + i] = buf_load16(rx, 4u * (uint32_t)(16 * tid + 4096 * k) + 16u * i);
  const float qsv = buf_loadf(buf_rsrc(qs, 4u * (uint32_t)((in + 127) / 128)), 4u * (uint32_t)tid);
  Fp4RegsT<NP> R;
  const int half = q.tr / 2;
  const int r0 = pair ? blockIdx.x * half : blockIdx.x * q.tr;
  if (pair)
    fp4_pair_load(R, a.W[0], a.S[0], a.W[1], a.S[1], in, a.rows, r0, q);
  else
    fp4_tile_load(R, a.W[0], a.S[0], in, a.rows, r0, q);
  uint8_t *cl = reinterpret_cast<uint8_t *>(lds) + (size_t)q.tr * pair_stride(q.G) * 8;
  uint8_t *x8 = cl + 4096;
  float *xs = reinterpret_cast<float *>(x8 + ((in + 15) & ~15));
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int base = 16 * tid + 4096 * k;
    if (base < in) {
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = xv[4 * k + i];
        c[i] = e4m3_code(u2f(v.x)) | (e4m3_code(u2f(v.y)) << 8) |
               (e4m3_code(u2f(v.z)) << 16) | (e4m3_code(u2f(v.w)) << 24);
      }
      *reinterpret_cast<uint4 *>(x8 + base) = make_uint4(c[0], c[1], c[2], c[3]);
    }
  }
  if (tid < (in + 127) / 128) xs[tid] = qsv;  // in <= 8192: at most 64 scales
  __syncthreads();
  fp4_tile_x_lds(R, x8, xs, q);
  float2 *ps = reinterpret_cast<float2 *>(lds);
  if (pair) {
    fp4_pair_finish(R, s_y, a.rows, r0, q, ps, cl);
    __syncthreads();
    if (a.swi_y) {  // routed_swiglu_quant's y (src/dsv4/dsv4_model.c:6258-6268)
      if (tid < half && r0 + tid < a.rows)
        a.swi_y[(size_t)b * a.y_stride + r0 + tid] =
            bf16_round(swiglu_t(s_y[tid], s_y[tid + half], a.swi_limit) *
                       (a.swi_w ? *a.swi_w : 1.0f));
    } else if (tid < q.tr && r0 + tid % half < a.rows) {
      a.y[tid / half][(size_t)b * a.y_stride + r0 + tid % half] = s_y[tid];
    }
  } else {
    fp4_tile_finish(R, a.y[0] + (size_t)b * a.y_stride, a.rows, r0, q, ps, cl);
  }
}

// ========================================================= FP8 GEMV =====
// dsv4_gemv_fp8_q / _pair_q / _batch_q (src/dsv4/dsv4_model.c:571-961) for
// any width up to 8192 and any number of token vectors, bit-exact: per
// (row, 128-column block) a 128-long sequential fmaf chain, then per row the
// block chain acc = fmaf(p, qscale * ws, acc) in order (NaN block scale:
// the block is skipped, as in the reference).
//
// Lane t of a workgroup is (row t / SL, slot t % SL) and owns blocks slot
// and slot + SL; SL (8, 16 or 32 lanes per row) is the smallest that leaves
// every lane at most two blocks, so a lane's whole weight slice (2 x 128 B)
// is loaded into registers before any arithmetic and the workgroup's rows
// stream from HBM in one go. Tokens are taken G at a time: each 16-column
// piece is decoded once and feeds G chains, and the weights stay in
// registers across all the token groups, so a batch reads them from HBM
// once. LDS: the G tokens' activations (padded to 132 floats per block) and
// their scales, and the (partial, scale) pairs of the block chains.
template <int SL, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G == 4 ? 4 : 1))) void k_fp8_proj(
    GemvArgs a, int nvec, int gpw, int vec4) {
  constexpr int TR = 256 / SL;
  extern __shared__ __align__(16) float lds[];
  const int m = blockIdx.z, t = threadIdx.x, lr = t / SL, slot = t % SL;
  const int in = a.in, rows = a.rows, r0 = blockIdx.x * TR;
  const int CB = (in + 127) / 128, stride = pair_stride(CB);
  float *xs = lds;                                   // [G][CB][132]
  float *qs = xs + (size_t)G * CB * 132;             // [G][CB]
  float2 *ps = reinterpret_cast<float2 *>(qs + ((G * CB + 3) & ~3));  // [G][TR][stride]
  // per wave: the exchange of its rows' weights (64 chunks of 128 B, 144 B
  // apart), over the space of xs, qs and ps before they are written
  uint8_t *xch = reinterpret_cast<uint8_t *>(lds) + (t / 64) * 9216;

  // this workgroup's token groups: gpw groups of G from blockIdx.y * gpw
  const int tbeg = blockIdx.y * gpw * G, tend = min(nvec, tbeg + gpw * G);
  // the first group's activations (up to 8192 values) are loaded ahead of the
  // weights: loads complete in order, so behind the weights they would wait
  // for every weight to land
  const bool xpre = vec4 && G * in <= 8192;  // then also G CB <= 256 scales
  float4 xr[8];
  float qr = 0.0f;
  if (xpre) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = 4 * t + 1024 * k;
      const int g = i / in, c = i % in;
      xr[k] = i < G * in && tbeg + g < nvec
                  ? *reinterpret_cast<const float4 *>(a.qx + (size_t)(tbeg + g) * a.qx_stride + c)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (t < G * CB && tbeg + t / CB < nvec)
      qr = a.qscale[(size_t)(tbeg + t / CB) * a.qs_stride + t % CB];
  }

  // the weights (zeros past the matrix): round j covers the row's columns
  // [128 SL j, 128 SL (j + 1)); load i of the SL lanes of a row reads 16 SL
  // contiguous bytes (chunk i SL + slot of the round), so every load
  // instruction covers whole lines; the chunks then go through the wave's
  // LDS region to the lane that owns their block (block slot + SL j)
  const uint32_t nrow = (uint32_t)max(0, min(TR, rows - r0));
  const BufRsrc rw = buf_rsrc(a.W[m] + (size_t)r0 * in, nrow * (uint32_t)in);
  const BufRsrc rs = buf_rsrc(a.S[m], (uint32_t)((rows + 127) / 128) * CB);
  uint4 w[16];
  uint32_t sc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t cb = (uint32_t)(slot + SL * j);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t c = (uint32_t)(SL * 128 * j + 16 * (SL * i + slot));
      w[8 * j + i] = buf_load16(rw, c < (uint32_t)in ? (uint32_t)lr * (uint32_t)in + c
                                                     : 0xFFFFFFF0u);
    }
    sc[j] = __builtin_amdgcn_raw_buffer_load_b8(
        rs, cb < (uint32_t)CB && (uint32_t)lr < nrow ? (uint32_t)((r0 + lr) / 128) * CB + cb
                                                      : 0xFFFFFFF0u, 0, 0);
  }
  {
    // the exchange: chunk q = SL i + slot of round j lies in block q / 8 at
    // piece q % 8; the wave's rows (lr % (64 / SL)) are SL 144 B apart
    const int wr = lr % (64 / SL);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (SL * 128 * j >= in) break;  // a round wholly past the row (uniform)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int q = SL * i + slot;
        *reinterpret_cast<uint4 *>(xch + (wr * SL + q / 8) * 144 + (q % 8) * 16) = w[8 * j + i];
      }
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 8; ++i)
        w[8 * j + i] = *reinterpret_cast<const uint4 *>(xch + (wr * SL + slot) * 144 + 16 * i);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();  // every wave's exchange read before xs, qs and ps take the space
  if (xpre) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = 4 * t + 1024 * k;
      const int g = i / in, c = i % in;
      if (i < G * in)
        *reinterpret_cast<float4 *>(xs + (size_t)g * CB * 132 + (c / 128) * 132 + (c % 128)) =
            xr[k];
    }
    if (t < G * CB) qs[t] = qr;
  }

  for (int t0 = tbeg; t0 < tend; t0 += G) {
    // the group's activations and scales into LDS (zeros past the last token)
    if (xpre && t0 == tbeg) {
      // loaded ahead of the weights
    } else if (vec4) {
      for (int i = 4 * t; i < G * in; i += 1024) {
        const int g = i / in, c = i % in;
        const float4 v = t0 + g < nvec
                             ? *reinterpret_cast<const float4 *>(
                                   a.qx + (size_t)(t0 + g) * a.qx_stride + c)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4 *>(xs + (size_t)g * CB * 132 + (c / 128) * 132 + (c % 128)) = v;
      }
    } else {
      for (int i = t; i < G * in; i += 256) {
        const int g = i / in, c = i % in;
        xs[(size_t)g * CB * 132 + (c / 128) * 132 + (c % 128)] =
            t0 + g < nvec ? a.qx[(size_t)(t0 + g) * a.qx_stride + c] : 0.0f;
      }
    }
    if (!(xpre && t0 == tbeg))
      for (int i = t; i < G * CB; i += 256) {
        const int g = i / CB;
        qs[i] = t0 + g < nvec ? a.qscale[(size_t)(t0 + g) * a.qs_stride + i % CB] : 0.0f;
      }
    __syncthreads();
    if (r0 + lr < rows) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cb = slot + SL * j;
        if (cb < CB) {
          const int len = min(128, in - cb * 128);
          float part[G];
#pragma unroll
          for (int g = 0; g < G; ++g) part[g] = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (16 * i < len) {
              const uint32_t wd[4] = {w[8 * j + i].x, w[8 * j + i].y, w[8 * j + i].z,
                                      w[8 * j + i].w};
              float v[16];
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                const float2 lo = fp8x2<false>(wd[d]), hi = fp8x2<true>(wd[d]);
                v[4 * d] = lo.x;
                v[4 * d + 1] = lo.y;
                v[4 * d + 2] = hi.x;
                v[4 * d + 3] = hi.y;
              }
#pragma unroll
              for (int g = 0; g < G; ++g) {
                const float *xb = xs + (size_t)g * CB * 132 + cb * 132 + 16 * i;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                  const float4 xv = *reinterpret_cast<const float4 *>(xb + 4 * d);
                  part[g] = fmaf(v[4 * d], xv.x, part[g]);
                  part[g] = fmaf(v[4 * d + 1], xv.y, part[g]);
                  part[g] = fmaf(v[4 * d + 2], xv.z, part[g]);
                  part[g] = fmaf(v[4 * d + 3], xv.w, part[g]);
                }
              }
            }
          }
#pragma unroll
          for (int g = 0; g < G; ++g) {
            float s = qs[g * CB + cb] * e8m0(sc[j]);
            float p = part[g];
            if (sc[j] == 255u) {  // NaN scale: the reference skips the block
              p = 0.0f;
              s = 0.0f;
            }
            ps[(size_t)(g * TR + lr) * stride + cb] = make_float2(p, s);
          }
        }
      }
    }
    __syncthreads();
    if (t < G * TR) {
      const int g = t / TR, r = t % TR;
      if (r0 + r < rows && t0 + g < nvec) {
        const float acc = pair_chain(ps + (size_t)(g * TR + r) * stride, CB);
        a.y[m][(size_t)(t0 + g) * a.y_stride + r0 + r] = a.round_out ? bf16_round(acc) : acc;
      }
    }
    __syncthreads();  // LDS is refilled by the next group
  }
}

// Token groups per workgroup: all of them when the row tiles alone give
// 1024 or more workgroups (each weight read from HBM once); otherwise the
// groups are spread so the launch still has about that many (a small
// matrix's re-reads come from the caches).
static size_t max_size(size_t a, size_t b) { return a > b ? a : b; }

template <int SL, int G>
static void launch_fp8_proj(const GemvArgs *a, int nvec, int nmat, hipStream_t st) {
  constexpr int TR = 256 / SL;
  const int CB = (a->in + 127) / 128;
  // xs, qs and ps, or the four waves' weight exchanges before them
  const size_t lds = max_size(((size_t)G * CB * 132 + ((G * CB + 3) & ~3)) * 4 +
                                  (size_t)G * TR * pair_stride(CB) * 8,
                              (size_t)4 * 9216);
  const int tiles = (a->rows + TR - 1) / TR * nmat, groups = (nvec + G - 1) / G;
  const int split = min(groups, max(1, 1024 / tiles));
  const int gpw = (groups + split - 1) / split;
  const int vec4 = ((uintptr_t)a->qx % 16 == 0) && (a->qx_stride % 4 == 0);
  hipLaunchKernelGGL((k_fp8_proj<SL, G>),
                     dim3((a->rows + TR - 1) / TR, (groups + gpw - 1) / gpw, nmat), dim3(256),
                     lds, st, *a, nvec, gpw, vec4);
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

// ====================================================== row chains =====
// The same chains, one lane per output row, for rows whose bytes are a
// multiple of 16: each lane reads its own row straight from HBM 16 bytes at
// a time through one buffer range over the wave's 64 rows (a row past the
// matrix reads zeros), 16 loads per chunk and two chunks in turn, so 32
// loads (512 bytes of the row) are in flight while a chunk is chained; x
// (every token, at most RC_XBYTES) and the FP8 block scales of the wave's
// row blocks are staged in LDS once and read as broadcasts. The per-column arithmetic is the reference's, so the results
// are bit for bit those of the one-load-at-a-time kernels above; they only
// wait less.
//   RC_BF16: acc_t = fmaf(bf16(w), x_t[c], acc_t) for MAXB tokens at most
//            (dsv4_gemv_bf16(_batch), src/dsv4/dsv4_model.c:266-367; the vocab
//            head's head_logits_block, :7221-7255);
//   RC_FP8_X: acc += w * (x * s)   (dsv4_gemv_fp8, src/dsv4/dsv4_ops.c:176-209);
//   RC_FP8_XS: the same when the wave's 64 rows share one row block (block a
//            multiple of 64): xs = x * s is formed once per column in LDS,
//            as the reference forms it once per row block;
//   RC_FP8_T: acc += (w * x) * s   (dsv4_gemv_fp8_tbl, :216-239),
// unfused as the reference is built; s = wscale[row / block][c / block],
// block a multiple of 16.
#define RC_BF16 0
#define RC_FP8_X 1
#define RC_FP8_T 2
#define RC_FP8_XS 3
#define RC_CHUNK 16           // 16-byte loads per chunk
#define RC_XBYTES (64 * 1024)  // LDS for x

struct RowChainArgs {
  float *y;
  const float *x;
  const uint8_t *W;
  const float *wscale;
  int in, rows, block, batch, round_out;
  size_t y_stride, x_stride;
};

// Pieces byte0, byte0 + 16, ... of the lane's row (at row_off in the
// wave's range; live: the lane has a row). Past the row, or without one:
// zeros, nothing read.
__device__ __forceinline__ void rc_load(uint4 (&w)[RC_CHUNK], BufRsrc r, uint32_t row_off,
                                        bool live, uint32_t byte0, uint32_t rb) {
#pragma unroll
  for (int i = 0; i < RC_CHUNK; ++i) {
    const uint32_t b = byte0 + 16u * i;
    w[i] = buf_load16(r, live && b < rb ? row_off + b : 0xFFFFFFF0u);
  }
}

// One chunk: columns c0 .. of the 16-byte pieces w (8 BF16 or 16 FP8 each);
// xs: x in LDS, token t at t * in.
template <int KIND, int MAXB>
__device__ __forceinline__ void rc_chain(const RowChainArgs &a, const uint4 (&w)[RC_CHUNK],
                                         int c0, float (&acc)[MAXB], const float *srow,
                                         const float *xs) {
  constexpr int CPP = KIND == RC_BF16 ? 8 : 16;  // columns per piece
#pragma unroll
  for (int i = 0; i < RC_CHUNK; ++i) {
    const int c = c0 + CPP * i;
    if (c >= a.in) break;  // uniform: the chunk's last pieces may lie past the row
    const uint32_t wd[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
    if (KIND == RC_BF16) {
#pragma unroll
      for (int t = 0; t < MAXB; ++t) {
        if (t >= a.batch) break;
        const float4 *xt = reinterpret_cast<const float4 *>(xs + (size_t)t * a.in + c);
        const float4 x0 = xt[0], x1 = xt[1];
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          acc[t] = fmaf(u2f(wd[d] << 16), xv[2 * d], acc[t]);
          acc[t] = fmaf(u2f(wd[d] & 0xFFFF0000u), xv[2 * d + 1], acc[t]);
        }
      }
    } else if (KIND == RC_FP8_XS) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float2 lo = fp8x2<false>(wd[d]), hi = fp8x2<true>(wd[d]);
        const float wv[4] = {lo.x, lo.y, hi.x, hi.y};
        const float4 x4 = *reinterpret_cast<const float4 *>(xs + c + 4 * d);
        const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[0] += wv[e] * xv[e];
      }
    } else {
      const float s = srow[c / a.block];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float2 lo = fp8x2<false>(wd[d]), hi = fp8x2<true>(wd[d]);
        const float wv[4] = {lo.x, lo.y, hi.x, hi.y};
        const float4 x4 = *reinterpret_cast<const float4 *>(xs + c + 4 * d);
        const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[0] += KIND == RC_FP8_X ? wv[e] * (xv[e] * s) : (wv[e] * xv[e]) * s;
      }
    }
  }
}

template <int KIND, int MAXB>
__global__ __launch_bounds__(64) void k_rowchain(RowChainArgs a) {
  extern __shared__ __align__(16) float xs[];  // batch * in floats
  const int r0 = blockIdx.x * 64, lane = threadIdx.x, row = r0 + lane;
  for (int t = 0; t < a.batch; ++t)
    for (int i = lane; i < a.in / 4; i += 64)
      reinterpret_cast<float4 *>(xs + (size_t)t * a.in)[i] =
          reinterpret_cast<const float4 *>(a.x + (size_t)t * a.x_stride)[i];
  const uint32_t rb = (uint32_t)a.in * (KIND == RC_BF16 ? 2u : 1u);
  const int nrow = min(64, a.rows - r0);
  const BufRsrc r = buf_rsrc(a.W + (size_t)r0 * rb, (uint32_t)nrow * rb);
  const bool live = lane < nrow;
  const uint32_t row_off = (uint32_t)lane * rb;
  const float *srow = nullptr;
  if (KIND == RC_FP8_XS) {
    // xs[c] = x[c] * s[row block][c / block], the row block of all 64 rows
    const int cblocks = (a.in + a.block - 1) / a.block;
    const float *s = a.wscale + (size_t)(r0 / a.block) * cblocks;
    __syncthreads();  // x in LDS
    for (int i = lane; i < a.in; i += 64) xs[i] = xs[i] * s[i / a.block];
  } else if (KIND != RC_BF16) {
    // the block scales of the wave's row blocks, after x in LDS
    const int cblocks = (a.in + a.block - 1) / a.block;
    const int rb0 = r0 / a.block, nrb = (min(r0 + 63, a.rows - 1)) / a.block - rb0 + 1;
    float *sc = xs + (size_t)a.batch * a.in;
    for (int i = lane; i < nrb * cblocks; i += 64)
      sc[i] = a.wscale[(size_t)rb0 * cblocks + i];
    srow = sc + (size_t)(min(row, a.rows - 1) / a.block - rb0) * cblocks;
  }
  float acc[MAXB];
#pragma unroll
  for (int t = 0; t < MAXB; ++t) acc[t] = 0.0f;
  constexpr uint32_t CB = 16u * RC_CHUNK;  // bytes per chunk
  constexpr int CPC = (KIND == RC_BF16 ? 8 : 16) * RC_CHUNK;  // columns per chunk
  uint4 A[RC_CHUNK], B[RC_CHUNK];
  rc_load(A, r, row_off, live, 0, rb);
  __syncthreads();  // x in LDS
  for (uint32_t b0 = 0; b0 < rb; b0 += 2 * CB) {
    const int c0 = (int)(b0 / CB) * CPC;
    rc_load(B, r, row_off, live, b0 + CB, rb);
    rc_chain<KIND, MAXB>(a, A, c0, acc, srow, xs);
    rc_load(A, r, row_off, live, b0 + 2 * CB, rb);
    rc_chain<KIND, MAXB>(a, B, c0 + CPC, acc, srow, xs);
  }
  if (row >= a.rows) return;
#pragma unroll
  for (int t = 0; t < MAXB; ++t) {
    if (t >= a.batch) break;
    a.y[(size_t)t * a.y_stride + row] = a.round_out ? bf16_round(acc[t]) : acc[t];
  }
}

// ================================================ product chains (FP8) ===
// dsv4_gemv_fp8 / dsv4_gemv_fp8_tbl with the products formed apart from the
// chain. The reference's per-row loop acc += p[c] (p[c] = w[c] * xs[c] with
// xs = x * s, or (w[c] * x[c]) * s; each product rounded on its own, the
// build unfused; src/dsv4/dsv4_ops.c:176-239) adds products that do not
// depend on acc. So all four waves of a workgroup form its PC_ROWS rows'
// products into LDS (rows padded by 16 bytes, so that the chain lanes'
// reads of one column fall in distinct banks), and then one lane per row
// runs only the dependent adds, in column order, four products per LDS read
// and the next 32 products' reads in flight while 32 are added. (One lane
// per row decoding, scaling, multiplying and adding every column ran at
// about 23 cycles per column; an add chain alone runs at its dependency
// latency.) The rows of a workgroup share one row block (block a multiple of
// 16); in a multiple of 32, at most PC_MAXIN.
#define PC_ROWS 8
#define PC_MAXIN 4096

// acc + p[0] + ... + p[4 N4 - 1] in order, p in LDS (16-byte aligned): fully
// unrolled, so every read is one instruction with an immediate offset and
// the lane's instruction stream holds nothing but reads and the dependent
// adds (in a single wave every other instruction delays the chain by its
// issue time). The reads run PC_LA float4 ahead of the adds in a register
// ring; an empty asm on acc after each float4's adds pins that order (left
// to itself the compiler keeps only one or two reads in flight).
#define PC_LA 7
template <int N4>
__device__ __forceinline__ float pc_chain_fixed(const float4 *p4, float acc) {
  constexpr int LA = N4 < PC_LA ? N4 : PC_LA, R = LA + 1;
  float4 v[R];
#pragma unroll
  for (int j = 0; j < LA; ++j) v[j] = p4[j];
#pragma unroll
  for (int j = 0; j < N4; ++j) {
    if (j + LA < N4) v[(j + LA) % R] = p4[j + LA];
    const float4 c = v[j % R];
    acc = acc + c.x;
    acc = acc + c.y;
    acc = acc + c.z;
    acc = acc + c.w;
    asm volatile("" : "+v"(acc)::"memory");
  }
  return acc;
}

// The whole row's chain in one unrolled ring (no block boundaries, where the
// ring would restart), one 384-column load at a time (96 float4, unrolled
// within the compiler's limit; the loads chained by template recursion):
// wait(c) returns once the products of columns < c are in LDS, and is called
// before the first read of each load.
template <int J0, int N4, typename Wait>
__device__ __forceinline__ void pc_chain_seg(const float4 *p4, float &acc,
                                             float4 (&v)[PC_LA + 1], Wait &wait) {
  constexpr int LA = PC_LA, R = LA + 1;
#pragma unroll
  for (int jj = 0; jj < 96; ++jj) {
    const int j = J0 + jj;
    if (j >= N4) break;
    if (j + LA < N4) {
      if ((j + LA) % 96 == 0) wait(4 * (j + LA) + 4);
      v[(j + LA) % R] = p4[j + LA];
    }
    const float4 c = v[j % R];
    acc = acc + c.x;
    acc = acc + c.y;
    acc = acc + c.z;
    acc = acc + c.w;
    asm volatile("" : "+v"(acc)::"memory");
  }
  if constexpr (J0 + 96 < N4) pc_chain_seg<J0 + 96, N4>(p4, acc, v, wait);
}

template <int N4, typename Wait>
__device__ __forceinline__ float pc_chain_row(const float4 *p4, float acc, Wait &wait) {
  float4 v[PC_LA + 1];
  wait(4 * PC_LA);
#pragma unroll
  for (int j = 0; j < PC_LA; ++j) v[j] = p4[j];
  pc_chain_seg<0, N4>(p4, acc, v, wait);
  return acc;
}

// The products of piece k of the calling thread (16 columns of one row) into
// the row's LDS products: p = w * xs (MODE 0) or (w * x) * s (MODE 1).
template <int MODE>
__device__ __forceinline__ void pc_products(const uint4 w, int r, int c, const float *xs,
                                            const float *srow, int block, int ps, float *pr) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  const float sc = MODE == 1 ? srow[c / block] : 1.0f;
  float4 *dst = reinterpret_cast<float4 *>(pr + (size_t)r * ps + c);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float2 lo = fp8x2<false>(wd[d]), hi = fp8x2<true>(wd[d]);
    const float4 xv = *reinterpret_cast<const float4 *>(xs + c + 4 * d);
    float4 p;
    if (MODE == 0) {
      p = make_float4(lo.x * xv.x, lo.y * xv.y, hi.x * xv.z, hi.y * xv.w);
    } else {
      p = make_float4((lo.x * xv.x) * sc, (lo.y * xv.y) * sc, (hi.x * xv.z) * sc,
                      (hi.y * xv.w) * sc);
    }
    dst[d] = p;
  }
}

// x is loaded first (its loads would otherwise wait behind every weight load:
// the memory counter is in order), staged as x or x * s, then waves 1-3 form
// every product as their weight loads land, in column order: load k of a
// producer lane is piece (tid - 64) + 192 k, that is row i % PC_ROWS of the
// 16-column chunk i / PC_ROWS, so load k covers columns [384 k, 384 k + 384)
// of all rows; after its products of load k a producer wave counts itself in
// s_cnt[k]. Wave 0's chain lanes start as soon as the first 384 columns are
// counted and check a count only when the chain reaches a load not yet seen
// complete; so the chain starts after one load round trip, not half the row.
#define PC_LOADS ((PC_ROWS * PC_MAXIN / 16 + 191) / 192)  // weight loads per producer lane
#define PC_XQ (PC_MAXIN / 4 / 256)                         // x float4 per thread
template <int MODE>
__global__ __launch_bounds__(256) void k_fp8_prodchain(float *__restrict__ y,
                                                       const float *__restrict__ x,
                                                       const uint8_t *__restrict__ W,
                                                       const float *__restrict__ wscale, int in,
                                                       int rows, int block) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_cnt[PC_LOADS];
  const int tid = threadIdx.x, wave = tid >> 6, r0 = blockIdx.x * PC_ROWS;
  const int cblocks = (in + block - 1) / block;
  const int ps = in + 4;             // product row stride (floats)
  float *xs = lds;                   // [in] x (MODE 1) or x * s (MODE 0)
  float *pr = lds + in;              // [PC_ROWS][ps] products
  float *ss = pr + PC_ROWS * ps;     // [cblocks] the row block's scales
  const float *srow = wscale + (size_t)(r0 / block) * cblocks;
  const int npiece = PC_ROWS * (in / 16);
  const int nrow = min(PC_ROWS, rows - r0);
  // the scales and x are loaded before the weights: a wait for them then
  // leaves the weight loads in flight (the memory counter is in order)
  const float sv = tid < cblocks ? srow[tid] : 0.0f;
  float4 xv[PC_XQ];
#pragma unroll
  for (int q = 0; q < PC_XQ; ++q) {
    const int i = tid + 256 * q;
    xv[q] = i < in / 4 ? reinterpret_cast<const float4 *>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const BufRsrc rw = buf_rsrc(W + (size_t)r0 * in, (uint32_t)(nrow * in));
  // every wave issues the same loads (wave 0's out of range: zeros, no
  // memory access), so the wait for x below counts exactly PC_LOADS later
  // loads on every path instead of draining them all
  uint4 w[PC_LOADS];
#pragma unroll
  for (int k = 0; k < PC_LOADS; ++k) {
    const int i = tid - 64 + 192 * k;
    w[k] = buf_load16(rw, wave > 0 && i < npiece ? (uint32_t)(i % PC_ROWS) * (uint32_t)in +
                                                       16u * (uint32_t)(i / PC_ROWS)
                                                 : 0xFFFFFFF0u);
  }
  if (tid < PC_LOADS) s_cnt[tid] = 0;
  if (tid < cblocks) ss[tid] = sv;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < PC_XQ; ++q) {
    const int i = tid + 256 * q;
    if (i < in / 4) {
      float4 v = xv[q];
      if (MODE == 0) {  // xs = x * s of the row block (the 4 columns share a column block)
        const float sc = ss[(4 * i) / block];
        v = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
      }
      reinterpret_cast<float4 *>(xs)[i] = v;
    }
  }
  __syncthreads();
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < PC_LOADS; ++k) {
      const int i = tid - 64 + 192 * k;
      if (192 * k >= npiece) break;  // uniform
      if (i < npiece) pc_products<MODE>(w[k], i % PC_ROWS, 16 * (i / PC_ROWS), xs, ss, block, ps, pr);
      // this wave's product stores of load k are issued before the count (the
      // empty asm keeps the compiler from moving them past it; LDS runs a
      // wave's operations in order, so they land first): count the wave in
      asm volatile("" ::: "memory");
      if ((tid & 63) == 0) atomicAdd(&s_cnt[k], 1);
    }
    return;
  }
  if (tid >= PC_ROWS || tid >= nrow) return;
  const float4 *p4 = reinterpret_cast<const float4 *>(pr + (size_t)tid * ps);
  const int n4 = in / 4;  // a multiple of 8
  float acc = 0.0f;
  int ready = -1;  // loads known to be counted by all three producer waves
  auto wait_cols = [&](int cend) {  // products of columns < cend are in LDS
    const int need = (cend - 1) / 384;
    if (need <= ready) return;
    // (an LDS pointer: a generic one would make the read a FLAT one)
    const volatile __attribute__((address_space(3))) int *cnt =
        (const volatile __attribute__((address_space(3))) int *)&s_cnt[need];
    for (unsigned it = 0; *cnt < 3 && it < (1u << 24); ++it) __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");  // the product reads stay after the count's
    ready = need;
  };
  if (n4 == 1024) {  // the model's width: one ring over the whole row
    acc = pc_chain_row<1024>(p4, acc, wait_cols);
  } else {
    int b = 0;
#pragma unroll 1
    for (; b + 64 <= n4; b += 64) {
      wait_cols(4 * (b + 64));
      acc = pc_chain_fixed<64>(p4 + b, acc);
    }
    for (; b + 8 <= n4; b += 8) {
      wait_cols(4 * (b + 8));
      acc = pc_chain_fixed<8>(p4 + b, acc);
    }
  }
  y[r0 + tid] = acc;
}

// ================================================ batched BF16 rows ====
// dsv4_gemv_bf16_batch / head_logits_batch (src/dsv4/dsv4_model.c:266-367,
// 7371-7445) for many tokens, where the fp32 FMA issue rate, not HBM, is the
// bound (64 tokens through the 129280 x 4096 head: 34 G dependent-chain
// fmaf). Register blocking: lane = (row group rg = lane / 4, token group
// tg = lane % 4) keeps 4 rows x KT tokens of chains, so each weight is read
// and widened once for KT tokens and each x value read from LDS feeds 4 rows.
// x moves through LDS in blocks of 8 columns (double-buffered, the next
// block's weights and x in flight while the current block is chained); the
// four token groups' rows sit 4 floats apart in LDS so that one 16-byte read
// of all four hits distinct banks. Per (row, token) the fmaf chain runs in
// column order, as the reference's. The reads of token k + 1 are issued
// while token k is chained: an empty asm on token k's accumulators pins that
// order, or the compiler hoists all reads of a block and runs out of
// registers. in a multiple of 8, x 16-byte aligned; tokens [t0, t0 + 4 KT)
// all present.
template <int KT>
__global__ __launch_bounds__(64) void k_bf16_rows_blocked(float *__restrict__ y,
                                                          const float *__restrict__ x,
                                                          const uint16_t *__restrict__ W, int in,
                                                          int rows, int round_out, int t0) {
  constexpr int NT = 4 * KT;            // tokens of this launch
  constexpr int XS = NT * 8 + 16;       // one block: token t at 8 t + 4 (t / KT)
  constexpr int NQ = (2 * NT + 63) / 64;  // 16-byte x pieces per lane per block
  __shared__ __align__(16) float xs[2][XS];
  const int lane = threadIdx.x, rg = lane >> 2, tg = lane & 3;
  const int r0 = blockIdx.x * 64, rr = 4 * rg;
  const int nrow = min(64, rows - r0);
  const uint32_t rb = 2u * (uint32_t)in;
  const BufRsrc rw = buf_rsrc(W + (size_t)r0 * in, (uint32_t)nrow * rb);
  // rows past the tile's end read row 0 (in bounds) and are not stored
  const uint32_t ro0 = rr < nrow ? (uint32_t)rr * rb : 0u;
  const uint32_t ro1 = rr + 1 < nrow ? (uint32_t)(rr + 1) * rb : 0u;
  const uint32_t ro2 = rr + 2 < nrow ? (uint32_t)(rr + 2) * rb : 0u;
  const uint32_t ro3 = rr + 3 < nrow ? (uint32_t)(rr + 3) * rb : 0u;
  const float *xb = x + (size_t)t0 * in;
  // x staging: piece p = lane + 64 q (q < NQ <= 2) is token p / 2, columns
  // 4 (p % 2) .. + 3; a lane past the last piece re-reads it and stores nothing
  static_assert(NQ <= 2, "x staging holds two pieces per lane");
  const int p0 = min(lane, 2 * NT - 1), p1 = min(lane + 64, 2 * NT - 1);
  const float *xp0 = xb + (size_t)(p0 >> 1) * in + 4 * (p0 & 1);
  const float *xp1 = xb + (size_t)(p1 >> 1) * in + 4 * (p1 & 1);
  const int so0 = 4 * p0 + 4 * ((p0 >> 1) / KT);  // 8 t + 4 (p % 2) + 4 (t / KT)
  const int so1 = 4 * p1 + 4 * ((p1 >> 1) / KT);
  const bool st0 = lane < 2 * NT, st1 = NQ > 1 && lane + 64 < 2 * NT;
  float acc[4][KT];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < KT; ++k) acc[j][k] = 0.0f;
  uint4 w0 = buf_load16(rw, ro0), w1 = buf_load16(rw, ro1), w2 = buf_load16(rw, ro2),
        w3 = buf_load16(rw, ro3);
  float4 xr0 = *reinterpret_cast<const float4 *>(xp0), xr1 = xr0;
  if (NQ > 1) xr1 = *reinterpret_cast<const float4 *>(xp1);
  if (st0) *reinterpret_cast<float4 *>(&xs[0][so0]) = xr0;
  if (st1) *reinterpret_cast<float4 *>(&xs[0][so1]) = xr1;
  __syncthreads();
  const int rd = 8 * KT * tg + 4 * tg;  // token KT tg of this lane's group
  int b = 0;
  for (int c0 = 0; c0 < in; c0 += 8) {
    const bool more = c0 + 8 < in;
    uint4 n0, n1, n2, n3;
    if (more) {
      const uint32_t o = 2u * (uint32_t)(c0 + 8);
      n0 = buf_load16(rw, ro0 + o);
      n1 = buf_load16(rw, ro1 + o);
      n2 = buf_load16(rw, ro2 + o);
      n3 = buf_load16(rw, ro3 + o);
      xr0 = *reinterpret_cast<const float4 *>(xp0 + c0 + 8);
      if (NQ > 1) xr1 = *reinterpret_cast<const float4 *>(xp1 + c0 + 8);
    }
    float wv[4][8];
    const uint4 wq[4] = {w0, w1, w2, w3};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wd[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wv[j][2 * k] = u2f(wd[k] << 16);
        wv[j][2 * k + 1] = u2f(wd[k] & 0xFFFF0000u);
      }
    }
    const float *xl = &xs[b][rd];
    float4 na = *reinterpret_cast<const float4 *>(xl);
    float4 nb = *reinterpret_cast<const float4 *>(xl + 4);
#pragma unroll
    for (int k = 0; k < KT; ++k) {
      const float4 xa = na, xc = nb;
      if (k + 1 < KT) {
        na = *reinterpret_cast<const float4 *>(xl + 8 * (k + 1));
        nb = *reinterpret_cast<const float4 *>(xl + 8 * (k + 1) + 4);
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float a = acc[j][k];
        a = fmaf(wv[j][0], xa.x, a);
        a = fmaf(wv[j][1], xa.y, a);
        a = fmaf(wv[j][2], xa.z, a);
        a = fmaf(wv[j][3], xa.w, a);
        a = fmaf(wv[j][4], xc.x, a);
        a = fmaf(wv[j][5], xc.y, a);
        a = fmaf(wv[j][6], xc.z, a);
        a = fmaf(wv[j][7], xc.w, a);
        acc[j][k] = a;
      }
      asm volatile("" : "+v"(acc[0][k]), "+v"(acc[1][k]), "+v"(acc[2][k]), "+v"(acc[3][k]));
    }
    if (more) {
      if (st0) *reinterpret_cast<float4 *>(&xs[b ^ 1][so0]) = xr0;
      if (st1) *reinterpret_cast<float4 *>(&xs[b ^ 1][so1]) = xr1;
      w0 = n0;
      w1 = n1;
      w2 = n2;
      w3 = n3;
    }
    __syncthreads();
    b ^= 1;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = r0 + rr + j;
    if (row < rows) {
#pragma unroll
      for (int k = 0; k < KT; ++k) {
        const float v = acc[j][k];
        y[(size_t)(t0 + KT * tg + k) * rows + row] = round_out ? bf16_round(v) : v;
      }
    }
  }
}

// The same chains for 1 to 3 tokens (decode, and the remainder of a batch
// split into runs of 4 KT), where HBM is the bound: a lane per output row
// reading its own row would touch 64 cache lines per load, so the wave loads
// tiles of 64 rows x 64 columns coalesced (lane l: rows 8 i + l / 8, 16
// bytes at column 8 (l % 8)), writes them to LDS (rows 144 bytes apart, so
// that the lanes' row reads hit distinct banks) and reads back its own row's
// 64 columns. Two tiles are in flight while one is chained; x enters each
// fmaf as a scalar operand. LDS holds one tile: the wave's LDS accesses run
// in order, and the empty asms keep the compiler from moving them across
// each other. in a multiple of 64; tokens [t0, t0 + TB) present.
#define RT_DEPTH 2
template <int TB>
__global__ __launch_bounds__(64) void k_bf16_rows_tiled(float *__restrict__ y,
                                                        const float *__restrict__ x,
                                                        const uint16_t *__restrict__ W, int in,
                                                        int rows, int round_out, int t0) {
  __shared__ __align__(16) uint4 tl[64 * 9];
  const int lane = threadIdx.x, r0 = blockIdx.x * 64;
  const int nrow = min(64, rows - r0);
  const uint32_t rb = 2u * (uint32_t)in;
  const BufRsrc rw = buf_rsrc(W + (size_t)r0 * in, (uint32_t)nrow * rb);
  const int lr = lane >> 3, lp = lane & 7;
  const uint32_t lo = (uint32_t)lr * rb + 16u * lp;  // tile t, rows 8 i + lr: + 8 rb i + 128 t
  const int nt = in / 64;
  typedef const __attribute__((address_space(4))) float cfloat;
  cfloat *xc = (cfloat *)(x + (size_t)t0 * in);
  uint4 T[RT_DEPTH][8];
#pragma unroll
  for (int d = 0; d < RT_DEPTH; ++d)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      T[d][i] = buf_load16(rw, d < nt ? lo + 8u * rb * i + 128u * d : 0xFFFFFFF0u);
  float acc[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) acc[t] = 0.0f;
  for (int tb = 0; tb < nt; tb += RT_DEPTH) {
#pragma unroll
    for (int d = 0; d < RT_DEPTH; ++d) {
      const int t = tb + d;
      if (t >= nt) break;  // uniform
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < 8; ++i) tl[(8 * i + lr) * 9 + lp] = T[d][i];
      if (t + RT_DEPTH < nt) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          T[d][i] = buf_load16(rw, lo + 8u * rb * i + 128u * (t + RT_DEPTH));
      }
      asm volatile("" ::: "memory");
      uint4 m[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) m[k] = tl[lane * 9 + k];
      asm volatile("" ::: "memory");
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t wd[4] = {m[k].x, m[k].y, m[k].z, m[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 64 * t + 8 * k + 2 * e;
          const float wl = u2f(wd[e] << 16), wh = u2f(wd[e] & 0xFFFF0000u);
#pragma unroll
          for (int u = 0; u < TB; ++u) {
            acc[u] = fmaf(wl, xc[(size_t)u * in + c], acc[u]);
            acc[u] = fmaf(wh, xc[(size_t)u * in + c + 1], acc[u]);
          }
        }
      }
    }
  }
  if (lane >= nrow) return;
#pragma unroll
  for (int u = 0; u < TB; ++u)
    y[(size_t)(t0 + u) * rows + r0 + lane] = round_out ? bf16_round(acc[u]) : acc[u];
}

// ======================================================= greedy pick ===
// The CLI's greedy token (src/cli/dsv4_run.c:357-359): best = 0, then every
// v with logits[v] > logits[best] in order; so the first index of the
// largest value, NaNs never taken, and 0 when logits[0] is NaN. One
// workgroup per row: each thread keeps its first largest non-NaN value of
// v = tid, tid + 256, ..., then (value, index) pairs merge with the larger
// value, or the smaller index on equal values.
__device__ __forceinline__ void am_merge(float &bv, int &bi, float ov, int oi) {
  if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
    bv = ov;
    bi = oi;
  }
}

__global__ __launch_bounds__(256) void k_argmax(int *idx, const float *logits, int vocab,
                                                size_t stride) {
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  const int tid = threadIdx.x;
  const float *l = logits + (size_t)blockIdx.x * stride;
  float bv = 0.0f;
  int bi = -1;
  for (int v = tid; v < vocab; v += 256) {
    const float f = l[v];
    if (f == f && (bi < 0 || f > bv)) {
      bv = f;
      bi = v;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    am_merge(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  if (tid % 64 == 0) {
    s_v[tid / 64] = bv;
    s_i[tid / 64] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) am_merge(bv, bi, s_v[w], s_i[w]);
    const float f0 = l[0];
    idx[blockIdx.x] = (f0 != f0 || bi < 0) ? 0 : bi;
  }
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

template <int NP>
static void launch_fp4_t(const GemvArgs *a, int nvec, int pair, hipStream_t st) {
  const Fp4Geom q = fp4_geom_np(a->in, NP);
  const int span = pair ? q.tr / 2 : q.tr;
  const dim3 grid((unsigned)((a->rows + span - 1) / span), (unsigned)nvec);
  const size_t lds = (size_t)q.tr * pair_stride(q.G) * 8 + 4096 + ((a->in + 15) & ~15) +
                     (size_t)((a->in + 127) / 128) * 4;
  hipLaunchKernelGGL(k_gemv_fp4_t<NP>, grid, dim3(256), lds, st, *a, pair);
}

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
  hipStream_t st = (hipStream_t)stream;
  // passes per tile: the most that still give about 1024 workgroups (paired
  // tiles hold at least one pass of each matrix)
  const int pair = nmat == 2;
  int np = 16;
  while (np > (pair ? 2 : 1)) {
    const int tr = fp4_geom_np(a->in, np).tr, span = pair ? tr / 2 : tr;
    if ((long)((a->rows + span - 1) / span) * nvec >= 1024) break;
    np /= 2;
  }
  if (a->np) np = a->np;
  switch (np) {
    case 1: launch_fp4_t<1>(a, nvec, pair, st); break;
    case 2: launch_fp4_t<2>(a, nvec, pair, st); break;
    case 4: launch_fp4_t<4>(a, nvec, pair, st); break;
    case 8: launch_fp4_t<8>(a, nvec, pair, st); break;
    default: launch_fp4_t<16>(a, nvec, pair, st); break;
  }
  return dsv4g_check_launch("gemv_fp4");
}

int dsv4g_launch_gemv_fp8(const GemvArgs *a, int nvec, int nmat, void *stream) {
  if (fp8_shape_ok(a->in, "gemv_fp8")) return DSV4G_EINVAL;
  if (a->rows <= 0 || nvec <= 0) return dsv4g_fail(DSV4G_EINVAL, "gemv_fp8: bad size");
  hipStream_t st = (hipStream_t)stream;
  // lanes per row: one 128-column block per lane up to 32 blocks (more
  // workgroups, so more weight loads in flight: 4096-wide rows 6.3 -> 5.4 us
  // at 1024 and 512 rows), two beyond (8192-wide rows: one block per lane
  // measured no faster at one token and slower at five), at least 8 lanes
  // per row (shorter rows: a lane per block, the rest idle)
  // tokens four at a time only when the row tiles alone fill the GPU (a
  // smaller matrix runs one token per workgroup, all tokens in parallel)
  const int CB = (a->in + 127) / 128;
  const int sl = CB <= 8 ? 8 : CB <= 16 ? 16 : 32;
  // (and the four tokens' activations fit LDS beside the rest: in <= 2048)
  const bool many = nvec > 1 && a->in <= 2048 &&
                    (long)(a->rows + 256 / sl - 1) / (256 / sl) * nmat >= 1024;
  switch (sl * (many ? 10 : 1)) {
    case 8: launch_fp8_proj<8, 1>(a, nvec, nmat, st); break;
    case 16: launch_fp8_proj<16, 1>(a, nvec, nmat, st); break;
    case 80: launch_fp8_proj<8, 4>(a, nvec, nmat, st); break;
    case 160: launch_fp8_proj<16, 4>(a, nvec, nmat, st); break;
    default: launch_fp8_proj<32, 1>(a, nvec, nmat, st); break;
  }
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
  const size_t xb = (size_t)batch * in * 4;
  if (in % 64 == 0 && ((uintptr_t)x & 15) == 0 && (size_t)64 * in * 2 < 0xFFFF0000u) {
    // runs of 64, 32, 16, 8 or 4 tokens through the register-blocked chains,
    // a remainder of 1 to 3 through the tiled chains
    const dim3 grid((out + 63) / 64);
    for (int t0 = 0; t0 < batch;) {
      const int rem = batch - t0;
      const int tb = rem >= 64 ? 64 : rem >= 32 ? 32 : rem >= 16 ? 16 : rem >= 8 ? 8 : rem >= 4 ? 4
                                                                                      : rem;
      auto k = tb == 64 ? k_bf16_rows_blocked<16> : tb == 32 ? k_bf16_rows_blocked<8>
               : tb == 16 ? k_bf16_rows_blocked<4> : tb == 8 ? k_bf16_rows_blocked<2>
               : tb == 4 ? k_bf16_rows_blocked<1> : tb == 3 ? k_bf16_rows_tiled<3>
               : tb == 2 ? k_bf16_rows_tiled<2> : k_bf16_rows_tiled<1>;
      hipLaunchKernelGGL(k, grid, dim3(64), 0, (hipStream_t)stream, y, x, W, in, out, round_out,
                         t0);
      DSV4G_TRY(dsv4g_check_launch("gemv_bf16"));
      t0 += tb;
    }
    return 0;
  }
  if (in % 8 == 0 && xb <= RC_XBYTES && (size_t)64 * in * 2 < 0xFFFF0000u &&
      ((uintptr_t)x & 15) == 0) {
    RowChainArgs a = {};
    a.y = y;
    a.x = x;
    a.W = reinterpret_cast<const uint8_t *>(W);
    a.in = in;
    a.rows = out;
    a.batch = batch;
    a.round_out = round_out;
    a.y_stride = (size_t)out;
    a.x_stride = (size_t)in;
    const dim3 grid((out + 63) / 64);
    if (batch == 1)
      hipLaunchKernelGGL((k_rowchain<RC_BF16, 1>), grid, dim3(64), xb, (hipStream_t)stream, a);
    else if (batch <= 4)
      hipLaunchKernelGGL((k_rowchain<RC_BF16, 4>), grid, dim3(64), xb, (hipStream_t)stream, a);
    else if (batch <= 8)
      hipLaunchKernelGGL((k_rowchain<RC_BF16, 8>), grid, dim3(64), xb, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((k_rowchain<RC_BF16, 33>), grid, dim3(64), xb, (hipStream_t)stream, a);
    return dsv4g_check_launch("gemv_bf16");
  }
  dim3 grid((out + 63) / 64, batch);
  hipLaunchKernelGGL(k_gemv_bf16, grid, dim3(64), 0, (hipStream_t)stream, y, x, W, in, out,
                     round_out, (size_t)out, (size_t)in);
  return dsv4g_check_launch("gemv_bf16");
}

int dsv4g_argmax(int *idx, const float *logits, int vocab, int n, size_t stride,
                 void *stream) {
  if (!idx || !logits || vocab <= 0 || n <= 0 || stride < (size_t)vocab)
    return dsv4g_fail(DSV4G_EINVAL, "argmax: bad arguments");
  hipLaunchKernelGGL(k_argmax, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream, idx,
                     logits, vocab, stride);
  return dsv4g_check_launch("argmax");
}

int dsv4g_gemv_fp8_float(float *y, const float *x, const uint8_t *W, const float *wscale,
                         int in, int rows, int block, int mode, void *stream) {
  if (in <= 0 || rows <= 0 || block <= 0)
    return dsv4g_fail(DSV4G_EINVAL, "gemv_fp8_float: bad size");
  if (in % 32 == 0 && in <= PC_MAXIN && block % 16 == 0 && ((uintptr_t)x & 15) == 0) {
    const size_t lds = ((size_t)in + (size_t)PC_ROWS * (in + 4) + (in + block - 1) / block) * 4;
    const void *fn = mode == 0 ? (const void *)k_fp8_prodchain<0> : (const void *)k_fp8_prodchain<1>;
    // more than the default 64 KB of LDS (a host-side setting of the kernel)
    DSV4G_HIP(hipFuncSetAttribute(
        fn, hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)(((size_t)PC_MAXIN + (size_t)PC_ROWS * (PC_MAXIN + 4) + PC_MAXIN / 16) * 4)));
    const dim3 grid((unsigned)((rows + PC_ROWS - 1) / PC_ROWS));
    if (mode == 0)
      hipLaunchKernelGGL(k_fp8_prodchain<0>, grid, dim3(256), lds, (hipStream_t)stream, y, x, W,
                         wscale, in, rows, block);
    else
      hipLaunchKernelGGL(k_fp8_prodchain<1>, grid, dim3(256), lds, (hipStream_t)stream, y, x, W,
                         wscale, in, rows, block);
    return dsv4g_check_launch("gemv_fp8_float");
  }
  if (in % 16 == 0 && block % 16 == 0 && (size_t)in * 4 * 2 <= RC_XBYTES &&
      ((uintptr_t)x & 15) == 0) {
    RowChainArgs a = {};
    a.y = y;
    a.x = x;
    a.W = W;
    a.wscale = wscale;
    a.in = in;
    a.rows = rows;
    a.block = block;
    a.batch = 1;
    const dim3 grid((rows + 63) / 64);
    const size_t xb = (size_t)in * 4 + (size_t)(64 / block + 2) * ((in + block - 1) / block) * 4;
    if (mode == 0 && block % 64 == 0)
      hipLaunchKernelGGL((k_rowchain<RC_FP8_XS, 1>), grid, dim3(64), xb, (hipStream_t)stream, a);
    else if (mode == 0)
      hipLaunchKernelGGL((k_rowchain<RC_FP8_X, 1>), grid, dim3(64), xb, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((k_rowchain<RC_FP8_T, 1>), grid, dim3(64), xb, (hipStream_t)stream, a);
    return dsv4g_check_launch("gemv_fp8_float");
  }
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
