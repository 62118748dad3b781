// dsv4_hc.hip - the caller's step around the MoE layer on gfx950: the
// Hyper-Connection pre/post mixes and RMSNorm of forward_loaded_layer
// (src/dsv4/dsv4_model.c:7512-7559), so a decode step keeps its residual
// state in HBM from one layer to the next. Bit-exact with the reference:
//
//  - hc_pre (src/dsv4/dsv4_model.c:7123-7156): 24 mixes (mult 4), each an
//    fmaf chain over mult*hidden = 16384 products in index order. The chains
//    are run as they are, one lane per chain, in wave 0 of a workgroup per
//    token; the other waves stream the rows and the state through an LDS ring
//    in 128-column chunks so the chains never wait on HBM. The kernel's time
//    is the chain's dependent-FMA latency (16384 steps), not bandwidth.
//  - the sums of squares of hc_pre and rmsnorm_bf16 (src/dsv4/dsv4_model.c:
//    4934-4951) are sequential double sums in the reference. Here they are
//    summed in parallel; every term is exact (a float squared fits a double),
//    so the sequential sum lies within n * 2^-53 (relative) of the parallel
//    one. When both ends of that interval give the same float scale the scale
//    is exact; otherwise (a sum within ~2^-38 of a float rounding boundary) one
//    lane repeats the sum in index order.
//  - dsv4_hc_split (src/dsv4/dsv4_ops.c:415-466) runs on the lanes of one wave,
//    one lane per comb entry, each row and column sum formed in index order;
//    expf is the bit-exact restatement of the host libm's.
#include <algorithm>

#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"

namespace {

using namespace dsv4;

constexpr int HC_C = 192;          // columns per staged chunk (12 groups of 16)
constexpr int HC_RS = HC_C + 4;    // LDS row stride of a chunk (floats)
constexpr int HC_MAX_MULT = 7;     // mix_n = (2 + mult) * mult <= 63 chains
constexpr int HC_MAX_RING = 6;     // staging slots
constexpr size_t HC_LDS_BUDGET = 150 * 1024;
constexpr unsigned HC_SPIN_CAP = 1u << 22;

struct HcArgs {
  float *bin, *post, *comb;     // [n][hid], [n][mult], [n][mult*mult]
  const float *state;           // [n][mult*hid]
  const float *fn;              // [mix_n][mult*hid]
  const float *scale3, *base;   // [3], [mix_n]
  const uint16_t *norm_w;       // [hid] BF16 gain: rmsnorm_bf16(bin, bin, w, .., 1)
  unsigned *status;             // sticky error word (a spin ran out), or null
  int mult, hid, iters, ring;
  float rms_eps, hc_eps;
};

// 1/sqrtf((float)(s/n) + eps): the scale of rmsnorm_bf16 and hc_pre.
__device__ __forceinline__ float rms_scale(double s, int n, float eps) {
  return 1.0f / sqrtf((float)(s / (double)n) + eps);
}

// The scale for the sequential double sum of n exact non-negative terms whose
// sum, formed in another order, is est; *exact false when the interval of
// possible sequential sums straddles a change of the float scale.
__device__ __forceinline__ float rms_scale_bounded(double est, int n, float eps, bool *exact) {
  const double d = 2.0 * ((double)n + 64.0) * 0x1p-53;
  const float lo = rms_scale(est * (1.0 - d), n, eps);
  const float hi = rms_scale(est * (1.0 + d), n, eps);
  *exact = __float_as_uint(lo) == __float_as_uint(hi);
  return lo;
}

__device__ __forceinline__ double wave_sum_d(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ int ld_flag(int *f) {
  return __hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_flag(int *f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Relaxed forms for the ring's hot path. The ring is in LDS, whose operations
// from one wave execute in program order (and the compiler keeps that order:
// each use sits between asm memory barriers), so a flag store issued after a
// wave's reads of a slot takes effect after those reads have returned, and a
// flag read issued before a wave's reads of a slot precedes them. Waiting for
// a relaxed load waits only for the operations issued before it, not for the
// reads issued after it, so the consumer's look-ahead is not drained.
__device__ __forceinline__ int ld_flag_relaxed(int *f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_flag_relaxed(int *f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until *f == want; false (and the status word set) if the bounded spin
// ran out, which only a broken ring could cause.
__device__ bool wait_flag(int *f, int want, unsigned *status) {
  for (unsigned k = 0; ld_flag(f) != want; k++) {
    if (k == HC_SPIN_CAP) {
      if (status) atomicOr(status, 2u);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// expf-based logistic of the reference's hc_split (src/dsv4/dsv4_ops.c:401-409).
__device__ __forceinline__ float hc_sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + dsv4_libm_expf_t(-x, dsv4_libm_exp2_tab));
  const float e = dsv4_libm_expf_t(x, dsv4_libm_exp2_tab);
  return e / (1.0f + e);
}

// dsv4_hc_split on the lanes of one wave (call from a whole wave): lane
// i < m gets pre[i], post[i]; lane a*m + b < m*m gets comb[a][b]. mixes: LDS.
// M: m when known at compile time (the model's 4), else 0. With M the row and
// column sums of the Sinkhorn passes fetch their M terms with independent
// shuffles (one LDS round trip per pass instead of M dependent ones) and add
// them in index order.
template <int M>
__device__ void hc_split_wave_t(float *pre, float *post, float *comb, const float *mixes,
                                const float *scale3, const float *base, int m_rt, int iters,
                                float eps) {
  const int m = M ? M : m_rt;
  const int lane = threadIdx.x & 63;
  if (lane < m) {
    pre[lane] = hc_sigmoid(mixes[lane] * scale3[0] + base[lane]) + eps;
    post[lane] = 2.0f * hc_sigmoid(mixes[m + lane] * scale3[1] + base[m + lane]);
  }
  const int mm = m * m;
  const int a = lane < mm ? lane / m : 0, b = lane < mm ? lane % m : 0;
  const int k = lane < mm ? lane : 0;
  float v = mixes[2 * m + k] * scale3[2] + base[2 * m + k];
  // row softmax + eps
  float mx = __shfl(v, a * m);
  for (int j = 1; j < m; j++) {
    const float c = __shfl(v, a * m + j);
    mx = c > mx ? c : mx;
  }
  const float ev = dsv4_libm_expf_t(v - mx, dsv4_libm_exp2_tab);
  float s = 0.0f;
  for (int j = 0; j < m; j++) s += __shfl(ev, a * m + j);
  v = ev / s + eps;
  // one column pass, then iters-1 (row, column) passes
  for (int pass = 0; pass < 2 * iters - 1; pass++) {
    const bool by_col = (pass & 1) == 0;
    s = 0.0f;
    if (M) {
      float t[M ? M : 1];
#pragma unroll
      for (int j = 0; j < M; j++) t[j] = __shfl(v, by_col ? j * M + b : a * M + j);
#pragma unroll
      for (int j = 0; j < M; j++) s += t[j];
    } else {
      for (int j = 0; j < m; j++) s += __shfl(v, by_col ? j * m + b : a * m + j);
    }
    v = v / (s + eps);
  }
  if (lane < mm) comb[lane] = v;
}

__device__ void hc_split_wave(float *pre, float *post, float *comb, const float *mixes,
                              const float *scale3, const float *base, int m, int iters,
                              float eps) {
  if (m == 4)
    hc_split_wave_t<4>(pre, post, comb, mixes, scale3, base, m, iters, eps);
  else
    hc_split_wave_t<0>(pre, post, comb, mixes, scale3, base, m, iters, eps);
}

// 16 columns of a chain's row and of the state from a staged chunk.
__device__ __forceinline__ void ld_group(float4 *w, float4 *x, const float *row,
                                         const float *st, int g) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    w[q] = *(const float4 *)(row + 16 * g + 4 * q);
    x[q] = *(const float4 *)(st + 16 * g + 4 * q);
  }
}

// acc = fmaf(w[i], x[i], acc) over the 16 columns in index order.
__device__ __forceinline__ void fma_group(float &acc, const float4 *w, const float4 *x) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    acc = fmaf(w[q].x, x[q].x, acc);
    acc = fmaf(w[q].y, x[q].y, acc);
    acc = fmaf(w[q].z, x[q].z, acc);
    acc = fmaf(w[q].w, x[q].w, acc);
  }
}

// A producer lane's share of every chunk: float4 k of a chunk is element
// f = lane + 64 k (row f / (HC_C/4): rows 0..mix_n-1 of fn, row mix_n the
// state; column 4 (f % (HC_C/4)) of the chunk). Addresses and LDS offsets are
// fixed per lane, so a full chunk costs one pointer step, one load and one
// LDS store per float4. Elements past the chunk's rows read the state (a
// valid address) and are stored into the row padding of row 0 (never read).
template <int PER>
struct HcLane {
  const float *src[PER];  // this producer's current chunk address of each element
  int step[PER];          // floats to its next chunk (0 past the chunk's rows)
  int col[PER];           // column within the chunk
  int dst[PER];           // float offset within a slot
};

// Lane addresses for the producer's first chunk c0; its chunks are nprod apart.
template <int PER>
__device__ __forceinline__ void hc_lane_init(HcLane<PER> &L, const float *fn,
                                             const float *state, int K, int mix_n, int c0,
                                             int nprod) {
  const int lane = threadIdx.x & 63, q4 = HC_C / 4, F = (mix_n + 1) * q4;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int f = lane + 64 * k, r = f / q4, col = 4 * (f % q4);
    const bool real = f < F;
    L.src[k] = real ? (r < mix_n ? fn + (size_t)r * K : state) + (size_t)c0 * HC_C + col : state;
    L.step[k] = real ? nprod * HC_C : 0;
    L.col[k] = real ? col : 0;
    L.dst[k] = real ? r * HC_RS + col : HC_C;
  }
}

// Chunk c (the producer's current one) into registers, zero past K; then the
// addresses step to the producer's next chunk.
template <int PER>
__device__ __forceinline__ void hc_load_chunk(float4 *v, HcLane<PER> &L, int K, int c) {
  const int c0 = c * HC_C;
  if (c0 + HC_C <= K) {
#pragma unroll
    for (int k = 0; k < PER; k++) v[k] = *(const float4 *)L.src[k];
  } else {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const bool ok = c0 + L.col[k] < K;  // K % 4 == 0: a float4 is all in or all out
      const float4 ld = *(const float4 *)(ok ? L.src[k] : L.src[k] - L.col[k]);
      v[k] = ok ? ld : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int k = 0; k < PER; k++) L.src[k] += L.step[k];
}

// Write the chunk into its (free) slot and mark the slot as holding chunk c.
template <int PER>
__device__ __forceinline__ void hc_store_chunk(const float4 *v, const HcLane<PER> &L, float *slot,
                                               int *flag, int c) {
#pragma unroll
  for (int k = 0; k < PER; k++) *(float4 *)(slot + L.dst[k]) = v[k];
  __asm__ volatile("" ::: "memory");  // the data writes are issued before the flag's
  if ((threadIdx.x & 63) == 0) st_flag_relaxed(flag, c + 1);
}

// One workgroup of NW waves (4 or 8) per token. The waves of a workgroup sit
// on the CU's four SIMDs in turn (wave w on SIMD w % 4), and the chain wave
// issues an instruction for every step of its 24 chains, so SIMD 0 is left
// to it: wave 0 runs the chains (at raised priority), wave SQW sums the
// state's squares (wave 4 of 8: briefly, then it waits at the barrier; wave
// 3 of 4), and the other waves (NPROD of them) stage chunks into the ring of
// a.ring slots. PER: float4 registers per producer lane,
// ceil((mix_n + 1) * HC_C / 4 / 64).
template <int PER, int NW>
__global__ void __launch_bounds__(64 * NW) k_hc_pre(HcArgs a) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  constexpr int SQW = NW == 8 ? 4 : 3, NPROD = NW == 8 ? 6 : 2;
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_full[HC_MAX_RING], s_done[HC_MAX_RING];
  __shared__ float s_mix[64], s_pre[8], s_post[8], s_comb[64];
  __shared__ double s_part[16];
  __shared__ float s_scale;

  const int t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = a.mult, hid = a.hid, K = m * hid, mix_n = (2 + m) * m;
  const int D = a.ring, NC = (K + HC_C - 1) / HC_C;
  const size_t slot_fl = (size_t)(mix_n + 1) * HC_RS;
  const float *state = a.state + (size_t)t * K;
  if (tid < HC_MAX_RING) {
    s_full[tid] = 0;
    s_done[tid] = 0;
  }
  __syncthreads();

  if (wave == 0) {
    __builtin_amdgcn_s_setprio(3);
    // ---- the chains: lane j < mix_n owns mixes[j]. A chunk is HC_C / 16
    // groups of 16 columns, zero-filled past K by the producers (fmaf(0, 0, acc)
    // returns acc, which is never -0: it starts at +0 and a sum rounding to
    // zero is +0). Three register sets in turn keep the LDS reads two groups
    // ahead of the FMAs; the first two groups of the next chunk are read
    // during the last two of this one. The empty asm statements tie acc so
    // the reads before one are issued before the FMAs after it.
    // Only the chain lanes run it (lane 0 is one), so each 16-byte LDS read
    // moves mix_n lanes' bytes rather than 64.
    float acc = 0.0f;
    if (lane < mix_n) {
    const size_t row_off = (size_t)lane * HC_RS, st_off = (size_t)mix_n * HC_RS;
    constexpr int GPC = HC_C / 16;  // groups per chunk (a multiple of 3)
    float4 w[3][4], x[3][4];
#define HC_TIE __asm__ volatile("" : "+v"(acc)::"memory")
#define HC_LD(k, b, g) ld_group(w[k], x[k], (b) + row_off, (b) + st_off, g)
    int slot = 0;
    wait_flag(&s_full[0], 1, a.status);
    HC_LD(0, lds, 0);
    HC_LD(1, lds, 1);
#pragma unroll 1
    for (int c = 0; c < NC; c++) {
      const float *b = lds + slot * slot_fl;
      const int nslot = slot + 1 == D ? 0 : slot + 1;
      const float *nb = b;  // past the last chunk: reads of this one, unused
      // the next chunk's flag, read now and looked at two groups before the end
      const int next = ld_flag_relaxed(&s_full[nslot]);
      HC_TIE;
#pragma unroll
      for (int g = 0; g < GPC; g++) {
        if (g + 2 == GPC && c + 1 < NC) {
          if (next != c + 2) wait_flag(&s_full[nslot], c + 2, a.status);
          nb = lds + nslot * slot_fl;
        }
        if (g + 2 < GPC)
          HC_LD((g + 2) % 3, b, g + 2);
        else
          HC_LD((g + 2) % 3, nb, g + 2 - GPC);
        HC_TIE;
        fma_group(acc, w[g % 3], x[g % 3]);
        HC_TIE;
      }
      // every read of this chunk was issued before this store: release its slot
      if (lane == 0) st_flag_relaxed(&s_done[slot], c / D + 1);
      HC_TIE;
      slot = nslot;
    }
#undef HC_LD
#undef HC_TIE
    }
    if (lane < mix_n) s_mix[lane] = acc;
    __builtin_amdgcn_s_setprio(0);
  } else if (wave != SQW) {
    // ---- producer p (of NPROD) stages chunks p, p + NPROD, ... into slot
    // c % D once the slot's previous chunk has been consumed (ticket s_done)
    const int p = wave - 1 - wave / 4;
    HcLane<PER> L;
    hc_lane_init<PER>(L, a.fn, state, K, mix_n, p, NPROD);
    float4 v[PER];
    for (int c = p; c < NC; c += NPROD) {
      hc_load_chunk<PER>(v, L, K, c);
      const int slot = c % D;
      wait_flag(&s_done[slot], c / D, a.status);
      hc_store_chunk<PER>(v, L, lds + slot * slot_fl, &s_full[slot], c);
    }
  } else {
    // ---- the state's sum of squares (exact terms, any order)
    double ss = 0.0;
    for (int i = 4 * lane; i < K; i += 256) {
      const float4 x = *(const float4 *)(state + i);
      const double x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
      ss += x0 * x0 + x1 * x1 + x2 * x2 + x3 * x3;
    }
    ss = wave_sum_d(ss);
    if (lane == 0) s_part[0] = ss;
  }
  __syncthreads();

  // ---- hc_pre's scale, the mixes and the split (wave 0)
  if (wave == 0) {
    if (lane == 0) {
      const double est = s_part[0];
      bool exact;
      float rs = rms_scale_bounded(est, K, a.rms_eps, &exact);
      if (!exact) {
        double ss = 0.0;
        for (int i = 0; i < K; i++) {
          const double d = (double)state[i];
          ss += d * d;
        }
        rs = rms_scale(ss, K, a.rms_eps);
      }
      s_scale = rs;
    }
    __builtin_amdgcn_wave_barrier();
    const float rs = s_scale;
    if (lane < mix_n) s_mix[lane] = s_mix[lane] * rs;
    __builtin_amdgcn_wave_barrier();
    hc_split_wave(s_pre, s_post, s_comb, s_mix, a.scale3, a.base, m, a.iters, a.hc_eps);
    if (lane < m) a.post[(size_t)t * m + lane] = s_post[lane];
    if (lane < m * m) a.comb[(size_t)t * m * m + lane] = s_comb[lane];
  }
  __syncthreads();

  // ---- bin = bf16(sum_i pre[i] * state[i][c]), then the optional RMSNorm
  float *s_bin = lds;  // the ring is free now
  double ss = 0.0;
  for (int c = tid; c < hid; c += blockDim.x) {
    float acc = 0.0f;
    for (int i = 0; i < m; i++) acc = fmaf(s_pre[i], state[(size_t)i * hid + c], acc);
    const float b = bf16_round(acc);
    s_bin[c] = b;
    ss += (double)b * (double)b;
  }
  float *out = a.bin + (size_t)t * hid;
  if (!a.norm_w) {
    for (int c = tid; c < hid; c += blockDim.x) out[c] = s_bin[c];
    return;
  }
  ss = wave_sum_d(ss);
  if (lane == 0) s_part[wave] = ss;
  __syncthreads();
  if (tid == 0) {
    double est = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) est += s_part[w];
    bool exact;
    float r = rms_scale_bounded(est, hid, a.rms_eps, &exact);
    if (!exact) {
      double s2 = 0.0;
      for (int c = 0; c < hid; c++) s2 += (double)s_bin[c] * (double)s_bin[c];
      r = rms_scale(s2, hid, a.rms_eps);
    }
    s_scale = r;
  }
  __syncthreads();
  const float r = s_scale;
  for (int c = tid; c < hid; c += blockDim.x)
    out[c] = bf16_round(s_bin[c] * r * bf16_to_f32(a.norm_w[c]));
}

// rmsnorm_bf16 over rows of x (one workgroup per row); y may alias x.
__global__ void __launch_bounds__(256) k_rmsnorm(float *y, const float *x, const uint16_t *w,
                                                 int n, size_t stride, float eps, int round_out) {
  __shared__ double s_part[4];
  __shared__ float s_r;
  const float *xr = x + (size_t)blockIdx.x * stride;
  float *yr = y + (size_t)blockIdx.x * stride;
  double ss = 0.0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) ss += (double)xr[i] * (double)xr[i];
  ss = wave_sum_d(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double est = ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3];
    bool exact;
    float r = rms_scale_bounded(est, n, eps, &exact);
    if (!exact) {
      double s2 = 0.0;
      for (int i = 0; i < n; i++) s2 += (double)xr[i] * (double)xr[i];
      r = rms_scale(s2, n, eps);
    }
    s_r = r;
  }
  __syncthreads();
  const float r = s_r;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float v = xr[i] * r;
    if (w) v = v * bf16_to_f32(w[i]);
    yr[i] = round_out ? bf16_round(v) : v;
  }
}

// hc_post: each thread owns one column c of one token (all mult rows), so the
// state is updated in place.
__global__ void __launch_bounds__(256) k_hc_post(float *state, const float *branch,
                                                 const float *post, const float *comb, int m,
                                                 int hid) {
  const int t = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= hid) return;
  float *st = state + (size_t)t * m * hid;
  const float *po = post + (size_t)t * m, *cb = comb + (size_t)t * m * m;
  float old[HC_MAX_MULT];
#pragma unroll
  for (int k = 0; k < HC_MAX_MULT; k++) old[k] = k < m ? st[(size_t)k * hid + c] : 0.0f;
  const float br = branch[(size_t)t * hid + c];
  for (int i = 0; i < m; i++) {
    float y = po[i] * br;
#pragma unroll
    for (int k = 0; k < HC_MAX_MULT; k++)
      if (k < m) y = fmaf(cb[i * m + k], old[k], y);
    st[(size_t)i * hid + c] = bf16_round(y);
  }
}

// dsv4_hc_split for n independent rows of mixes (one wave each).
__global__ void __launch_bounds__(64) k_hc_split(float *pre, float *post, float *comb,
                                                 const float *mixes, const float *scale3,
                                                 const float *base, int m, int iters,
                                                 float eps) {
  __shared__ float s_mix[64];
  const int t = blockIdx.x, mix_n = (2 + m) * m;
  if (threadIdx.x < mix_n) s_mix[threadIdx.x] = mixes[(size_t)t * mix_n + threadIdx.x];
  __syncthreads();
  hc_split_wave(pre + (size_t)t * m, post + (size_t)t * m, comb + (size_t)t * m * m, s_mix,
                scale3, base, m, iters, eps);
}

int hc_ring(int mult) {
  const size_t slot = (size_t)((2 + mult) * mult + 1) * HC_RS * sizeof(float);
  return (int)std::min<size_t>(HC_MAX_RING, HC_LDS_BUDGET / slot);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" {

int dsv4g_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps,
                       int round_out, int rows, void *stream) {
  if (!y || !x || n <= 0 || rows < 0)
    return dsv4g_fail(DSV4G_EINVAL, "rmsnorm_bf16: bad arguments");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), 0, (hipStream_t)stream, y, x, w, n,
                     (size_t)n, eps, round_out);
  return dsv4g_check_launch("rmsnorm_bf16");
}

int dsv4g_hc_split(float *pre, float *post, float *comb, const float *mixes,
                   const float *scale3, const float *base, int mult, int iters, float eps,
                   int n, void *stream) {
  if (!pre || !post || !comb || !mixes || !scale3 || !base || mult < 1 ||
      mult > HC_MAX_MULT || iters < 1 || n < 0)
    return dsv4g_fail(DSV4G_EINVAL, "hc_split: bad arguments (mult 1..%d)", HC_MAX_MULT);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_hc_split, dim3(n), dim3(64), 0, (hipStream_t)stream, pre, post, comb,
                     mixes, scale3, base, mult, iters, eps);
  return dsv4g_check_launch("hc_split");
}

int dsv4g_hc_pre(float *bin, float *post, float *comb, const float *state, const float *fn,
                 const float *scale3, const float *base, const uint16_t *norm_w, int mult,
                 int hidden, int iters, float rms_eps, float hc_eps, int n_tokens,
                 unsigned *status, void *stream) {
  if (!bin || !post || !comb || !state || !fn || !scale3 || !base || mult < 1 ||
      mult > HC_MAX_MULT || hidden < 4 || hidden % 4 || iters < 1 || n_tokens < 0)
    return dsv4g_fail(DSV4G_EINVAL, "hc_pre: bad arguments (mult 1..%d, hidden a multiple "
                      "of 4)", HC_MAX_MULT);
  if (!aligned16(state) || !aligned16(fn))
    return dsv4g_fail(DSV4G_EINVAL, "hc_pre: state and fn must be 16-byte aligned");
  if (n_tokens == 0) return 0;
  HcArgs a;
  a.bin = bin;
  a.post = post;
  a.comb = comb;
  a.state = state;
  a.fn = fn;
  a.scale3 = scale3;
  a.base = base;
  a.norm_w = norm_w;
  a.status = status;
  a.mult = mult;
  a.hid = hidden;
  a.iters = iters;
  a.ring = hc_ring(mult);
  a.rms_eps = rms_eps;
  a.hc_eps = hc_eps;
  const size_t ring = (size_t)a.ring * ((2 + mult) * mult + 1) * HC_RS * sizeof(float);
  const size_t lds = std::max(ring, (size_t)hidden * sizeof(float));
  if (lds > HC_LDS_BUDGET)
    return dsv4g_fail(DSV4G_EINVAL, "hc_pre: hidden %d too large", hidden);
  // mult <= 4: 8 waves, 6 of them producers (19 float4 each); larger mult:
  // 4 waves, 2 producers (48 float4 each)
  const int rows = (2 + mult) * mult + 1;
  if (rows * (HC_C / 4) <= 64 * 19)
    hipLaunchKernelGGL((k_hc_pre<19, 8>), dim3(n_tokens), dim3(64 * 8), lds,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((k_hc_pre<48, 4>), dim3(n_tokens), dim3(64 * 4), lds,
                       (hipStream_t)stream, a);
  return dsv4g_check_launch("hc_pre");
}

int dsv4g_hc_post(float *state, const float *branch, const float *post, const float *comb,
                  int mult, int hidden, int n_tokens, void *stream) {
  if (!state || !branch || !post || !comb || mult < 1 || mult > HC_MAX_MULT || hidden < 1 ||
      n_tokens < 0)
    return dsv4g_fail(DSV4G_EINVAL, "hc_post: bad arguments (mult 1..%d)", HC_MAX_MULT);
  if (n_tokens == 0) return 0;
  hipLaunchKernelGGL(k_hc_post, dim3((hidden + 255) / 256, n_tokens), dim3(256), 0,
                     (hipStream_t)stream, state, branch, post, comb, mult, hidden);
  return dsv4g_check_launch("hc_post");
}

// The FFN half of forward_loaded_layer (src/dsv4/dsv4_model.c:7549-7559) on
// device: hc_pre + rmsnorm_bf16 -> moe_forward -> hc_post. Workspace: the
// decode MoE workspace at its start (its status word also takes hc_pre's),
// and x [n][hid], out [n][hid], post [n][mult], comb [n][mult*mult] at its
// end. The end of the workspace does not move with the call's token count,
// while the MoE workspace's token pieces grow from its start: a call with
// fewer tokens than the workspace was sized for never writes over the
// records and flags of a later call's extra tokens (they must stay zero).
static size_t ffn_align(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t ffn_tail_bytes(const DSV4GLayer *L, int mult, int n_tokens) {
  const size_t n = (size_t)n_tokens, H = (size_t)L->hidden, m = (size_t)mult;
  return 2 * ffn_align(n * H * 4) + ffn_align(n * m * 4) + ffn_align(n * m * m * 4);
}

size_t dsv4g_ffn_step_workspace_bytes(const DSV4GLayer *L, int mult, int n_tokens) {
  if (!L || n_tokens <= 0 || mult < 1 || mult > HC_MAX_MULT) return 0;
  const size_t moe = dsv4g_moe_workspace_bytes(L, n_tokens);
  if (!moe) return 0;
  return ffn_align(moe) + ffn_tail_bytes(L, mult, n_tokens);
}

int dsv4g_ffn_step(float *state, const float *hc_fn, const float *hc_scale,
                   const float *hc_base, const uint16_t *ffn_norm, const DSV4GLayer *L,
                   const int *token_ids, int n_tokens, int mult, int iters, float rms_eps,
                   float hc_eps, void *workspace, size_t workspace_bytes, int *idx_out,
                   float *wt_out, void *stream) {
  if (!L || !workspace || ((uintptr_t)workspace & 255))
    return dsv4g_fail(DSV4G_EINVAL, "ffn_step: layer and 256-byte aligned workspace needed");
  const size_t need = dsv4g_ffn_step_workspace_bytes(L, mult, n_tokens);
  if (!need || workspace_bytes < need)
    return dsv4g_fail(DSV4G_EINVAL, "ffn_step: workspace of %zu bytes, %zu needed",
                      workspace_bytes, need);
  const size_t n = (size_t)n_tokens, H = (size_t)L->hidden, m = (size_t)mult;
  const size_t moe = dsv4g_moe_workspace_bytes(L, n_tokens);
  uint8_t *p = (uint8_t *)workspace;
  // 256-byte aligned start of the tail; at or past ffn_align(moe) since
  // workspace_bytes >= need
  const size_t tail0 = (workspace_bytes - ffn_tail_bytes(L, mult, n_tokens)) & ~(size_t)255;
  float *x = (float *)(p + tail0);
  float *out = x + ffn_align(n * H * 4) / 4;
  float *post = out + ffn_align(n * H * 4) / 4;
  float *comb = post + ffn_align(n * m * 4) / 4;
  DSV4G_TRY(dsv4g_hc_pre(x, post, comb, state, hc_fn, hc_scale, hc_base, ffn_norm, mult,
                         L->hidden, iters, rms_eps, hc_eps, n_tokens,
                         dsv4g_decode_status_word(workspace), stream));
  DSV4G_TRY(dsv4g_moe_forward(out, x, L, token_ids, n_tokens, workspace, moe, idx_out, wt_out,
                              stream));
  return dsv4g_hc_post(state, out, post, comb, mult, L->hidden, n_tokens, stream);
}

}  // extern "C"
