// dsv4_grouped.hip - the batched MoE layer for gfx950 (speculative verify and
// prefill): moe_forward_batch (src/dsv4/dsv4_model.c:6812-7117) as grouped
// GEMMs on the CDNA4 BF16 MFMA with exact FP4/FP8 x E8M0 operands.
//
// Pipeline (one stream):
//   1. activations -> FP8 E4M3 codes + per-128 E8M0 scale codes
//      (the reference's activation quant, exact);
//   2. router: BF16 MFMA logits with sum|g*x| for a rigorous error bound,
//      candidate experts per token, exact sequential fmaf chains for the
//      candidates, then the reference's selection and weights - indices and
//      weights identical to the reference (up to 256 tokens: logits,
//      candidates, and chains with the selection fused into the token's last
//      chain workgroup - three launches);
//   3. dispatch: deterministic per-expert position lists (ascending token, as
//      expert_forward_batch_routes gathers them, src/dsv4/dsv4_model.c:6498-6524)
//      and a token-tile table (one workgroup up to 1024 routes); the shared
//      expert is expert number E;
//   4. gate/up grouped GEMM on V_MFMA_F32_16X16X32_BF16: FP4 (routed) or FP8
//      (shared) weights are converted in registers to BF16 already multiplied
//      by their E8M0 block scale (V_CVT_SCALEF32_PK_BF16_FP4/FP8, exact: at
//      most 4 significant bits times a power of two), activations are the
//      exact BF16 dequantisation of their FP8 quantisation; epilogue = BF16
//      round of gate/up, SwiGLU, x route weight, BF16 round, per-128 FP8
//      requant (one 128-row tile = one requant group), stored dequantised;
//   5. down grouped GEMM, BF16 outputs per (token, route);
//   6. per-token combine in ascending expert id + shared, BF16.
// The products are exact; the MFMA sums them in fp32 in its own order, so
// expert outputs agree with the reference to fp32 rounding, not bit for bit;
// routing is exact. (The block-scaled FP8/FP4 MFMA was measured to sum each
// 128-K window with only ~12 bits below its largest product - error up to
// 2^-11 of the largest term - which moves results by ~5e-3; its FP8-rate
// throughput is not used for that reason.)
#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"

#include <mutex>

using namespace dsv4;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

namespace dsv4 {

#define GT_TN 64     // positions (tokens) per tile: 4 MFMA column fragments
#define GT_TM 128    // weight rows per tile: 4 waves x 2 fragments of 16
#define GT_BROW 144  // LDS bytes per staged activation row (128 + 16 pad)
#define MX_FP8 0
#define MX_FP4 4

__device__ __forceinline__ v8i u4x2_to_v8i(uint4 a, uint4 b) {
  v8i r;
  r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
  r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
  return r;
}

template <int AFMT>
__device__ __forceinline__ v4f mx_mfma(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, AFMT, MX_FP8, 0, sa, 0, sb);
}

__device__ __forceinline__ uint32_t scale_code(float s) { return (f2u(s) >> 23) & 0xFFu; }

// Operand layouts of V_MFMA_SCALE_F32_16X16X128_F8F6F4 (measured on gfx950 with
// the test library's probe, probe/dsv4_probe.hip): lane l serves row/column l%16; with g = l/16,
//   4-bit operand: nibbles 0..31 (4 VGPRs) = K 32g .. 32g+31, low nibble first;
//   8-bit operand: bytes 0..15 = K 16g .. 16g+15, bytes 16..31 = K 64+16g ..;
//   scale byte of lane l = E8M0 scale of K block g (K 32g .. 32g+31);
//   result: lane l holds D[4g + v][l%16], v = 0..3.

// ------------------------------------------------------- batch quant ----
// The reference activation quant per (token, 128-group), stored as the
// exact BF16 value of each quantised element (E4M3 grid value x scale), and
// per 256-column piece of a token a flag: 1 when a value of x in it is not
// BF16-valued (the router bound then widens), written either way; and
// zeroes *zero (the route placement's counter) for the kernels after it.
// 16-byte loads: a half wave per group.
__global__ __launch_bounds__(256) void k_batch_quant(uint16_t *__restrict__ xb,
                                                     int *__restrict__ off_bf16,
                                                     int *__restrict__ zero,
                                                     const float *__restrict__ x, int T, int H) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *zero = 0;
  // a wave: 256 columns of one token (two groups, 32 lanes x 4 columns each)
  const size_t w = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) / 64;
  const int lane = threadIdx.x % 64;
  const size_t per = (size_t)H / 256;  // H % 128 == 0; an odd half group is handled below
  const size_t t = w / (per + (H % 256 ? 1 : 0)), c0 = (w % (per + (H % 256 ? 1 : 0))) * 256;
  if (t >= (size_t)T) return;
  const int c = (int)c0 + 4 * lane;
  const bool live = c < H;  // false only for the upper half of a trailing 128-group
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) v = *reinterpret_cast<const float4 *>(x + t * H + c);
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));  // within 32 lanes
  const float scale = act_scale(m);
  const float inv = 1.0f / scale;
  // dequantised grid value qx * scale: <= 4 significant bits, exact in BF16
  const uint32_t h0 = f2u(quant_e4m3(v.x, inv) * scale) >> 16;
  const uint32_t h1 = f2u(quant_e4m3(v.y, inv) * scale) >> 16;
  const uint32_t h2 = f2u(quant_e4m3(v.z, inv) * scale) >> 16;
  const uint32_t h3 = f2u(quant_e4m3(v.w, inv) * scale) >> 16;
  if (live) *reinterpret_cast<uint2 *>(xb + t * H + c) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
  const bool exact = bf16_round(v.x) == v.x && bf16_round(v.y) == v.y &&
                     bf16_round(v.z) == v.z && bf16_round(v.w) == v.w;
  const bool any_off = __any(!exact);
  if (lane == 0) off_bf16[w] = any_off ? 1 : 0;  // w = t * pieces + c0 / 256
}

// ---------------------------------------------------------- router ------
// Approximate logits and sum|g*x| with BF16 MFMA. Tile: 64 tokens x 64
// experts; wave w takes experts e0+16w..+15 against all 64 tokens. K runs in
// steps of 128: x (truncated to BF16: exact for BF16-valued inputs) is staged
// into a double-buffered LDS tile, one barrier per step; each thread's x and
// gate operands are loaded two steps ahead into a register ring of
// range-checked loads (rows past T or E read zeros).
struct RlRegs {
  uint4 x[8];  // 4 columns (fp32) of tokens 16 w + 2 i + l / 32, i = 0..7
  uint4 g[4];  // this lane's gate operands of the step's 4 MFMA k-steps
};

__device__ __forceinline__ void rl_load(RlRegs &R, BufRsrc rx, uint32_t xo, uint32_t xstep,
                                        BufRsrc rg, uint32_t go, int k0) {
#pragma unroll
  for (int i = 0; i < 8; ++i) R.x[i] = buf_load16(rx, xo + i * xstep + 4u * (uint32_t)k0);
#pragma unroll
  for (int j = 0; j < 4; ++j) R.g[j] = buf_load16(rg, go + 2u * (uint32_t)(k0 + 32 * j));
  __builtin_amdgcn_sched_barrier(0);  // issue here, not next to the first use
}

__device__ __forceinline__ void rl_store(const RlRegs &R, uint16_t *xs, int wv, int l) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint4 u = R.x[i];
    *reinterpret_cast<uint2 *>(xs + (16 * wv + 2 * i + l / 32) * 136 + 4 * (l % 32)) =
        make_uint2((u.x >> 16) | (u.y & 0xFFFF0000u), (u.z >> 16) | (u.w & 0xFFFF0000u));
  }
}

__device__ __forceinline__ void rl_mfma(v4f (&acc)[4], v4f (&aab)[4], const RlRegs &R,
                                        const uint16_t *xs, int l) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 a = R.g[j];
    const uint4 aa = make_uint4(a.x & 0x7FFF7FFFu, a.y & 0x7FFF7FFFu, a.z & 0x7FFF7FFFu,
                                a.w & 0x7FFF7FFFu);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const uint4 b =
          *reinterpret_cast<const uint4 *>(xs + (16 * f + l % 16) * 136 + 32 * j + 8 * (l / 16));
      const uint4 bb = make_uint4(b.x & 0x7FFF7FFFu, b.y & 0x7FFF7FFFu, b.z & 0x7FFF7FFFu,
                                  b.w & 0x7FFF7FFFu);
      acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), acc[f], 0, 0, 0);
      aab[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aa),
                                                       __builtin_bit_cast(bf16x8, bb), aab[f], 0, 0, 0);
    }
  }
}

template <int NS>  // H / 128 when known at compile time (fully unrolled K), else 0
__global__ __launch_bounds__(256) void k_router_logits_mfma(float *__restrict__ z,
                                                            float *__restrict__ zabs,
                                                            const float *__restrict__ x,
                                                            const uint16_t *__restrict__ G,
                                                            int T, int H, int E) {
  __shared__ __align__(16) uint16_t xs[2][64 * 136];  // [buf][token][128 + 8 pad] bf16
  const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
  const int tid = threadIdx.x, l = tid % 64;
  const int wv = __builtin_amdgcn_readfirstlane(tid / 64);
  v4f acc[4], aab[4];
  for (int f = 0; f < 4; ++f) {
    acc[f] = (v4f){0.f, 0.f, 0.f, 0.f};
    aab[f] = (v4f){0.f, 0.f, 0.f, 0.f};
  }
  // staging: wave w brings tokens 16 w .. + 15, two 512-byte rows per load
  // (rows past T lie beyond the range and read zeros)
  const BufRsrc rx = buf_rsrc(x + (size_t)t0 * H, 4u * (uint32_t)(min(T - t0, 64) * H));
  const uint32_t xo = 4u * (uint32_t)((16 * wv + l / 32) * H + 4 * (l % 32)), xstep = 8u * H;
  // one range per wave (a per-lane range would serialise the loads); expert
  // rows past E lie beyond it and read zeros
  const int we = e0 + 16 * wv;
  const uint32_t grange = __builtin_amdgcn_readfirstlane(2u * (uint32_t)(max(min(E - we, 16), 0) * H));
  const BufRsrc rg = buf_rsrc(G + (size_t)min(we, E - 1) * H, grange);
  const uint32_t go = 2u * (uint32_t)((l % 16) * H + 8 * (l / 16));
  RlRegs R[3];
  rl_load(R[0], rx, xo, xstep, rg, go, 0);
  rl_load(R[1], rx, xo, xstep, rg, go, 128);
  rl_store(R[0], xs[0], wv, l);
  __syncthreads();
  // step s computes from xs[s & 1] with the gate operands of ring slot s % 3,
  // stores step s + 1 into the other buffer and loads step s + 2 (loads past
  // the row end are never used)
  if constexpr (NS > 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s + 2 < NS) rl_load(R[(s + 2) % 3], rx, xo, xstep, rg, go, 128 * (s + 2));
      rl_mfma(acc, aab, R[s % 3], xs[s & 1], l);
      if (s + 1 < NS) {
        rl_store(R[(s + 1) % 3], xs[(s + 1) & 1], wv, l);
        __syncthreads();
      }
    }
  } else {
    // unrolled by three so that the ring slots are compile-time
    const int ns = H / 128;  // H % 128 == 0
    for (int s = 0; s < ns; s += 3) {
      rl_load(R[2], rx, xo, xstep, rg, go, 128 * (s + 2));
      rl_mfma(acc, aab, R[0], xs[s & 1], l);
      if (s + 1 < ns) rl_store(R[1], xs[(s + 1) & 1], wv, l);
      __syncthreads();
      if (s + 1 >= ns) break;
      rl_load(R[0], rx, xo, xstep, rg, go, 128 * (s + 3));
      rl_mfma(acc, aab, R[1], xs[(s + 1) & 1], l);
      if (s + 2 < ns) rl_store(R[2], xs[s & 1], wv, l);
      __syncthreads();
      if (s + 2 >= ns) break;
      rl_load(R[1], rx, xo, xstep, rg, go, 128 * (s + 4));
      rl_mfma(acc, aab, R[2], xs[s & 1], l);
      if (s + 3 < ns) rl_store(R[0], xs[(s + 1) & 1], wv, l);
      __syncthreads();
    }
  }
  for (int f = 0; f < 4; ++f) {
    const int t = t0 + 16 * f + l % 16;
    if (t >= T) continue;
    for (int v = 0; v < 4; ++v) {
      const int e = e0 + 16 * wv + 4 * (l / 16) + v;
      if (e < E) {
        z[(size_t)t * E + e] = acc[f][v];
        zabs[(size_t)t * E + e] = aab[f][v];
      }
    }
  }
}

// Wave argmax with the reference's tie rule (largest value, lowest index).
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (ov > v || (ov == v && oi >= 0 && (i < 0 || oi < i))) {
      v = ov;
      i = oi;
    }
  }
}

__device__ __forceinline__ float gamma_n2(int n) {
  const double nu = (double)n * 0x1p-24;
  return (float)(nu / (1.0 - nu));
}

// One wave per token: approximate choices, the k-th best, and every expert
// within the rigorous error margin of it -> candidate list (ascending id).
// z / zabs: the router logits and sum|g*x| [T][E]; off_bf16: k_batch_quant's
// flags, np per token.
template <int PER>  // experts per lane: E <= 64 PER
__global__ __launch_bounds__(256) void k_router_cand(int *__restrict__ cand,
                                                     int *__restrict__ ncand,
                                                     const float *__restrict__ z,
                                                     const float *__restrict__ zabs,
                                                     const int *__restrict__ off_bf16, int np,
                                                     const float *__restrict__ bias,
                                                     const int64_t *__restrict__ tid2eid,
                                                     const int *__restrict__ token_ids, int T,
                                                     int H, int E, int K) {
  const int t = blockIdx.x * 4 + threadIdx.x / 64, l = threadIdx.x % 64;
  if (t >= T) return;
  int *ct = cand + (size_t)t * E;
  if (tid2eid) {
    if (l < K) ct[l] = (int)tid2eid[(size_t)token_ids[t] * K + l];
    if (l == 0) ncand[t] = K;
    return;
  }
  // every lane's logits loaded at once (indices clamped into the row, no
  // branch), then masked past E
  float ch[PER], zv[PER], av[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const size_t i = (size_t)t * E + min(l + 64 * j, E - 1);
    zv[j] = z[i];
    av[j] = zabs[i];
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = l + 64 * j;
    ch[j] = -__builtin_inff();
    if (e < E) {
      const float c = sqrt_softplus(zv[j]) + (bias ? bias[e] : 0.0f);
      ch[j] = c == c ? c : -__builtin_inff();  // NaN is never selected
      amax = fmaxf(amax, av[j]);
    }
  }
  amax = wave_max(amax) * 1.001f;
  // is x of this token BF16-valued (the MFMA logits used its BF16 truncation)?
  bool off = false;
  for (int j = l; j < np; j += 64) off |= off_bf16[(size_t)t * np + j] != 0;
  // any-order summation bound, twice (approximate and sequential), plus the
  // BF16 conversion of a non-BF16 input; |d score/dz| <= 1/2; score slack
  float bound_z = 2.0f * gamma_n2(H) * amax;
  if (__any(off)) bound_z += 0x1p-8f * amax;
  const float delta = 2.0f * (0.5f * bound_z + 1e-5f);
  unsigned long long used = 0ull;  // bit j: expert l+64j taken
  float kth = -__builtin_inff();
  for (int k = 0; k < K; ++k) {
    // the k-th largest choice: DPP wave maximum, then the lowest index
    // holding it is taken (no LDS round trips)
    float m = -__builtin_inff();
    int mj = -1;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (!((used >> j) & 1ull) && ch[j] > m) {
        m = ch[j];
        mj = j;
      }
    const float wm = wave_max_dpp(m);
    kth = wm;
    const int bi = wave_min_dpp(mj >= 0 && m == wm ? l + 64 * mj : 0x7fffffff);
    if (bi != 0x7fffffff && (bi % 64) == l) used |= 1ull << (bi / 64);
  }
  const float thr = cand_threshold(kth, delta);
  // compaction in ascending id: pass j holds ids 64j .. 64j + 63 in lane
  // order, and each pass appends after the previous one
  int base = 0;
  for (int j = 0; j < PER; ++j) {
    const int e = l + 64 * j;
    const bool take = e < E && ch[j] >= thr;
    const unsigned long long m = __ballot(take);
    const int before = __popcll(m & ((1ull << l) - 1ull));
    if (take) ct[base + before] = e;
    base += __popcll(m);
  }
  if (l == 0) ncand[t] = base;
}

// Exclusive prefix sum of n[0..T) into off[0..T], one workgroup.
__global__ __launch_bounds__(1024) void k_scan_counts(int *__restrict__ off,
                                                      const int *__restrict__ n, int T) {
  // exclusive prefix of n[0, T) into off, off[T] = the total: 4096 counts a
  // pass, 4 consecutive per thread, a wave scan by shuffles, the 16 wave
  // totals scanned by wave 0 (two barriers a pass)
  __shared__ int wsum[16];
  __shared__ int carry;
  const int tid = threadIdx.x, lane = tid % 64, wv = tid / 64;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int b = 0; b < T; b += 4096) {
    const int i0 = b + 4 * tid;
    int v[4], run = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = i0 + j < T ? n[i0 + j] : 0;
      run += v[j];
    }
    int inc = run;  // inclusive scan of the threads' sums within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(inc, o, 64);
      if (lane >= o) inc += u;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    if (wv == 0) {
      int ws = lane < 16 ? wsum[lane] : 0;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int u = __shfl_up(ws, o, 64);
        if (lane >= o) ws += u;
      }
      if (lane < 16) wsum[lane] = ws;  // inclusive over waves
    }
    __syncthreads();
    int x = carry + (wv > 0 ? wsum[wv - 1] : 0) + inc - run;  // exclusive at i0
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (i0 + j < T) off[i0 + j] = x;
      x += v[j];
    }
    __syncthreads();  // every thread has read carry and wsum
    if (tid == 0) carry += wsum[15];
    __syncthreads();
  }
  if (tid == 0) off[T] = carry;
}

// Exact logits of every candidate: the reference's column-order fmaf chain
// (src/dsv4/dsv4_model.c:298-303), one lane per (token, candidate). A wave
// takes 64 consecutive chains (the candidates of a few consecutive tokens).
// Per 64-column step the wave's 64 gate pieces (128 bytes each) are loaded
// as whole lines, 8 lanes a row, and staged in the wave's own LDS rows, from
// which each lane reads its row; x is loaded directly (the lanes of one
// token share its lines). Both are loaded a step ahead into registers. A
// lane per chain reading its own row straight from memory touches 64 lines
// per load instruction, and the L1 cannot hold the rows between uses.
#define RC_ROW 144          // LDS bytes per staged gate piece (128 + 16: conflict-free row reads)
#define RC_BAD 0x80000000u  // an offset past the gate matrix (reads zeros)
__global__ __launch_bounds__(256) void k_router_chains(float *__restrict__ cscore,
                                                       float *__restrict__ cchoice,
                                                       const int *__restrict__ cand,
                                                       const int *__restrict__ chain_off,
                                                       const float *__restrict__ x,
                                                       const uint16_t *__restrict__ G,
                                                       const float *__restrict__ bias, int T,
                                                       int H, int E) {
  __shared__ __align__(16) uint8_t gs[4][64 * RC_ROW];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), l = threadIdx.x % 64;
  const int total = chain_off[T];
  const BufRsrc rg = buf_rsrc(G, 2u * (uint32_t)E * (uint32_t)H);
  uint8_t *buf = gs[wv];
  const int nst = H / 64;  // H % 128 == 0
  for (int g0 = (blockIdx.x * 4 + wv) * 64; g0 < total; g0 += gridDim.x * 256) {
    const int g = g0 + l;
    int t = 0, c = 0, e = -1;
    if (g < total) {
      int lo = 0, hi = T;  // chain_off[lo] <= g < chain_off[lo+1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (chain_off[mid] <= g) lo = mid;
        else hi = mid;
      }
      t = lo;
      c = g - chain_off[t];
      e = cand[(size_t)t * E + c];
      if (e < 0 || e >= E) e = -1;
    }
    // staging: load k brings piece l % 8 of chain 8 k + l / 8's row
    uint32_t srow[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int ek = __shfl(e, 8 * k + l / 8, 64);
      srow[k] = ek >= 0 ? 2u * (uint32_t)ek * (uint32_t)H + 16u * (l % 8) : RC_BAD;
    }
    auto goff = [&](int k, int st) { return srow[k] == RC_BAD ? RC_BAD : srow[k] + 128u * st; };
    const float *xr = x + (size_t)t * H;
    uint4 gv[8];
    float4 xv[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) gv[k] = buf_load16(rg, goff(k, 0));
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = *reinterpret_cast<const float4 *>(xr + 4 * i);
    float acc = 0.0f;
    for (int st = 0; st < nst; ++st) {
      // the wave's LDS operations run in order: these writes follow the
      // previous step's reads and precede this step's
#pragma unroll
      for (int k = 0; k < 8; ++k)
        *reinterpret_cast<uint4 *>(buf + (8 * k + l / 8) * RC_ROW + 16 * (l % 8)) = gv[k];
      float4 xc[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xc[i] = xv[i];
      if (st + 1 < nst) {
#pragma unroll
        for (int k = 0; k < 8; ++k) gv[k] = buf_load16(rg, goff(k, st + 1));
#pragma unroll
        for (int i = 0; i < 16; ++i)
          xv[i] = *reinterpret_cast<const float4 *>(xr + 64 * (st + 1) + 4 * i);
      }
      const uint8_t *mine = buf + l * RC_ROW;
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const uint4 w = *reinterpret_cast<const uint4 *>(mine + 16 * cc);
        const float4 xa = xc[2 * cc], xb = xc[2 * cc + 1];
        acc = fmaf(u2f(w.x << 16), xa.x, acc);
        acc = fmaf(u2f(w.x & 0xFFFF0000u), xa.y, acc);
        acc = fmaf(u2f(w.y << 16), xa.z, acc);
        acc = fmaf(u2f(w.y & 0xFFFF0000u), xa.w, acc);
        acc = fmaf(u2f(w.z << 16), xb.x, acc);
        acc = fmaf(u2f(w.z & 0xFFFF0000u), xb.y, acc);
        acc = fmaf(u2f(w.w << 16), xb.z, acc);
        acc = fmaf(u2f(w.w & 0xFFFF0000u), xb.w, acc);
      }
    }
    if (g < total) {
      float sc = 0.0f, ch = -__builtin_inff();
      if (e >= 0) {
        sc = sqrt_softplus(acc);
        ch = sc + (bias ? bias[e] : 0.0f);
      }
      cscore[(size_t)t * E + c] = sc;
      cchoice[(size_t)t * E + c] = ch;
    }
  }
}


// k_router_chains with x staged in LDS: a wave's 64 consecutive chains
// belong to at most 63 / K + 2 tokens (every token has at least K
// candidates), at most RCX_TOK for K >= 5, so per 64-column step the wave
// stages those tokens' x slices (16-byte pieces, 4 per lane) beside its
// gate pieces in its own LDS rows, and registers carry both RCX_DEPTH steps
// ahead (a one-step read-ahead left each step waiting a memory round trip;
// the x slice per lane alone took 64 VGPRs a step). Loads of steps past the
// row are range-checked and never used; no load sits under a branch. Same
// chains, same column order, same outputs.
#define RCX_TOK 16
#define RCX_DEPTH 4
#define RCX_XROW (64 * 4 + 16)  // LDS bytes per staged x slice
__global__ __launch_bounds__(256) void k_router_chains_x(float *__restrict__ cscore,
                                                         float *__restrict__ cchoice,
                                                         const int *__restrict__ cand,
                                                         const int *__restrict__ chain_off,
                                                         const float *__restrict__ x,
                                                         const uint16_t *__restrict__ G,
                                                         const float *__restrict__ bias, int T,
                                                         int H, int E) {
  __shared__ __align__(16) uint8_t gs[4][64 * RC_ROW];
  __shared__ __align__(16) uint8_t xsh[4][RCX_TOK * RCX_XROW];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), l = threadIdx.x % 64;
  const int total = chain_off[T];
  const BufRsrc rg = buf_rsrc(G, 2u * (uint32_t)E * (uint32_t)H);
  uint8_t *gbuf = gs[wv], *xbuf = xsh[wv];
  const int nst = H / 64;  // H % 128 == 0
  for (int g0 = (blockIdx.x * 4 + wv) * 64; g0 < total; g0 += gridDim.x * 256) {
    const int g = g0 + l;
    int t = 0, c = 0, e = -1;
    if (g < total) {
      int lo = 0, hi = T;  // chain_off[lo] <= g < chain_off[lo+1]
      while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (chain_off[mid] <= g) lo = mid;
        else hi = mid;
      }
      t = lo;
      c = g - chain_off[t];
      e = cand[(size_t)t * E + c];
      if (e < 0 || e >= E) e = -1;
    }
    const int tf = __builtin_amdgcn_readfirstlane(t);  // lane 0's chain is live
    const int tt = min(max(t - tf, 0), RCX_TOK - 1);
    uint32_t srow[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int ek = __shfl(e, 8 * k + l / 8, 64);
      srow[k] = ek >= 0 ? 2u * (uint32_t)ek * (uint32_t)H + 16u * (l % 8) : RC_BAD;
    }
    // x of tokens tf .. tf + RCX_TOK - 1 (rows past T read zeros); piece
    // p = l + 64 i: token p / 16, columns 4 (p % 16) of the step
    const BufRsrc rx = buf_rsrc(x + (size_t)tf * H, 4u * (uint32_t)min(T - tf, RCX_TOK) * (uint32_t)H);
    auto gload = [&](uint4 (&gv)[8], int st) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        gv[k] = buf_load16(rg, srow[k] == RC_BAD ? RC_BAD : srow[k] + 128u * st);
    };
    auto xload = [&](uint4 (&xq)[4], int st) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = l + 64 * i;
        xq[i] = buf_load16(rx, 4u * ((uint32_t)(p / 16) * (uint32_t)H + 64u * st + 4u * (p % 16)));
      }
    };
    uint4 gv[RCX_DEPTH][8], xq[RCX_DEPTH][4];
#pragma unroll
    for (int d = 0; d < RCX_DEPTH; ++d) {
      gload(gv[d], d);
      xload(xq[d], d);
    }
    float acc = 0.0f;
    int s0 = 0;
    do {
#pragma unroll
      for (int d = 0; d < RCX_DEPTH; ++d) {
        const int st = s0 + d;
        // the wave's LDS operations run in order: these writes follow the
        // previous step's reads and precede this step's
#pragma unroll
        for (int k = 0; k < 8; ++k)
          *reinterpret_cast<uint4 *>(gbuf + (8 * k + l / 8) * RC_ROW + 16 * (l % 8)) = gv[d][k];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = l + 64 * i;
          *reinterpret_cast<uint4 *>(xbuf + (p / 16) * RCX_XROW + 16 * (p % 16)) = xq[d][i];
        }
        gload(gv[d], st + RCX_DEPTH);
        xload(xq[d], st + RCX_DEPTH);
        if (st < nst) {
          const uint8_t *mine = gbuf + l * RC_ROW;
          const float4 *xr = reinterpret_cast<const float4 *>(xbuf + tt * RCX_XROW);
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {
            const uint4 w = *reinterpret_cast<const uint4 *>(mine + 16 * cc);
            const float4 xa = xr[2 * cc], xb = xr[2 * cc + 1];
            acc = fmaf(u2f(w.x << 16), xa.x, acc);
            acc = fmaf(u2f(w.x & 0xFFFF0000u), xa.y, acc);
            acc = fmaf(u2f(w.y << 16), xa.z, acc);
            acc = fmaf(u2f(w.y & 0xFFFF0000u), xa.w, acc);
            acc = fmaf(u2f(w.z << 16), xb.x, acc);
            acc = fmaf(u2f(w.z & 0xFFFF0000u), xb.y, acc);
            acc = fmaf(u2f(w.w << 16), xb.z, acc);
            acc = fmaf(u2f(w.w & 0xFFFF0000u), xb.w, acc);
          }
        }
      }
      s0 += RCX_DEPTH;
    } while (s0 < nst);
    if (g < total) {
      float sc = 0.0f, ch = -__builtin_inff();
      if (e >= 0) {
        sc = sqrt_softplus(acc);
        ch = sc + (bias ? bias[e] : 0.0f);
      }
      cscore[(size_t)t * E + c] = sc;
      cchoice[(size_t)t * E + c] = ch;
    }
  }
}

// The routes of one token (one wave; lane k carries route k in selection
// order): the reference selection (src/dsv4/dsv4_model.c:6866-6906) over nc
// scored choices cc[i] of experts ct[i] (ct null: expert i, all of them),
// strict '>' in ascending position so the lowest id wins a tie; weights from
// the unbiased scores cs[i]; then an exchange sort by id. Hash layers take
// the token's tid2eid experts in table order (hash_e: lane k's expert, -1
// past K) with cs indexed by route (ct given) or by expert (ct null; an
// expert outside [0, E) scores 0). PER: choices per lane (nc <= 64 PER).
template <int PER>
__device__ __forceinline__ void router_finalize_wave(int l, int *__restrict__ idx,
                                                     float *__restrict__ wt,
                                                     const int *__restrict__ ct, int nc,
                                                     const float *__restrict__ cs,
                                                     const float *__restrict__ cc, bool hash,
                                                     int hash_e, int E, int K,
                                                     float route_scale) {
  int my_e = -1;
  float my_sc = 0.0f;
  if (hash) {
    if (l < K) {
      my_e = hash_e;
      my_sc = ct ? cs[l] : (my_e >= 0 && my_e < E ? cs[my_e] : 0.0f);
    }
  } else {
    // choices, scores and ids all loaded up front (a score or id fetched
    // per route would be a dependent memory round trip per route)
    float v[PER], sv[PER];
    int ev[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = l + 64 * j;
      const float c = i < nc ? cc[i] : -__builtin_inff();
      v[j] = c == c ? c : -__builtin_inff();  // NaN is never selected
      sv[j] = i < nc ? cs[i] : 0.0f;
      ev[j] = ct && i < nc ? ct[i] : i;
    }
    for (int k = 0; k < K; ++k) {
      // the largest choice, the lowest index among equals (the reference's
      // strict '>' in ascending id): DPP reductions, no LDS round trips
      float m = -__builtin_inff();
      int mj = -1;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (v[j] > m) {
          m = v[j];
          mj = j;
        }
      const float wm = wave_max_dpp(m);
      if (!(wm > -__builtin_inff())) continue;  // nothing left: route k empty
      const int bi = wave_min_dpp(mj >= 0 && m == wm ? l + 64 * mj : 0x7fffffff);
      // bi is wave-uniform: its slot j, then the value from its lane
      float bs = 0.0f;
      int be = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (j == bi / 64) {
          bs = sv[j];
          be = ev[j];
        }
      bs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), bi % 64));
      be = __builtin_amdgcn_readlane(be, bi % 64);
      if (bi % 64 == l) {
#pragma unroll
        for (int j = 0; j < PER; ++j)
          if (j == bi / 64) v[j] = -__builtin_inff();  // taken
      }
      if (l == k) {
        my_e = be;
        my_sc = bs;
      }
    }
  }
  // weights: the unbiased scores summed in selection order, then the routes
  // sorted by id (equal ids carry equal weights)
  float sum = 0.0f;
  for (int k = 0; k < K; ++k)
    sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sc), k));
  const float rs = sum > 0.0f ? route_scale / sum : 0.0f;
  const float my_w = sum > 0.0f ? my_sc * rs : 0.0f;
  int rank = 0;
  for (int k = 0; k < K; ++k) {
    const int ek = __builtin_amdgcn_readlane(my_e, k);
    rank += (ek < my_e || (ek == my_e && k < l)) ? 1 : 0;
  }
  if (l < K) {
    idx[rank] = my_e;
    wt[rank] = my_w;
  }
}

// Candidate form (many tokens): the chains of k_router_chains.
__global__ __launch_bounds__(256) void k_router_finalize(
    int *__restrict__ idx, float *__restrict__ wt, const int *__restrict__ cand,
    const int *__restrict__ ncand, const float *__restrict__ cscore,
    const float *__restrict__ cchoice, int hash, int T, int E, int K, float route_scale) {
  const int t = blockIdx.x * 4 + threadIdx.x / 64, l = threadIdx.x % 64;
  if (t >= T) return;
  const size_t r = (size_t)t * E;
  router_finalize_wave<16>(l, idx + (size_t)t * K, wt + (size_t)t * K, cand + r, ncand[t],
                              cscore + r, cchoice + r, hash != 0, l < K ? cand[r + l] : -1, E,
                              K, route_scale);
}

// ---- few tokens (T <= 256): every score exact, no candidates.
// The router logit of (token t, expert e) is the reference's column-order
// fmaf chain over H (dsv4_gemv_bf16, src/dsv4/dsv4_model.c:298-303, called
// at src/dsv4/dsv4_model.c:6864-6867). Here every lane runs one whole chain:
// a one-wave workgroup takes 8 tokens x 8 experts, lane l the token
// t0 + l % 8 and the expert e0 + l / 8. The columns stream in chunks of 128
// through a double-buffered LDS tile (x fp32, the gate rows widened to fp32;
// rows padded by 16 bytes so that the 8 rows a read touches sit in distinct
// banks), each lane's share of a chunk (four 16-byte x pieces, two of the
// gate) loaded RX_DEPTH chunks ahead into a register ring, and the lane
// chains from LDS at the fma latency (chain_cols_deep: with every lane reading,
// the LDS is most of a clock per chain step busy and its reads need more
// than two batches of cover). One wave per workgroup
// because the chain reads two 16-byte LDS operands per 4 fmas per lane: the
// LDS returns 128 bytes a clock per CU, which one wave's chain nearly fills
// (64 tokens x 256 experts: 256 workgroups, one per CU). Scores go to
// cscore / cchoice [T][E]; k_router_select then picks the routes.
#define RX_TOK 8
#define RX_EXP 8
#define RX_COLS 128
#define RX_ROW (RX_COLS * 4 + 16)  // LDS bytes per staged row
#define RX_DEPTH 6
#define RX_LA 4  // LDS batches of 8 columns read ahead of the chain
#define RX_BUF ((RX_TOK + RX_EXP) * RX_ROW)

struct RxChunk {
  uint4 x[4], g[2];
};

// Chunks past the last (ch >= H / 128, the ring's run-out) are loaded too but
// never used: their offsets stay below 2^31 and either fall inside the range
// (the next row's columns) or beyond it (zeros). No select on ch: the
// compiler would branch around the load and drain the ring.
__device__ __forceinline__ void rx_load(RxChunk &R, BufRsrc rx, BufRsrc rg, int H, int ch) {
  const int l = threadIdx.x;
  const uint32_t c0 = (uint32_t)ch * RX_COLS;
  // x piece p = l + 64 k: row p / 32, columns 4 (p % 32); gate piece p = l +
  // 64 k: row p / 16, columns 8 (p % 16)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = l + 64 * k;
    R.x[k] = buf_load16(rx, 4u * ((uint32_t)(p / 32) * H + c0 + 4u * (p % 32)));
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int p = l + 64 * k;
    R.g[k] = buf_load16(rg, 2u * ((uint32_t)(p / 16) * H + c0 + 8u * (p % 16)));
  }
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void rx_store(const RxChunk &R, uint8_t *buf) {
  const int l = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = l + 64 * k;
    *reinterpret_cast<uint4 *>(buf + (p / 32) * RX_ROW + 16 * (p % 32)) = R.x[k];
  }
  uint8_t *gs = buf + RX_TOK * RX_ROW;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int p = l + 64 * k;
    const uint4 g = R.g[k];
    float4 *d = reinterpret_cast<float4 *>(gs + (p / 16) * RX_ROW + 32 * (p % 16));
    d[0] = make_float4(u2f(g.x << 16), u2f(g.x & 0xFFFF0000u), u2f(g.y << 16),
                       u2f(g.y & 0xFFFF0000u));
    d[1] = make_float4(u2f(g.z << 16), u2f(g.z & 0xFFFF0000u), u2f(g.w << 16),
                       u2f(g.w & 0xFFFF0000u));
  }
}

__global__ __launch_bounds__(64) void k_router_exact(float *__restrict__ cscore,
                                                     float *__restrict__ cchoice,
                                                     const float *__restrict__ x,
                                                     const uint16_t *__restrict__ G,
                                                     const float *__restrict__ bias, int T, int H,
                                                     int E) {
  __shared__ __align__(16) uint8_t lds[2 * RX_BUF];
  const int l = threadIdx.x;
  const int t0 = blockIdx.x * RX_TOK, e0 = blockIdx.y * RX_EXP;
  const int nch = H / RX_COLS;  // H % 128 == 0
  // rows past T or E lie beyond the ranges and read zeros
  const BufRsrc rx = buf_rsrc(x + (size_t)t0 * H, 4u * (uint32_t)(min(T - t0, RX_TOK) * H));
  const BufRsrc rg = buf_rsrc(G + (size_t)e0 * H, 2u * (uint32_t)(min(E - e0, RX_EXP) * H));
  RxChunk R[RX_DEPTH];
#pragma unroll
  for (int d = 0; d < RX_DEPTH; ++d) rx_load(R[d], rx, rg, H, d);
  const int tr = l % RX_TOK, er = RX_TOK + l / RX_TOK;  // this lane's LDS rows
  float acc = 0.0f;
  // chunk c: its ring slot c % RX_DEPTH is stored into buffer c & 1 (last
  // read by chunk c - 2) and refilled with chunk c + RX_DEPTH; then the
  // chain of chunk c. Whole groups of RX_DEPTH chunks, unrolled so the slots
  // are compile-time, in a loop with one entry and one back edge and no load
  // under a branch: the compiler's load-count waits then stay exact (each
  // slot waits only for its own loads). Chunks past the last move run-out
  // data and skip the chain.
  int c0 = 0;
  do {
#pragma unroll
    for (int d = 0; d < RX_DEPTH; ++d) {
      const int c = c0 + d;
      uint8_t *b = lds + (c & 1) * RX_BUF;
      rx_store(R[d], b);
      rx_load(R[d], rx, rg, H, c + RX_DEPTH);
      __syncthreads();
      if (c < nch)
        acc = chain_cols_deep<RX_COLS / 8, RX_LA>(
            reinterpret_cast<const float4 *>(b + er * RX_ROW),
            reinterpret_cast<const float4 *>(b + tr * RX_ROW), acc);
    }
    c0 += RX_DEPTH;
  } while (c0 < nch);
  const int t = t0 + tr, e = e0 + l / RX_TOK;
  if (t < T && e < E) {
    const float sc = sqrt_softplus(acc);
    cscore[(size_t)t * E + e] = sc;
    cchoice[(size_t)t * E + e] = sc + (bias ? bias[e] : 0.0f);
  }
}

// One wave per token over every expert's exact score (k_router_exact); hash
// layers take the token's tid2eid experts.
template <int PER>  // experts per lane: E <= 64 PER
__global__ __launch_bounds__(256) void k_router_select(
    int *__restrict__ idx, float *__restrict__ wt, const float *__restrict__ cscore,
    const float *__restrict__ cchoice, const int64_t *__restrict__ tid2eid,
    const int *__restrict__ token_ids, int T, int E, int K, float route_scale) {
  const int t = blockIdx.x * 4 + threadIdx.x / 64, l = threadIdx.x % 64;
  if (t >= T) return;
  const size_t r = (size_t)t * E;
  const int he = tid2eid && l < K ? (int)tid2eid[(size_t)token_ids[t] * K + l] : -1;
  router_finalize_wave<PER>(l, idx + (size_t)t * K, wt + (size_t)t * K, nullptr, E, cscore + r,
                            cchoice + r, tid2eid != nullptr, he, E, K, route_scale);
}

// -------------------------------------------------------- dispatch -------
// Dispatch in three passes over the T K routes, in blocks of 256 routes:
// per-block expert histograms (LDS atomics: counts do not depend on order),
// prefixes (each block's base within each expert, then expert and tile
// offsets), and the placement: block b writes its routes of expert e
// from its base, in route order (a route's rank among the block's earlier
// routes of the same expert). Positions of an expert are thus in ascending
// (token, route) order, as one sequential pass would give them.
#define DP_ROUTES 256
__global__ __launch_bounds__(256) void k_dispatch_hist(int *__restrict__ bh,
                                                       const int *__restrict__ idx, int TK,
                                                       int E) {
  __shared__ int hist[1024];  // E <= 1024
  const int b = blockIdx.x, nb = gridDim.x;
  for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
  __syncthreads();
  const int i = b * DP_ROUTES + threadIdx.x;
  const int e = i < TK ? idx[i] : -1;
  if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) bh[(size_t)e * nb + b] = hist[e];
}

// block e: bh[e][b] -> exclusive prefix over the route blocks b; the total
// into cnt[e]
__global__ __launch_bounds__(256) void k_dispatch_scan_blocks(int *__restrict__ bh,
                                                              int *__restrict__ cnt, int nb) {
  __shared__ int part[256];
  int *row = bh + (size_t)blockIdx.x * nb;
  int carry = 0;
  for (int b0 = 0; b0 < nb; b0 += 256) {
    const int b = b0 + threadIdx.x;
    const int v = b < nb ? row[b] : 0;
    part[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const int a = threadIdx.x >= (unsigned)o ? part[threadIdx.x - o] : 0;
      __syncthreads();
      part[threadIdx.x] += a;
      __syncthreads();
    }
    if (b < nb) row[b] = carry + part[threadIdx.x] - v;
    carry += part[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) cnt[blockIdx.x] = carry;
}

// one block of 1024 threads: position and tile offsets over experts (the
// shared expert is group E)
__global__ __launch_bounds__(1024) void k_dispatch_scan(const int *__restrict__ cnt,
                                                        int *__restrict__ pos_off,
                                                        int *__restrict__ tile_off, int T, int E) {
  __shared__ int sp[1024], st[1024];
  const int e = threadIdx.x;
  const int tot = e < E ? cnt[e] : 0;
  sp[e] = tot;
  st[e] = (tot + GT_TN - 1) / GT_TN;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {  // inclusive scans
    const int a = e >= o ? sp[e - o] : 0, c = e >= o ? st[e - o] : 0;
    __syncthreads();
    sp[e] += a;
    st[e] += c;
    __syncthreads();
  }
  if (e < E) {
    pos_off[e] = sp[e] - tot;
    tile_off[e] = st[e] - (tot + GT_TN - 1) / GT_TN;
  }
  if (e == 0) {
    const int P = sp[E - 1], TT = st[E - 1];
    pos_off[E] = P;
    tile_off[E] = TT;
    pos_off[E + 1] = P + T;
    tile_off[E + 1] = TT + (T + GT_TN - 1) / GT_TN;
  }
}

__global__ __launch_bounds__(256) void k_dispatch_fill(
    int *__restrict__ pos_token, int *__restrict__ pos_route, float *__restrict__ pos_wt,
    const int *__restrict__ bh, const int *__restrict__ pos_off, const int *__restrict__ idx,
    const float *__restrict__ wt, int T, int K, int E) {
  __shared__ int es[DP_ROUTES];
  const int b = blockIdx.x, nb = gridDim.x, TK = T * K;
  const int i = b * DP_ROUTES + threadIdx.x;
  int e = i < TK ? idx[i] : -1;
  if (e >= E) e = -1;
  es[threadIdx.x] = e;
  __syncthreads();
  if (e >= 0) {
    int rank = 0;
    for (int k = 0; k < (int)threadIdx.x; ++k) rank += es[k] == e;
    const int p = pos_off[e] + bh[(size_t)e * nb + b] + rank;
    pos_token[p] = i / K;
    pos_route[p] = i % K;
    pos_wt[p] = wt[i];
  }
  // the shared expert's positions: every token, route slot K, weight 1
  const int p0 = pos_off[E];
  for (int t = b * DP_ROUTES + threadIdx.x; t < T; t += nb * DP_ROUTES) {
    pos_token[p0 + t] = t;
    pos_route[p0 + t] = K;
    pos_wt[p0 + t] = 1.0f;
  }
}

// The same placement in one workgroup of 1024 threads for at most 1024
// routes: expert counts, position and tile offsets, and each route's rank
// among the earlier routes of its expert counted directly.
__global__ __launch_bounds__(1024) void k_dispatch_small(
    int *__restrict__ pos_token, int *__restrict__ pos_route, float *__restrict__ pos_wt,
    int *__restrict__ pos_off, int *__restrict__ tile_off, const int *__restrict__ idx,
    const float *__restrict__ wt, int T, int K, int E) {
  __shared__ __align__(16) int es[1024];
  __shared__ int sp[1024], st[1024];
  const int i = threadIdx.x, TK = T * K;
  int e = i < TK ? idx[i] : -1;
  if (e >= E) e = -1;
  es[i] = e;
  sp[i] = 0;
  __syncthreads();
  if (e >= 0) atomicAdd(&sp[e], 1);
  __syncthreads();
  const int tot = i < E ? sp[i] : 0;
  st[i] = (tot + GT_TN - 1) / GT_TN;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {  // inclusive scans over experts
    const int a = i >= o ? sp[i - o] : 0, c = i >= o ? st[i - o] : 0;
    __syncthreads();
    sp[i] += a;
    st[i] += c;
    __syncthreads();
  }
  if (i < E) {
    pos_off[i] = sp[i] - tot;
    tile_off[i] = st[i] - (tot + GT_TN - 1) / GT_TN;
  }
  const int P = sp[E - 1], TT = st[E - 1];
  if (i == 0) {
    pos_off[E] = P;
    tile_off[E] = TT;
    pos_off[E + 1] = P + T;
    tile_off[E + 1] = TT + (T + GT_TN - 1) / GT_TN;
  }
  if (e >= 0) {
    int rank = 0;  // earlier routes of expert e, four per LDS read
    const int4 *e4 = reinterpret_cast<const int4 *>(es);
    for (int k = 0; k < i / 4; ++k) {
      const int4 v = e4[k];
      rank += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
    }
    for (int k = i & ~3; k < i; ++k) rank += es[k] == e;
    const int p = (e > 0 ? sp[e - 1] : 0) + rank;  // the exclusive prefix of expert e
    pos_token[p] = i / K;
    pos_route[p] = i % K;
    pos_wt[p] = wt[i];
  }
  for (int t = i; t < T; t += 1024) {  // the shared expert: every token, slot K
    pos_token[P + t] = t;
    pos_route[P + t] = K;
    pos_wt[P + t] = 1.0f;
  }
}

// Few tokens (T K <= 1024, the exact router's scores): the routes of every
// token and their placement in one launch of ceil(T / 16) workgroups of 1024
// threads. Wave w of workgroup b selects the routes of token 16 b + w
// (router_finalize_wave), written through; each workgroup then counts itself
// done on cnt[0] (zeroed by k_batch_quant) once its stores are complete, and
// the last one places every route: route i (thread i, in (token, route)
// order) takes position pos_off[e] + (routes of expert e in earlier waves:
// per-wave histograms) + (earlier lanes of its own wave with expert e) - the
// order k_dispatch_fill gives. Expert and tile offsets and the shared
// expert's positions as there. No workgroup waits for another.
#define SD_WAVES 16
template <typename V>
__device__ __forceinline__ V ld_agent(const V *p) {
  return __hip_atomic_load(const_cast<V *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ void st_agent(V *p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int PER>  // experts per lane: E <= 64 PER
__global__ __launch_bounds__(1024) void k_select_dispatch(
    int *__restrict__ idx, float *__restrict__ wt, int *__restrict__ cnt,
    int *__restrict__ pos_token, int *__restrict__ pos_route, float *__restrict__ pos_wt,
    int *__restrict__ pos_off, int *__restrict__ tile_off, const float *__restrict__ cscore,
    const float *__restrict__ cchoice, const int64_t *__restrict__ tid2eid,
    const int *__restrict__ token_ids, int T, int E, int K, float route_scale) {
  __shared__ int es[1024];
  __shared__ float wsel[1024];
  __shared__ int hist[SD_WAVES][1024];  // E <= 1024
  __shared__ int sp[1024], st[1024];
  __shared__ int s_last;
  const int i = threadIdx.x, wv = i / 64, l = i % 64, TK = T * K;
  {
    const int t = blockIdx.x * SD_WAVES + wv;
    if (t < T) {
      const size_t r = (size_t)t * E;
      const int he = tid2eid && l < K ? (int)tid2eid[(size_t)token_ids[t] * K + l] : -1;
      router_finalize_wave<PER>(l, es + t % SD_WAVES * K, wsel + t % SD_WAVES * K, nullptr, E,
                                cscore + r, cchoice + r, tid2eid != nullptr, he, E, K,
                                route_scale);
      if (l < K) {
        st_agent(idx + (size_t)t * K + l, es[t % SD_WAVES * K + l]);
        st_agent(wt + (size_t)t * K + l, wsel[t % SD_WAVES * K + l]);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (i == 0)
    s_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (int)gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  for (int e = l; e < E; e += 64) hist[wv][e] = 0;
  int e = i < TK ? ld_agent(idx + i) : -1;
  const float we = i < TK ? ld_agent(wt + i) : 0.0f;
  if (e >= E) e = -1;  // never dispatched (its slot adds nothing in the combine)
  // earlier lanes of this wave with the same expert
  int r_in = 0;
  for (int k = 0; k < 64; ++k) {
    const int ek = __builtin_amdgcn_readlane(e, k);
    r_in += (k < l && ek == e) ? 1 : 0;
  }
  __syncthreads();
  if (e >= 0) atomicAdd(&hist[wv][e], 1);
  __syncthreads();
  int tot = 0;
  if (i < E)
    for (int w = 0; w < SD_WAVES; ++w) tot += hist[w][i];
  sp[i] = tot;
  st[i] = (tot + GT_TN - 1) / GT_TN;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {  // inclusive scans over experts
    const int a = i >= o ? sp[i - o] : 0, c = i >= o ? st[i - o] : 0;
    __syncthreads();
    sp[i] += a;
    st[i] += c;
    __syncthreads();
  }
  if (i < E) {
    pos_off[i] = sp[i] - tot;
    tile_off[i] = st[i] - (tot + GT_TN - 1) / GT_TN;
  }
  const int P = sp[E - 1], TT = st[E - 1];
  if (i == 0) {
    pos_off[E] = P;
    tile_off[E] = TT;
    pos_off[E + 1] = P + T;
    tile_off[E + 1] = TT + (T + GT_TN - 1) / GT_TN;
  }
  if (e >= 0) {
    int before = 0;  // routes of expert e in earlier waves
    for (int w = 0; w < wv; ++w) before += hist[w][e];
    const int p = (e > 0 ? sp[e - 1] : 0) + before + r_in;
    pos_token[p] = i / K;
    pos_route[p] = i % K;
    pos_wt[p] = we;
  }
  for (int t = i; t < T; t += 1024) {  // the shared expert: every token, slot K
    pos_token[P + t] = t;
    pos_route[P + t] = K;
    pos_wt[P + t] = 1.0f;
  }
}

// ---------------------------------------------------- grouped GEMMs ------
// BF16 operands over a 128-K super-window. Lane group g = l/16 owns the 32
// physical columns [32g, 32g+32) of the super-window; MFMA step q (0..3)
// feeds it columns [32g+8q, 32g+8q+8). The same permutation of K is used for
// both operands, so each step still computes exact products of matching
// columns, and every lane reads 16-64 contiguous bytes.
#define GT_BROW2 272  // LDS bytes per staged BF16 activation row (256 + 16 pad)

struct GroupedArgs {
  const uint8_t *experts;
  size_t expert_stride, scale_run;
  const uint8_t *shw[3], *shs[3];
  const int *tile_off, *pos_off, *pos_token, *pos_route;
  const float *pos_wt;
  const uint16_t *xb;  // [T][H] BF16 activations (dequantised FP8)
  uint16_t *yb;        // [P][I] BF16 intermediate (dequantised FP8)
  uint16_t *ro;        // [T][K+1][H] BF16 bits
  float *ro32;         // optional [T][K+1][H]: the same outputs before BF16 rounding
  uint32_t xb_bytes, yb_bytes;
  int H, I, E, K, T, row_tiles;
  float limit;
  int sh_base;  // the shared expert's positions: sh_base + token (yb rows)
  int sh_wgs;   // with the shared expert folded in: its workgroups, first
};

// (token tile, row tile) of workgroup b of nb. Workgroups go to the 8 XCDs
// round-robin by index and each XCD has its own L2: when the row tiles split
// evenly, XCD x takes row tiles [x RT/8, (x+1) RT/8) for every token tile,
// token tile by token tile, so a row tile's weights are read into that L2
// once and reused by every token tile, and a token tile's activations by
// the XCD's row tiles. Otherwise row tiles vary fastest.
__device__ __forceinline__ void tile_coords(int b, int nb, int rt_n, int &tt, int &rt) {
  if (rt_n % 8 == 0 && nb % 8 == 0) {
    const int per = rt_n / 8, k = b / 8;
    tt = k / per;
    rt = (b % 8) * per + k % per;
  } else {
    tt = b / rt_n;
    rt = b % rt_n;
  }
}

__device__ __forceinline__ int tile_expert(const int *tile_off, int E, int tt) {
  int lo = 0, hi = E + 1;
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (tile_off[mid] <= tt) lo = mid;
    else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ uint32_t bf2_bits(bf16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ v4f mfma_bf16(uint4 a, uint4 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void load_b_ops(uint4 (&op)[4], const uint8_t *bt, int j, int l) {
  const uint4 *p = reinterpret_cast<const uint4 *>(bt + j * GT_BROW2 + (l / 16) * 64);
#pragma unroll
  for (int q = 0; q < 4; ++q) op[q] = p[q];
}

// ---- software-pipelined K loop. Per 128-K window a wave needs, for each of
// its NM x 2 weight fragments (NM matrices, two 16-row fragments), the lane's
// 16 (FP4) or 32 (FP8) weight bytes and one scale code, and each thread
// stages 64 bytes of one activation row into LDS. Those raw operands are
// buffer-loaded GT_DEPTH windows ahead, window by window in consumption
// order (loads complete in order, so a window's wait never waits on a later
// window); the activation tile is double-buffered in LDS, one barrier per
// window. A operands are converted one MFMA step (q) at a time to keep
// registers for the ring. Windows run in chunks of GT_CHUNK, fully unrolled
// (a loop-carried prefetch would be drained at every iteration); windows
// past the end read zeros and skip their MFMAs.
#define GT_CHUNK 12
#define GT_DEPTH 3
#define GU_PD_SMALL 3  // FP4 pair slots of the gate/up loop for tiles of <= 32 positions
#define DN_PD_SMALL 3  // and of the down loop
#define GT_BT_BYTES (GT_TN * GT_BROW2)
#define GT_BAD 0x80000000u  // an offset past every range (and its +48)

template <int AFMT, int NM>
struct WinRaw {
  uint4 a0[NM][2], a1[NM][2];  // a1: the second 16 bytes of an FP8 fragment
  uint32_t code[NM][2];        // FP8 only (FP4 codes are staged in LDS per tile)
  uint4 b[4];
};

// FP4 tiles: the E8M0 codes of the tile's 128 rows of each matrix (in / 32
// bytes a row in the scale matrix) are copied once per tile into LDS with
// direct-to-LDS loads, instead of one byte per lane per window: a
// per-window byte load fetches a whole line for every row and misses the L1
// each time. LDS layout of matrix m (from m * codes_stride(in)): [window
// quad j][row][16 bytes: codes of windows 4 j .. 4 j + 3, 4 per window].
// A window's code reads (16 rows x 4 bytes, the four lanes of a row reading
// one dword) then fall in 16 distinct banks; row-major rows of 128 bytes
// put all 16 rows in two banks (8-way conflicts). Each load instruction
// moves one quad of 64 rows (the source rows are 16-byte pieces, one per
// lane). The copy is the first load of each wave, so the in-order wait on
// the tile's first window covers it, and the first window's barrier
// publishes it.
__host__ __device__ constexpr uint32_t codes_stride(int in) {
  return (uint32_t)((in / 128 + 3) / 4) * 16u * GT_TM;
}

__device__ __forceinline__ uint32_t code_offset(int row, int sw, int g) {
  return (uint32_t)(sw / 4) * 16u * GT_TM + 16u * row + 4u * (sw % 4) + g;
}

template <int NM>
__device__ __forceinline__ void stage_codes(uint8_t *cs, const BufRsrc (&S)[NM], int rt, int in) {
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), l = threadIdx.x % 64;
  const uint32_t rowb = (uint32_t)(in / 32), cst = codes_stride(in);
  const uint32_t nu = 2u * ((in / 128 + 3) / 4);  // (quad, half of the rows) pieces
#pragma unroll
  for (int m = 0; m < NM; ++m)
    for (uint32_t u = wv; u < nu; u += 4u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          S[m], (__attribute__((address_space(3))) void *)(cs + m * cst + 1024u * u), 16,
          ((uint32_t)rt * GT_TM + 64u * (u % 2) + l) * rowb + 16u * (u / 2), 0, 0, 0);
}

// W[m], S[m]: buffers of matrix m and its scales; in: K width; rbase: the
// wave's first row; brow[k]: the activation row of tile row tid / 16 + 16 k
// (-1: none), of which this thread stages the 16-byte piece tid % 16 (a
// wave's load covers 4 whole 256-byte rows: 8 cache lines); bsrc: buffer
// over the activation matrix (row stride in BF16 elements). The loads
// of a window come in four parts (matrix 0, matrix 1, two halves of the
// activation row), issued between MFMA steps so that the vector memory path
// works while the matrix cores do; every part of a window is issued before
// any part of the next (waits are in-order).
template <int AFMT, int NM>
__device__ __forceinline__ void win_load_part(WinRaw<AFMT, NM> &R, int part,
                                              const BufRsrc (&W)[NM], const BufRsrc (&S)[NM],
                                              BufRsrc bsrc, int in, int rbase, const int (&brow)[4],
                                              int sw, int nsw) {
  const int l = threadIdx.x % 64, g = l / 16;
  const bool ok = sw < nsw;
  if (part < 2) {
    const int m = part;
    if (m < NM) {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const uint32_t row = (uint32_t)(rbase + 16 * f + l % 16);
        if (AFMT == MX_FP4) {
          R.a0[m][f] = buf_load16(W[m], ok ? row * (uint32_t)(in / 2) + sw * 64u + g * 16u : GT_BAD);
        } else {
          const uint32_t o = ok ? row * (uint32_t)in + sw * 128u + g * 32u : GT_BAD;
          R.a0[m][f] = buf_load16(W[m], o);
          R.a1[m][f] = buf_load16(W[m], o + 16u);
          R.code[m][f] = __builtin_amdgcn_raw_buffer_load_b8(
              S[m], ok ? (row / 128u) * (uint32_t)(in / 128) + sw : GT_BAD, 0, 0);
        }
      }
    }
  } else {
    const int k0 = (part - 2) * 2;
#pragma unroll
    for (int k = k0; k < k0 + 2; ++k) {
      const uint32_t bo = (ok && brow[k] >= 0)
                              ? 2u * ((uint32_t)brow[k] * (uint32_t)in + sw * 128u) +
                                    16u * (uint32_t)(threadIdx.x % 16)
                              : GT_BAD;
      R.b[k] = buf_load16(bsrc, bo);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the parts in order
}

template <int AFMT, int NM>
__device__ __forceinline__ void win_load(WinRaw<AFMT, NM> &R, const BufRsrc (&W)[NM],
                                         const BufRsrc (&S)[NM], BufRsrc bsrc, int in, int rbase,
                                         const int (&brow)[4], int sw, int nsw) {
#pragma unroll
  for (int part = 0; part < 4; ++part)
    win_load_part<AFMT, NM>(R, part, W, S, bsrc, in, rbase, brow, sw, nsw);
}

// MFMA step q's A operand (8 K values) from the raw bytes: BF16 weight times
// its block scale (exact); a NaN scale zeroes the block, as the reference
// skips it (zero bytes at scale 1, selected without a branch).
template <int AFMT>
__device__ __forceinline__ uint4 win_op(uint4 r0, uint4 r1, uint32_t code, int q) {
  const bool nan = code == 255u;
  const float s = nan ? 1.0f : e8m0(code);
  uint4 o;
  if (AFMT == MX_FP4) {
    const uint32_t d = nan ? 0u : (q == 0 ? r0.x : q == 1 ? r0.y : q == 2 ? r0.z : r0.w);
    o.x = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 0));
    o.y = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 1));
    o.z = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 2));
    o.w = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, s, 3));
  } else {
    const uint32_t d0 = nan ? 0u : (q == 0 ? r0.x : q == 1 ? r0.z : q == 2 ? r1.x : r1.z);
    const uint32_t d1 = nan ? 0u : (q == 0 ? r0.y : q == 1 ? r0.w : q == 2 ? r1.y : r1.w);
    o.x = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, s, false));
    o.y = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, s, true));
    o.z = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, s, false));
    o.w = bf2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, s, true));
  }
  return o;
}

// The K loop of one tile: acc[m][f][c] += A_m rows (rbase + 16 f ..) x the
// staged activation rows of fragment c < nf. rows: the tile's activation
// rows (LDS, -1: none), published by the caller before (barrier).
template <int AFMT, int NM>
__device__ __forceinline__ void gemm_k_loop(v4f (&acc)[NM][2][4], const BufRsrc (&W)[NM],
                                            const BufRsrc (&S)[NM], BufRsrc bsrc, int in,
                                            int rbase, const int *rows, int nf, uint8_t *bt,
                                            const uint8_t *cs) {
  const int tid = threadIdx.x, l = tid % 64;
  const int nsw = in / 128;
  int brow[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) brow[k] = rows[tid / 16 + 16 * k];
  for (int c0 = 0; c0 < nsw; c0 += GT_CHUNK) {
    WinRaw<AFMT, NM> R[GT_DEPTH];
#pragma unroll
    for (int d = 0; d < GT_DEPTH; ++d)
      win_load<AFMT, NM>(R[d], W, S, bsrc, in, rbase, brow, c0 + d, nsw);
#pragma unroll
    for (int i = 0; i < GT_CHUNK; ++i) {
      const int sw = c0 + i;
      WinRaw<AFMT, NM> &Rc = R[i % GT_DEPTH];
      uint8_t *bb = bt + (sw & 1) * GT_BT_BYTES;
      {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          *reinterpret_cast<uint4 *>(bb + (tid / 16 + 16 * k) * GT_BROW2 + 16 * (tid % 16)) =
              Rc.b[k];
      }
      // this window's A bytes, kept while the ring slot is refilled
      uint4 A0[NM][2], A1[NM][2];
      uint32_t Ac[NM][2];
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          A0[m][f] = Rc.a0[m][f];
          A1[m][f] = Rc.a1[m][f];
          Ac[m][f] = AFMT == MX_FP4 ? 0u : Rc.code[m][f];
        }
      const bool pre = i + GT_DEPTH < GT_CHUNK;  // refill this ring slot, window sw + DEPTH
      __syncthreads();
      if (sw >= nsw && pre) win_load<AFMT, NM>(Rc, W, S, bsrc, in, rbase, brow, sw + GT_DEPTH, nsw);
      if (sw < nsw) {
        if (AFMT == MX_FP4) {
          // this lane's code of window sw: row rbase % 128 + 16 f + l % 16,
          // byte 4 sw + l / 16
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int f = 0; f < 2; ++f)
              Ac[m][f] = cs[m * codes_stride(in) +
                            code_offset(rbase % GT_TM + 16 * f + l % 16, sw, l / 16)];
        }
        // every fragment, whatever nf: rows past the tile are staged as
        // zeros, and branches here would serialise the LDS reads. The
        // activation operands of step q + 1 are read during step q's MFMAs.
        const uint8_t *brow_p = bb + (l % 16) * GT_BROW2 + (l / 16) * 64;
        uint4 Bq[2][4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          Bq[0][c] = *reinterpret_cast<const uint4 *>(brow_p + 16 * c * GT_BROW2);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (pre) win_load_part<AFMT, NM>(Rc, q, W, S, bsrc, in, rbase, brow, sw + GT_DEPTH, nsw);
          if (q + 1 < 4) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              Bq[(q + 1) & 1][c] =
                  *reinterpret_cast<const uint4 *>(brow_p + 16 * c * GT_BROW2 + 16 * (q + 1));
          }
          uint4 A[NM][2];
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int f = 0; f < 2; ++f) A[m][f] = win_op<AFMT>(A0[m][f], A1[m][f], Ac[m][f], q);
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
              for (int f = 0; f < 2; ++f)
                acc[m][f][c] = mfma_bf16(A[m][f], Bq[q & 1][c], acc[m][f][c]);
        }
      }
    }
  }
}

// ---- the FP4 K loop. A row's FP4 weights of two consecutive 128-K windows
// share one 128-byte cache line (64 bytes each); fetched a window apart,
// the line leaves the L1 in between and is fetched twice. So the weights are
// loaded a window pair at a time (both halves of every line back to back)
// into a two-slot pair ring, issued during the first window of the pair
// before it (distance 2-3 windows); the activation rows keep one window per
// slot, two slots, distance 2. Codes come from the tile's LDS copy. The
// windows are fully unrolled for the model's widths (H = 4096 for gate/up,
// I = 2048 for down): a loop carrying loads across its back edge is drained
// at the loop head. Other widths take the per-window loop.
template <int NM>
struct Fp4Pair {
  uint4 w[NM][2][2];  // [matrix][fragment][window of the pair]
};

// The fast loops permute K within each pair of windows (a 128-byte FP4 block
// of a row, 256 K): lane group g takes the 32 contiguous bytes [32 g, 32 g +
// 32) of the block, the first 16 as window 2 s and the rest as window
// 2 s + 1. So window w = 2 s + h holds, for lane group g, the K range
// 256 s + 64 g + 32 h + [0, 32): E8M0 block 8 s + 2 g + h (fp4k_block), and
// the activations are staged in the same order (act_load). Each of the two
// loads then touches every 32-byte sector of the row's 128-byte line; with
// window w's bytes [64 w, 64 w + 64) per load, each load reads half a line and
// the row's two halves are fetched apart (about 4.8 against 6.1 TB/s for the
// same bytes, measured with a probe of the two patterns). Windows come in
// pairs, so the window count must be even.
__device__ __forceinline__ int fp4k_block(int sw, int g) { return 8 * (sw / 2) + 2 * g + sw % 2; }

template <int NM>
__device__ __forceinline__ void fp4_pair_load(Fp4Pair<NM> &P, int m, const BufRsrc (&W)[NM],
                                              int in, int rbase, int pw, int nsw) {
  const int l = threadIdx.x % 64, g = l / 16;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const uint32_t row = (uint32_t)(rbase + 16 * f + l % 16);
    const uint32_t o = row * (uint32_t)(in / 2) + (pw / 2) * 128u + g * 32u;
    P.w[m][f][0] = buf_load16(W[m], pw < nsw ? o : GT_BAD);
    P.w[m][f][1] = buf_load16(W[m], pw + 1 < nsw ? o + 16u : GT_BAD);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// half h of this thread's activation staging loads of window sw (tile rows
// tid / 16 + 16 k, k = 2 h, 2 h + 1; 16-byte piece pc = tid % 16 of the staged
// row: K 128 sw + 8 pc, or with PERM the FP4 pair order, K 256 (sw / 2) +
// 64 (pc / 4) + 32 (sw % 2) + 8 (pc % 4))
template <bool PERM>
__device__ __forceinline__ void act_load(uint4 (&b)[4], int h, BufRsrc bsrc, int in,
                                         const int (&brow)[4], int sw, int nsw) {
  const uint32_t pc = threadIdx.x % 16;
  const uint32_t k0 = PERM ? 256u * (sw / 2) + 32u * (sw % 2) + 64u * (pc / 4) + 8u * (pc % 4)
                           : 128u * sw + 8u * pc;
#pragma unroll
  for (int k = 2 * h; k < 2 * h + 2; ++k) {
    const uint32_t bo = (sw < nsw && brow[k] >= 0)
                            ? 2u * ((uint32_t)brow[k] * (uint32_t)in + k0)
                            : GT_BAD;
    b[k] = buf_load16(bsrc, bo);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// FP8 weights: a window of a row is one whole 128-byte line (32 bytes a
// lane). Two window slots; window sw + 2 is loaded into the slot of window
// sw during its last MFMA step (the slot's last conversion is done by then),
// with the block's E8M0 code (one per 128 rows x 128 K: one byte a wave).
template <int NM>
struct Fp8Win {
  uint4 a0[NM][2], a1[NM][2];
  uint32_t code[NM];
};

template <int NM>
__device__ __forceinline__ void fp8_win_load(Fp8Win<NM> &R, const BufRsrc (&W)[NM],
                                             const BufRsrc (&S)[NM], int in, int rbase, int sw,
                                             int nsw) {
  const int l = threadIdx.x % 64, g = l / 16;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const uint32_t row = (uint32_t)(rbase + 16 * f + l % 16);
      const uint32_t o = sw < nsw ? row * (uint32_t)in + sw * 128u + g * 32u : GT_BAD;
      R.a0[m][f] = buf_load16(W[m], o);
      R.a1[m][f] = buf_load16(W[m], o + 16u);
    }
    R.code[m] = __builtin_amdgcn_raw_buffer_load_b8(
        S[m], sw < nsw ? (uint32_t)(rbase / 128) * (uint32_t)(in / 128) + sw : GT_BAD, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// NSW = in / 128 windows, fully unrolled; NF: token fragments computed (a
// tile of at most 16 NF positions skips the MFMAs and staging of the rest).
// FP4 weights come in window pairs, FP8 weights in window slots (above).
// PD: FP4 pair slots. Pair p (windows 2p, 2p + 1) is loaded during window
// 2 (p - PD + 1) into slot p % PD, and the activations of window w during
// window w - AD, AD = 2 (PD - 1), into register slot w % AD: weights and
// activations the same distance ahead, so that the in-order wait for a
// window's activations never waits on weights loaded for a later window.
// A tile of one or two token fragments does little MFMA work per window and
// needs the deeper ring to keep enough weight bytes in flight.
template <int AFMT, int NM, int NSW, int NF, int PD = 2>
__device__ __forceinline__ void gemm_k_loop_fast(v4f (&acc)[NM][2][4], const BufRsrc (&W)[NM],
                                                 const BufRsrc (&S)[NM], BufRsrc bsrc, int in,
                                                 int rbase, const int *rows, uint8_t *bt,
                                                 const uint8_t *cs) {
  constexpr bool FP4 = AFMT == MX_FP4;
  const int tid = threadIdx.x, l = tid % 64;
  int brow[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) brow[k] = k < NF ? rows[tid / 16 + 16 * k] : -1;
  // FP4: this lane's codes: row rbase % 128 + 16 f + l % 16, block
  // fp4k_block(sw, l / 16) (the LDS holds each row's blocks 16 j .. 16 j + 15
  // in 16 consecutive bytes, as code_offset lays them out)
  static_assert(!FP4 || NSW % 2 == 0, "FP4 windows come in pairs");
  auto code = [&](int m, int f, int sw) -> uint32_t {
    const int b = fp4k_block(sw, l / 16);
    return cs[m * codes_stride(in) + (uint32_t)(b / 16) * 16u * GT_TM +
              16u * (uint32_t)(rbase % GT_TM + 16 * f + l % 16) + (uint32_t)(b % 16)];
  };
  static_assert(FP4 || PD == 2, "FP8 windows use two slots");
  constexpr int AD = 2 * (PD - 1);
  Fp4Pair<NM> P[PD];
  Fp8Win<NM> R8[2];
  uint4 B[AD][4];
  if constexpr (FP4) {
#pragma unroll
    for (int p = 0; p + 1 < PD; ++p) {
#pragma unroll
      for (int m = 0; m < NM; ++m) fp4_pair_load<NM>(P[p], m, W, in, rbase, 2 * p, NSW);
      act_load<FP4>(B[2 * p], 0, bsrc, in, brow, 2 * p, NSW);
      act_load<FP4>(B[2 * p], 1, bsrc, in, brow, 2 * p, NSW);
      act_load<FP4>(B[2 * p + 1], 0, bsrc, in, brow, 2 * p + 1, NSW);
      act_load<FP4>(B[2 * p + 1], 1, bsrc, in, brow, 2 * p + 1, NSW);
    }
  } else {
    fp8_win_load<NM>(R8[0], W, S, in, rbase, 0, NSW);
    fp8_win_load<NM>(R8[1], W, S, in, rbase, 1, NSW);
    act_load<FP4>(B[0], 0, bsrc, in, brow, 0, NSW);
    act_load<FP4>(B[0], 1, bsrc, in, brow, 0, NSW);
    act_load<FP4>(B[1], 0, bsrc, in, brow, 1, NSW);
    act_load<FP4>(B[1], 1, bsrc, in, brow, 1, NSW);
  }
  // the A operand of (window w, step q): BF16 weights x block scale
  auto a_op = [&](int w, int m, int f, int q, uint32_t c) -> uint4 {
    if constexpr (FP4) {
      const uint4 r = P[(w / 2) % PD].w[m][f][w & 1];
      return win_op<MX_FP4>(r, r, c, q);
    } else {
      return win_op<MX_FP8>(R8[w & 1].a0[m][f], R8[w & 1].a1[m][f], R8[w & 1].code[m], q);
    }
  };
  // A operands are converted one MFMA step ahead (step q + 1, or the next
  // window's step 0, during step q's MFMAs), so that the conversions can
  // issue between the MFMAs instead of in front of them
  uint32_t Ac[NM][2] = {}, Acn[NM][2] = {};
  uint4 A[NM][2];
  if constexpr (!FP4) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < 2; ++f) A[m][f] = a_op(0, m, f, 0, 0u);
  }
#pragma unroll
  for (int sw = 0; sw < NSW; ++sw) {
    uint8_t *bb = bt + (sw & 1) * GT_BT_BYTES;
#pragma unroll
    for (int k = 0; k < NF; ++k)
      *reinterpret_cast<uint4 *>(bb + (tid / 16 + 16 * k) * GT_BROW2 + 16 * (tid % 16)) =
          B[sw % AD][k];
    __syncthreads();
    if (FP4 && sw == 0) {
      // the tile's codes were staged into LDS by every wave's direct-to-LDS
      // loads (stage_codes), and a wave reads rows another wave staged: only
      // after this barrier, which every wave reaches with its own staging
      // complete (the staging loads precede the activation loads whose
      // values it just stored, and loads complete in order), are they all in
      // place
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          Ac[m][f] = code(m, f, 0);
          A[m][f] = a_op(0, m, f, 0, Ac[m][f]);
        }
    }
    const bool pre = sw + AD < NSW;
    const uint8_t *brow_p = bb + (l % 16) * GT_BROW2 + (l / 16) * 64;
    uint4 Bq[2][4];
#pragma unroll
    for (int c = 0; c < NF; ++c)
      Bq[0][c] = *reinterpret_cast<const uint4 *>(brow_p + 16 * c * GT_BROW2);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (pre) {
        if constexpr (FP4) {
          if (sw % 2 == 0 && q < NM)
            fp4_pair_load<NM>(P[(sw / 2 + PD - 1) % PD], q, W, in, rbase, sw + AD, NSW);
        } else {
          if (q == 3) fp8_win_load<NM>(R8[sw & 1], W, S, in, rbase, sw + 2, NSW);
        }
        if (q >= 2) act_load<FP4>(B[sw % AD], q - 2, bsrc, in, brow, sw + AD, NSW);
      }
      if (q + 1 < 4) {
#pragma unroll
        for (int c = 0; c < NF; ++c)
          Bq[(q + 1) & 1][c] =
              *reinterpret_cast<const uint4 *>(brow_p + 16 * c * GT_BROW2 + 16 * (q + 1));
      }
      if (FP4 && q == 1 && sw + 1 < NSW) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int f = 0; f < 2; ++f) Acn[m][f] = code(m, f, sw + 1);
      }
      uint4 An[NM][2];
      if (q + 1 < 4) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int f = 0; f < 2; ++f) An[m][f] = a_op(sw, m, f, q + 1, Ac[m][f]);
      } else if (sw + 1 < NSW) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int f = 0; f < 2; ++f) An[m][f] = a_op(sw + 1, m, f, 0, Acn[m][f]);
      }
#pragma unroll
      for (int c = 0; c < NF; ++c)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int f = 0; f < 2; ++f)
            acc[m][f][c] = mfma_bf16(A[m][f], Bq[q & 1][c], acc[m][f][c]);
      // one MFMA, then up to two VALU instructions, repeated
#pragma unroll
      for (int i = 0; i < NF * NM * 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      if (q + 1 < 4 || sw + 1 < NSW) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int f = 0; f < 2; ++f) A[m][f] = An[m][f];
      }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int f = 0; f < 2; ++f) Ac[m][f] = Acn[m][f];
  }
}

template <int AFMT, int NSW>  // NSW > 0: H = 128 NSW, the unrolled loop
__device__ __forceinline__ void gateup_tile(const GroupedArgs &a, int e, int rt, int p0, int np,
                                            uint8_t *bt, int *rows_s, float *wt_s,
                                            float (*amax_s)[GT_TN], uint64_t *s_tab, uint8_t *cs) {
  const int tid = threadIdx.x, wv = tid / 64, l = tid % 64;
  const int H = a.H, I = a.I;
  const uint8_t *Wg, *Wu, *Sg, *Su;
  uint32_t wbytes, sbytes;
  if (AFMT == MX_FP4) {
    const uint8_t *sc = a.experts + (size_t)e * a.expert_stride;
    const uint8_t *wt = sc + a.scale_run;
    const size_t w1 = (size_t)I * (H / 2), w2 = (size_t)H * (I / 2);
    const size_t s1 = (size_t)I * (H / 32), s2 = (size_t)H * (I / 32);
    Wg = wt;
    Wu = wt + w1 + w2;
    Sg = sc;
    Su = sc + s1 + s2;
    wbytes = (uint32_t)w1;
    sbytes = (uint32_t)s1;
  } else {
    Wg = a.shw[0];
    Wu = a.shw[1];
    Sg = a.shs[0];
    Su = a.shs[1];
    wbytes = (uint32_t)I * (uint32_t)H;
    sbytes = (uint32_t)((I + 127) / 128) * (uint32_t)(H / 128);
  }
  if (tid < GT_TN) {
    if (AFMT == MX_FP8) {  // shared expert: position sh_base + t, weight 1
      rows_s[tid] = tid < np ? p0 - a.sh_base + tid : -1;
      wt_s[tid] = tid < np ? 1.0f : 0.0f;
    } else {
      rows_s[tid] = tid < np ? a.pos_token[p0 + tid] : -1;
      wt_s[tid] = tid < np ? a.pos_wt[p0 + tid] : 0.0f;
    }
  }
  libm_stage_table(s_tab);  // SwiGLU's expf table, read from LDS in the epilogue
  __syncthreads();
  const int nf = (np + 15) / 16;  // active token fragments (block-uniform)
  v4f acc[2][2][4];
  for (int m = 0; m < 2; ++m)
    for (int f = 0; f < 2; ++f)
      for (int c = 0; c < 4; ++c) acc[m][f][c] = (v4f){0.f, 0.f, 0.f, 0.f};
  const int rbase = rt * GT_TM + 32 * wv;
  const BufRsrc W[2] = {buf_rsrc(Wg, wbytes), buf_rsrc(Wu, wbytes)};
  const BufRsrc S[2] = {buf_rsrc(Sg, sbytes), buf_rsrc(Su, sbytes)};
  if (AFMT == MX_FP4) stage_codes<2>(cs, S, rt, H);
  if constexpr (NSW > 0) {
    const BufRsrc xr = buf_rsrc(a.xb, a.xb_bytes);
    if (AFMT == MX_FP4 && nf <= 1)
      gemm_k_loop_fast<AFMT, 2, NSW, 1, AFMT == MX_FP4 ? GU_PD_SMALL : 2>(acc, W, S, xr, H, rbase,
                                                                          rows_s, bt, cs);
    else if (AFMT == MX_FP4 && nf <= 2)
      gemm_k_loop_fast<AFMT, 2, NSW, 2, AFMT == MX_FP4 ? GU_PD_SMALL : 2>(acc, W, S, xr, H, rbase,
                                                                          rows_s, bt, cs);
    else if (AFMT == MX_FP4 && nf <= 3)
      gemm_k_loop_fast<AFMT, 2, NSW, 3>(acc, W, S, xr, H, rbase, rows_s, bt, cs);
    else
      gemm_k_loop_fast<AFMT, 2, NSW, 4>(acc, W, S, xr, H, rbase, rows_s, bt, cs);
  } else
    gemm_k_loop<AFMT, 2>(acc, W, S, buf_rsrc(a.xb, a.xb_bytes), H, rbase, rows_s, nf, bt, cs);
  // epilogue: y = bf16((silu(bf16(g)) * bf16(u)) * w), per-128 requant,
  // stored as the exact BF16 of the dequantised FP8 value
  float y[2][4][4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int j = 16 * c + l % 16;
    float m = 0.0f;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float yy = 0.0f;
        if (c < nf) {
          const float g = bf16_round(acc[0][f][c][v]), u = bf16_round(acc[1][f][c][v]);
          yy = bf16_round(swiglu_t(g, u, a.limit, s_tab) * wt_s[j]);
        }
        y[f][c][v] = yy;
        m = fmaxf(m, fabsf(yy));
      }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (l < 16) amax_s[wv][j] = m;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int j = 16 * c + l % 16;
    if (c >= nf || j >= np) continue;
    const float am = fmaxf(fmaxf(amax_s[0][j], amax_s[1][j]), fmaxf(amax_s[2][j], amax_s[3][j]));
    const float scale = act_scale(am);
    const float inv = 1.0f / scale;
    const int pos = p0 + j;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      uint32_t h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) h[v] = f2u(quant_e4m3(y[f][c][v], inv) * scale) >> 16;
      const int row = rbase + 16 * f + 4 * (l / 16);
      *reinterpret_cast<uint2 *>(a.yb + (size_t)pos * I + row) =
          make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
  }
}

// The tile of a routed expert's positions (token tile tt of the dispatch's
// tile table), or false past the last one.
__device__ __forceinline__ bool routed_tile(const GroupedArgs &a, int tt, int &e, int &p0,
                                            int &np) {
  if (tt >= a.tile_off[a.E]) return false;
  e = tile_expert(a.tile_off, a.E, tt);
  p0 = a.pos_off[e] + (tt - a.tile_off[e]) * GT_TN;
  np = min(GT_TN, a.pos_off[e + 1] - p0);
  return true;
}

// The shared expert's tile tt: every token, no routing needed.
__device__ __forceinline__ bool shared_tile(const GroupedArgs &a, int tt, int &e, int &p0,
                                            int &np) {
  if (tt * GT_TN >= a.T) return false;
  e = a.E;
  p0 = a.sh_base + tt * GT_TN;
  np = min(GT_TN, a.T - tt * GT_TN);
  return true;
}

// The first a.sh_wgs workgroups (0: none) take the shared expert's FP8 tiles
// (K windows SHNSW, 0: the generic loop): up to 256 tokens in the same launch
// as the routed tiles (no second stream, no fork and join, at the cost of the
// shared expert's bytes in the routed stream); beyond, as a launch of their
// own on the second stream with a grid of exactly those workgroups. The
// others take the routed experts' FP4 tiles (K windows NSW): grid = token-
// tile bound x row tiles (I / 128), workgroups past tile_off[E] exit at once.
// At most 256 registers (two waves per SIMD: the LDS admits two workgroups
// per CU). The LDS is declared once for both tile kinds.
template <int NSW, int SHNSW>
__device__ __forceinline__ void grouped_gateup(const GroupedArgs &a) {
  __shared__ __align__(16) uint8_t bt[2 * GT_BT_BYTES];
  __shared__ int rows_s[GT_TN];
  __shared__ float wt_s[GT_TN];
  __shared__ float amax_s[4][GT_TN];
  __shared__ uint64_t s_tab[32];
  extern __shared__ __align__(16) uint8_t codes_s[];  // FP4: 2 x codes_stride(H)
  int b = blockIdx.x, tt, rt, e, p0, np;
  if (b < a.sh_wgs) {
    tile_coords(b, a.sh_wgs, a.row_tiles, tt, rt);
    if (shared_tile(a, tt, e, p0, np))
      gateup_tile<MX_FP8, SHNSW>(a, e, rt, p0, np, bt, rows_s, wt_s, amax_s, s_tab, codes_s);
    return;
  }
  b -= a.sh_wgs;
  tile_coords(b, (int)gridDim.x - a.sh_wgs, a.row_tiles, tt, rt);
  if (routed_tile(a, tt, e, p0, np))
    gateup_tile<MX_FP4, NSW>(a, e, rt, p0, np, bt, rows_s, wt_s, amax_s, s_tab, codes_s);
}

template <int NSW, int SHNSW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_grouped_gateup(
    GroupedArgs a) {
  grouped_gateup<NSW, SHNSW>(a);
}

template <int AFMT, int NSW>  // NSW > 0: I = 128 NSW, the unrolled loop
__device__ __forceinline__ void down_tile(const GroupedArgs &a, int e, int rt, int p0, int np,
                                          uint8_t *bt, int *rows_s, uint8_t *cs) {
  const int tid = threadIdx.x, wv = tid / 64, l = tid % 64;
  const int H = a.H, I = a.I;
  const uint8_t *Wp, *Sp;
  uint32_t wbytes, sbytes;
  if (AFMT == MX_FP4) {
    const uint8_t *sc = a.experts + (size_t)e * a.expert_stride;
    Wp = sc + a.scale_run + (size_t)I * (H / 2);
    Sp = sc + (size_t)I * (H / 32);
    wbytes = (uint32_t)((size_t)H * (I / 2));
    sbytes = (uint32_t)((size_t)H * (I / 32));
  } else {
    Wp = a.shw[2];
    Sp = a.shs[2];
    wbytes = (uint32_t)H * (uint32_t)I;
    sbytes = (uint32_t)((H + 127) / 128) * (uint32_t)(I / 128);
  }
  if (tid < GT_TN) rows_s[tid] = tid < np ? p0 + tid : -1;  // positions are contiguous
  __syncthreads();
  const int nf = (np + 15) / 16;
  v4f acc[1][2][4];
  for (int f = 0; f < 2; ++f)
    for (int c = 0; c < 4; ++c) acc[0][f][c] = (v4f){0.f, 0.f, 0.f, 0.f};
  const int rbase = rt * GT_TM + 32 * wv;
  const BufRsrc W[1] = {buf_rsrc(Wp, wbytes)};
  const BufRsrc S[1] = {buf_rsrc(Sp, sbytes)};
  if (AFMT == MX_FP4) stage_codes<1>(cs, S, rt, I);
  if constexpr (NSW > 0) {
    const BufRsrc yr = buf_rsrc(a.yb, a.yb_bytes);
    if (AFMT == MX_FP4 && nf <= 1)
      gemm_k_loop_fast<AFMT, 1, NSW, 1, AFMT == MX_FP4 ? DN_PD_SMALL : 2>(acc, W, S, yr, I, rbase,
                                                                          rows_s, bt, cs);
    else if (AFMT == MX_FP4 && nf <= 2)
      gemm_k_loop_fast<AFMT, 1, NSW, 2, AFMT == MX_FP4 ? DN_PD_SMALL : 2>(acc, W, S, yr, I, rbase,
                                                                          rows_s, bt, cs);
    else if (AFMT == MX_FP4 && nf <= 3)
      gemm_k_loop_fast<AFMT, 1, NSW, 3>(acc, W, S, yr, I, rbase, rows_s, bt, cs);
    else
      gemm_k_loop_fast<AFMT, 1, NSW, 4>(acc, W, S, yr, I, rbase, rows_s, bt, cs);
  } else
    gemm_k_loop<AFMT, 1>(acc, W, S, buf_rsrc(a.yb, a.yb_bytes), I, rbase, rows_s, nf, bt, cs);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int j = 16 * c + l % 16;
    if (c >= nf || j >= np) continue;
    const int pos = p0 + j;
    const int t = AFMT == MX_FP8 ? pos - a.sh_base : a.pos_token[pos];
    const int k = AFMT == MX_FP8 ? a.K : a.pos_route[pos];
    uint16_t *dst = a.ro + ((size_t)t * (a.K + 1) + k) * H;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int row = rbase + 16 * f + 4 * (l / 16);
      uint2 o;
      o.x = (f2u(bf16_round(acc[0][f][c][0])) >> 16) |
            (f2u(bf16_round(acc[0][f][c][1])) & 0xFFFF0000u);
      o.y = (f2u(bf16_round(acc[0][f][c][2])) >> 16) |
            (f2u(bf16_round(acc[0][f][c][3])) & 0xFFFF0000u);
      *reinterpret_cast<uint2 *>(dst + row) = o;
      if (a.ro32)  // validation output: the fp32 accumulators themselves
        *reinterpret_cast<float4 *>(a.ro32 + ((size_t)t * (a.K + 1) + k) * H + row) =
            make_float4(acc[0][f][c][0], acc[0][f][c][1], acc[0][f][c][2], acc[0][f][c][3]);
    }
  }
}

// As k_grouped_gateup (shared and routed tiles), at most 168 registers:
// three waves per SIMD, as many as the LDS admits workgroups per CU.
template <int NSW, int SHNSW>
__device__ __forceinline__ void grouped_down(const GroupedArgs &a) {
  __shared__ __align__(16) uint8_t bt[2 * GT_BT_BYTES];
  __shared__ int rows_s[GT_TN];
  extern __shared__ __align__(16) uint8_t codes_s[];  // FP4: codes_stride(I)
  int b = blockIdx.x, tt, rt, e, p0, np;
  if (b < a.sh_wgs) {
    tile_coords(b, a.sh_wgs, a.row_tiles, tt, rt);
    if (shared_tile(a, tt, e, p0, np))
      down_tile<MX_FP8, SHNSW>(a, e, rt, p0, np, bt, rows_s, codes_s);
    return;
  }
  b -= a.sh_wgs;
  tile_coords(b, (int)gridDim.x - a.sh_wgs, a.row_tiles, tt, rt);
  if (routed_tile(a, tt, e, p0, np)) down_tile<MX_FP4, NSW>(a, e, rt, p0, np, bt, rows_s, codes_s);
}

template <int NSW, int SHNSW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_grouped_down(
    GroupedArgs a) {
  grouped_down<NSW, SHNSW>(a);
}

#define CB_SLOTS 8  // route slots (K + 1) summed from registers

// out[t][i] = bf16(((0 + r_0) + ... + r_{K-1}) + shared), routes in
// ascending expert id (src/dsv4/dsv4_model.c:7096-7112).
// out[t][c .. c + 7]: the routes in ascending expert id, then the shared
// expert (route slot K), each element summed in that order
// (src/dsv4/dsv4_model.c:6795-6805); 16-byte loads of 8 BF16 columns.
// A route without an expert (idx outside [0, E): no selectable choice was
// left, or a tid2eid entry out of range) was never dispatched, so its slot
// holds no output of this call: it adds nothing.
__global__ void k_combine_batch(float *__restrict__ out, const uint16_t *__restrict__ ro,
                                const int *__restrict__ idx, int T, int K, int H, int E) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;  // 8-column group
  const size_t g8 = (size_t)H / 8;
  if (i >= (size_t)T * g8) return;
  const size_t t = i / g8, c = (i % g8) * 8;
  const uint16_t *r = ro + t * (size_t)(K + 1) * H + c;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  auto add = [&](const uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] += u2f(w[j] << 16);
      acc[2 * j + 1] += u2f(w[j] & 0xFFFF0000u);
    }
  };
  if (K + 1 <= CB_SLOTS) {
    // every id and every slot loaded at once (addresses clamped into the
    // token's K + 1 slots, no branch), then summed in slot order
    int e[CB_SLOTS];
    uint4 v[CB_SLOTS];
#pragma unroll
    for (int k = 0; k < CB_SLOTS; ++k) e[k] = idx[t * K + min(k, K - 1)];
#pragma unroll
    for (int k = 0; k < CB_SLOTS; ++k)
      v[k] = *reinterpret_cast<const uint4 *>(r + (size_t)min(k, K) * H);
#pragma unroll
    for (int k = 0; k < CB_SLOTS; ++k)
      if (k < K ? (unsigned)e[k] < (unsigned)E : k == K) add(v[k]);
  } else {
    for (int k = 0; k <= K; ++k) {
      if (k < K && (unsigned)idx[t * K + k] >= (unsigned)E) continue;
      add(*reinterpret_cast<const uint4 *>(r + (size_t)k * H));
    }
  }
  float4 *o = reinterpret_cast<float4 *>(out + t * (size_t)H + c);
  o[0] = make_float4(bf16_round(acc[0]), bf16_round(acc[1]), bf16_round(acc[2]), bf16_round(acc[3]));
  o[1] = make_float4(bf16_round(acc[4]), bf16_round(acc[5]), bf16_round(acc[6]), bf16_round(acc[7]));
}

}  // namespace dsv4

// ============================================================ C-ABI =====
using namespace dsv4;

namespace {
struct BatchWs {
  uint16_t *xb, *yb;
  float *z, *zabs, *cscore, *cchoice, *wt, *pos_wt;
  int *off_bf16, *rcnt, *cand, *ncand, *chain_off, *idx, *counts, *bh, *pos_off, *tile_off, *pos_token,
      *pos_route;
  uint16_t *ro;
  size_t bytes;
};

// The shared expert's stream of each device, created on the first call that
// is not being captured into a graph (creating a stream there is not
// allowed; such a call runs the shared expert on the caller's stream).
// Default priority, non-blocking.
struct SideStream {
  hipStream_t s;
  hipEvent_t fork, join;
};
std::mutex g_side_mu;
SideStream g_side[64];
bool g_side_made[64];

int side_stream(hipStream_t st, SideStream **out) {
  *out = nullptr;
  int dev = 0;
  DSV4G_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return 0;
  if (!g_side_made[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    DSV4G_HIP(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone) return 0;
    SideStream n;
    DSV4G_HIP(hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking));
    DSV4G_HIP(hipEventCreateWithFlags(&n.fork, hipEventDisableTiming));
    DSV4G_HIP(hipEventCreateWithFlags(&n.join, hipEventDisableTiming));
    g_side[dev] = n;
    g_side_made[dev] = true;
  }
  *out = &g_side[dev];
  return 0;
}

// Up to this many tokens the router computes every score exactly
// (k_router_exact); beyond, candidates from approximate logits.
#define RX_MAX_TOKENS 256
// Up to this many tokens the shared expert's tiles are folded into the
// routed GEMM launches (one stream); beyond, they run on a second stream.
#define FOLD_MAX_TOKENS 256

BatchWs batch_ws_layout(const DSV4GLayer *L, int T, void *base) {
  const size_t t = (size_t)T, K = (size_t)L->topk, E = (size_t)L->n_experts;
  const size_t H = (size_t)L->hidden, I = (size_t)L->inter, P = t * K + t;
  BatchWs w = {};
  // the first 4096 bytes stay untouched: a workspace shared with the decode
  // entry keeps that entry's (zero) control words there
  uintptr_t p = (((uintptr_t)base + 255) & ~(uintptr_t)255) + 4096;
  const uintptr_t p0 = (uintptr_t)base;
  auto take = [&](size_t bytes) {
    void *r = (void *)p;
    p += (bytes + 255) & ~(size_t)255;
    return r;
  };
  w.xb = (uint16_t *)take(t * H * 2);
  w.off_bf16 = (int *)take(t * ((H + 255) / 256) * 4);
  w.rcnt = (int *)take(4);
  w.z = (float *)take(t * E * 4);
  w.zabs = (float *)take(t * E * 4);
  w.cand = (int *)take(t * E * 4);
  w.ncand = (int *)take(t * 4);
  w.chain_off = (int *)take((t + 1) * 4);
  w.cscore = (float *)take(t * E * 4);
  w.cchoice = (float *)take(t * E * 4);
  w.idx = (int *)take(t * K * 4);
  w.wt = (float *)take(t * K * 4);
  w.counts = (int *)take(E * 4);
  w.bh = (int *)take(((t * K + DP_ROUTES - 1) / DP_ROUTES) * E * 4);
  w.pos_off = (int *)take((E + 2) * 4);
  w.tile_off = (int *)take((E + 2) * 4);
  w.pos_token = (int *)take(P * 4);
  w.pos_route = (int *)take(P * 4);
  w.pos_wt = (float *)take(P * 4);
  w.yb = (uint16_t *)take(P * I * 2);
  w.ro = (uint16_t *)take(t * (K + 1) * H * 2);
  w.bytes = (size_t)(p - p0) + 256;
  return w;
}
}  // namespace

extern "C" {

size_t dsv4g_moe_batch_workspace_bytes(const DSV4GLayer *L, int n_tokens) {
  return batch_ws_layout(L, n_tokens, nullptr).bytes;
}

// Batched MoE layer (moe_forward_batch semantics) for n_tokens rows of x
// (BF16 values in fp32). out [n][hidden]; idx/wt (optional, device).
int dsv4g_moe_forward_batch(float *out, const float *x, const DSV4GLayer *L,
                            const int *token_ids, int n_tokens, void *workspace,
                            size_t workspace_bytes, int *idx_out, float *wt_out,
                            void *stream) {
  return dsv4g_moe_forward_batch_routes(out, x, L, token_ids, n_tokens, workspace,
                                        workspace_bytes, idx_out, wt_out, nullptr, stream);
}

int dsv4g_moe_forward_batch_routes(float *out, const float *x, const DSV4GLayer *L,
                                   const int *token_ids, int n_tokens, void *workspace,
                                   size_t workspace_bytes, int *idx_out, float *wt_out,
                                   float *route_out, void *stream) {
  if (!L || !L->gate_w || !L->experts || !L->sh1 || !L->sh2 || !L->sh3)
    return dsv4g_fail(DSV4G_EINVAL, "moe_forward_batch: layer descriptor incomplete");
  const int T = n_tokens, K = L->topk, E = L->n_experts, H = L->hidden, I = L->inter;
  if (T <= 0 || H % 128 || I % 128 || H > 8192 || I > 8192 || E <= 0 || E > 1024 || K <= 0 ||
      K > 32 || K > E)
    return dsv4g_fail(DSV4G_EINVAL, "moe_forward_batch: unsupported shape");
  if (L->tid2eid && !token_ids)
    return dsv4g_fail(DSV4G_EINVAL, "moe_forward_batch: hash layer needs token_ids");
  // the GEMMs address the activation buffers with 32-bit offsets below 2 GiB
  if ((size_t)T * (K + 1) * I * 2 >= (1ull << 31) || (size_t)T * H * 2 >= (1ull << 31))
    return dsv4g_fail(DSV4G_EINVAL, "moe_forward_batch: too many tokens for one call (%d)", T);
  if (workspace_bytes < dsv4g_moe_batch_workspace_bytes(L, T))
    return dsv4g_fail(DSV4G_EINVAL, "moe_forward_batch: workspace too small (%zu < %zu)",
                      workspace_bytes, dsv4g_moe_batch_workspace_bytes(L, T));
  hipStream_t st = (hipStream_t)stream;
  BatchWs w = batch_ws_layout(L, T, workspace);
  // the routes go straight into the caller's buffers when given
  if (idx_out) w.idx = idx_out;
  if (wt_out) w.wt = wt_out;

  const bool exact_router = T <= RX_MAX_TOKENS;
  // 1. activation quant (+ BF16-valued flags)
  {
    const size_t waves = (size_t)T * ((H + 255) / 256);
    hipLaunchKernelGGL(k_batch_quant, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, w.xb,
                       w.off_bf16, w.rcnt, x, T, H);
  }
  DSV4G_TRY(dsv4g_check_launch("batch_quant"));
  GroupedArgs g = {};
  g.experts = L->experts;
  g.expert_stride = L->expert_stride;
  g.scale_run = L->scale_run;
  g.shw[0] = L->sh1;
  g.shw[1] = L->sh3;
  g.shw[2] = L->sh2;
  g.shs[0] = L->sh1_s;
  g.shs[1] = L->sh3_s;
  g.shs[2] = L->sh2_s;
  g.tile_off = w.tile_off;
  g.pos_off = w.pos_off;
  g.pos_token = w.pos_token;
  g.pos_route = w.pos_route;
  g.pos_wt = w.pos_wt;
  g.xb = w.xb;
  g.yb = w.yb;
  g.xb_bytes = (uint32_t)((size_t)T * H * 2);
  g.yb_bytes = (uint32_t)((size_t)T * (K + 1) * I * 2);
  g.ro = w.ro;
  g.ro32 = route_out;
  g.H = H;
  g.I = I;
  g.E = E;
  g.K = K;
  g.T = T;
  g.limit = (float)(int)L->swiglu_limit;
  g.sh_base = T * K;  // past every routed position (at most T K)
  // routed token tiles: at most ceil(T K / 64) + E (one partial tile per
  // expert); the shared expert's: ceil(T / 64)
  const long routed_bound = ((long)T * K + GT_TN - 1) / GT_TN + E;
  const long shared_tiles = (T + GT_TN - 1) / GT_TN;
  const uint32_t gu_codes = 2u * codes_stride(H), dn_codes = codes_stride(I);
  // the unrolled K loops for the model's widths, else the per-window loop.
  // Few tokens: the shared expert's tiles go into the routed launches (its
  // second stream would cost a fork and a join, several microseconds each,
  // on a path of a few hundred); many tokens: it runs on the second stream
  // beside the router, which it then hides behind.
  const bool fold = T <= FOLD_MAX_TOKENS;
  const void *gu4 = H == 4096 ? (const void *)k_grouped_gateup<32, 32>
                              : (const void *)k_grouped_gateup<0, 0>;
  const void *dn4 = I == 2048 ? (const void *)k_grouped_down<16, 16>
                              : (const void *)k_grouped_down<0, 0>;
  // calls hold this lock while they set up and enqueue: the attribute
  // flags below, and the fork and join events of two calls, cannot interleave
  std::lock_guard<std::mutex> lock(g_side_mu);
  {
    // the kernels' dynamic LDS limit (H, I <= 8192: <= 64 KiB), once per
    // device (under the enqueue lock)
    static bool attr_set[64];
    int dev = 0;
    DSV4G_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < 64 && !attr_set[dev]) {
      const void *fs[4] = {(const void *)k_grouped_gateup<32, 32>,
                           (const void *)k_grouped_gateup<0, 0>,
                           (const void *)k_grouped_down<16, 16>,
                           (const void *)k_grouped_down<0, 0>};
      for (int i = 0; i < 4; ++i)
        DSV4G_HIP(hipFuncSetAttribute(fs[i], hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
      attr_set[dev] = true;
    }
  }
  // the shared expert needs only the quantised activations: its gate/up and
  // down run on a second stream beside the router, dispatch and routed
  // GEMMs (joined before the combine). Calls hold a lock while they enqueue,
  // so the fork and join events of two calls cannot interleave.
  SideStream *side = nullptr;
  if (!fold) DSV4G_TRY(side_stream(st, &side));
  if (side) {
    // a capture forked into the side stream stays open there until its
    // caller ends it: a call that is not part of that same capture runs the
    // shared expert on its own stream instead of joining a foreign graph
    hipStreamCaptureStatus cs_side = hipStreamCaptureStatusNone, cs = hipStreamCaptureStatusNone;
    unsigned long long id_side = 0, id = 0;
    DSV4G_HIP(hipStreamGetCaptureInfo(side->s, &cs_side, &id_side));
    if (cs_side != hipStreamCaptureStatusNone) {
      DSV4G_HIP(hipStreamGetCaptureInfo(st, &cs, &id));
      if (cs != hipStreamCaptureStatusActive || id != id_side) side = nullptr;
    }
  }
  hipStream_t sst = side ? side->s : st;
  if (side) {
    DSV4G_HIP(hipEventRecord(side->fork, st));
    DSV4G_HIP(hipStreamWaitEvent(sst, side->fork, 0));
  }
  if (!fold) {
    // the same kernels with a grid of exactly the shared expert's workgroups
    // (no routed tiles; the FP8 tiles use no code buffer: no dynamic LDS)
    g.row_tiles = I / GT_TM;
    g.sh_wgs = (int)(shared_tiles * g.row_tiles);
    hipLaunchKernelGGL((void (*)(GroupedArgs))gu4, dim3((unsigned)g.sh_wgs), dim3(256), 0, sst, g);
    DSV4G_TRY(dsv4g_check_launch("grouped_gateup_shared"));
    g.row_tiles = H / GT_TM;
    g.sh_wgs = (int)(shared_tiles * g.row_tiles);
    hipLaunchKernelGGL((void (*)(GroupedArgs))dn4, dim3((unsigned)g.sh_wgs), dim3(256), 0, sst, g);
    DSV4G_TRY(dsv4g_check_launch("grouped_down_shared"));
  }
  if (side) DSV4G_HIP(hipEventRecord(side->join, sst));
  // 2. router
  if (exact_router) {
    hipLaunchKernelGGL(k_router_exact, dim3((unsigned)((T + RX_TOK - 1) / RX_TOK),
                                            (unsigned)((E + RX_EXP - 1) / RX_EXP)),
                       dim3(64), 0, st, w.cscore, w.cchoice, x, L->gate_w, L->bias, T, H, E);
    if (T * K > 1024) {
      auto sel = E <= 64 ? k_router_select<1> : E <= 128 ? k_router_select<2>
               : E <= 256 ? k_router_select<4> : E <= 512 ? k_router_select<8>
                          : k_router_select<16>;
      hipLaunchKernelGGL(sel, dim3((T + 3) / 4), dim3(256), 0, st, w.idx, w.wt, w.cscore,
                         w.cchoice, L->tid2eid, token_ids, T, E, K, L->route_scale);
    }
  } else {
    const dim3 grid((T + 63) / 64, (E + 63) / 64);
    if (H == 4096)
      hipLaunchKernelGGL(k_router_logits_mfma<32>, grid, dim3(256), 0, st, w.z, w.zabs, x,
                         L->gate_w, T, H, E);
    else
      hipLaunchKernelGGL(k_router_logits_mfma<0>, grid, dim3(256), 0, st, w.z, w.zabs, x,
                         L->gate_w, T, H, E);
    auto cand = E <= 64 ? k_router_cand<1> : E <= 128 ? k_router_cand<2> : E <= 256 ? k_router_cand<4>
              : E <= 512 ? k_router_cand<8> : k_router_cand<16>;
    hipLaunchKernelGGL(cand, dim3((T + 3) / 4), dim3(256), 0, st, w.cand, w.ncand, w.z, w.zabs,
                       w.off_bf16, (H + 255) / 256, L->bias, L->tid2eid, token_ids, T, H, E, K);
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, st, w.chain_off, w.ncand, T);
    const long bound = (long)T * (K + 4);
    const int blocks = (int)((bound + 255) / 256 < 4096 ? (bound + 255) / 256 : 4096);
    // every token has at least K candidates: for K >= 5 a wave's 64 chains
    // span at most 14 tokens, whose x slices k_router_chains_x stages in LDS
    if (K >= 5)
      hipLaunchKernelGGL(k_router_chains_x, dim3(blocks), dim3(256), 0, st, w.cscore, w.cchoice,
                         w.cand, w.chain_off, x, L->gate_w, L->bias, T, H, E);
    else
      hipLaunchKernelGGL(k_router_chains, dim3(blocks), dim3(256), 0, st, w.cscore, w.cchoice,
                         w.cand, w.chain_off, x, L->gate_w, L->bias, T, H, E);
    hipLaunchKernelGGL(k_router_finalize, dim3((T + 3) / 4), dim3(256), 0, st, w.idx, w.wt,
                       w.cand, w.ncand, w.cscore, w.cchoice, L->tid2eid ? 1 : 0, T, E, K,
                       L->route_scale);
  }
  DSV4G_TRY(dsv4g_check_launch("router"));
  // 3. dispatch
  if (exact_router && T * K <= 1024) {
    auto sd = E <= 64 ? k_select_dispatch<1> : E <= 128 ? k_select_dispatch<2>
            : E <= 256 ? k_select_dispatch<4> : E <= 512 ? k_select_dispatch<8>
                       : k_select_dispatch<16>;
    hipLaunchKernelGGL(sd, dim3((unsigned)((T + SD_WAVES - 1) / SD_WAVES)), dim3(1024), 0, st,
                       w.idx, w.wt, w.rcnt, w.pos_token, w.pos_route, w.pos_wt, w.pos_off,
                       w.tile_off, w.cscore, w.cchoice, L->tid2eid, token_ids, T, E, K,
                       L->route_scale);
  } else if (T * K <= 1024) {
    hipLaunchKernelGGL(k_dispatch_small, dim3(1), dim3(1024), 0, st, w.pos_token, w.pos_route,
                       w.pos_wt, w.pos_off, w.tile_off, w.idx, w.wt, T, K, E);
  } else {
    const int nb = (T * K + DP_ROUTES - 1) / DP_ROUTES;
    hipLaunchKernelGGL(k_dispatch_hist, dim3(nb), dim3(256), 0, st, w.bh, w.idx, T * K, E);
    hipLaunchKernelGGL(k_dispatch_scan_blocks, dim3(E), dim3(256), 0, st, w.bh, w.counts, nb);
    hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(1024), 0, st, w.counts, w.pos_off,
                       w.tile_off, T, E);
    hipLaunchKernelGGL(k_dispatch_fill, dim3(nb), dim3(256), 0, st, w.pos_token, w.pos_route,
                       w.pos_wt, w.bh, w.pos_off, w.idx, w.wt, T, K, E);
  }
  DSV4G_TRY(dsv4g_check_launch("dispatch"));
  // 4-5. routed grouped GEMMs
  g.row_tiles = I / GT_TM;
  g.sh_wgs = fold ? (int)(shared_tiles * g.row_tiles) : 0;
  hipLaunchKernelGGL((void (*)(GroupedArgs))gu4,
                     dim3((unsigned)(g.sh_wgs + routed_bound * g.row_tiles)), dim3(256), gu_codes,
                     st, g);
  DSV4G_TRY(dsv4g_check_launch("grouped_gateup"));
  g.row_tiles = H / GT_TM;
  g.sh_wgs = fold ? (int)(shared_tiles * g.row_tiles) : 0;
  hipLaunchKernelGGL((void (*)(GroupedArgs))dn4,
                     dim3((unsigned)(g.sh_wgs + routed_bound * g.row_tiles)), dim3(256), dn_codes,
                     st, g);
  DSV4G_TRY(dsv4g_check_launch("grouped_down"));
  // 6. combine, after the shared expert's stream
  if (side) DSV4G_HIP(hipStreamWaitEvent(st, side->join, 0));
  const size_t total = (size_t)T * H / 8;  // 8-column groups (H % 128 == 0)
  hipLaunchKernelGGL(k_combine_batch, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     out, w.ro, w.idx, T, K, H, E);
  DSV4G_TRY(dsv4g_check_launch("combine_batch"));
  return 0;
}

}  // extern "C"
