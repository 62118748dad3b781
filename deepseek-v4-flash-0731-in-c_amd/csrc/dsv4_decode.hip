// dsv4_decode.hip - the decode MoE layer on gfx950: moe_forward
// (src/dsv4/dsv4_model.c:6599-6807) for a few tokens, bit for bit, as four
// kernels per layer.
//
//   k_dec_router   approximate router logits z and sum|w*x| for every
//                  (token, expert) and the approximate choice
//                  sqrt_softplus(z) + bias, one workgroup per expert; the
//                  FP8 activation quant of x.
//   k_dec_gateup   every workgroup that needs them derives the token's
//                  candidate experts (below) from the approximate choices
//                  first; then gate and up GEMVs of every candidate (FP4) and of the
//                  shared expert (FP8), a workgroup holding the same rows of
//                  both so that it writes t = silu(bf16 gate) * bf16 up
//                  (src/dsv4/dsv4_model.c:6264-6268); beside them one
//                  workgroup per candidate slot runs the reference's exact
//                  sequential logit chain (dsv4_gemv_bf16,
//                  src/dsv4/dsv4_model.c:298-303), and the last of those
//                  takes the exact top-k and route weights
//                  (src/dsv4/dsv4_model.c:6615-6676).
//   k_dec_down     per (token, route): y = bf16(t * w), per-128 FP8 requant
//                  into LDS (src/dsv4/dsv4_model.c:6239-6287), the down GEMV.
//   k_dec_combine  the routes in ascending expert id, then the shared expert,
//                  rounded to BF16 (src/dsv4/dsv4_model.c:6795-6805).
//
// Candidates. A parallel logit differs from the sequential fmaf chain by at
// most gamma_d + gamma_H times sum|w*x| (d: the parallel sum's rounding
// depth, dec_par_depth). Mapped through |d score / dz| <= 1/2 plus slack for
// the score's own rounding, and doubled for both sides, that gives delta: an
// expert whose approximate choice is below (k-th best approximate choice) -
// delta has k experts surely above it and cannot be selected. The others are
// the candidates, in ascending expert id. Gate/up runs for every candidate
// (persistent workgroups over (candidate, tile) items) while the exact
// chains run beside it, one chain workgroup per candidate position modulo
// maxc, so the chains' latency (a 4096-long dependent fmaf chain, about
// 15 us) hides under the weight stream. Near-ties (a constant gate) only
// make more items.
//
// The candidates are derived redundantly by each workgroup of k_dec_gateup
// that needs them (a few hundred cycles of one wave, beside the workgroup's
// first loads): a last-arrival hand-off in k_dec_router would cost a
// device-scope fence and a memory round trip on the critical path. The
// hand-off from the chains to the selection uses one device-scope release
// fence and counter increment per workgroup; the last arrival acquires, does
// the work and resets its counter. The counters
// sit in the first bytes of the workspace, which must be zero before the
// first call (dsv4g_moe_workspace_init); every call leaves them zero.
#include <mutex>

#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"
#include "dsv4_tiles.h"

namespace dsv4 {

#define DEC_CTL_BYTES 4096  // control words: [0] + one per token, so n <= 1023
#define DEC_NP 8            // passes per FP4 tile (gate/up pairs and down)

struct DecArgs {
  const float *x;
  float *out;
  const uint16_t *gate;
  const float *bias;
  const int64_t *tid2eid;
  const int *token_ids;
  const uint8_t *experts;
  size_t expert_stride, scale_run;
  const uint8_t *sh[3], *sh_s[3];  // shared gate, up, down
  unsigned *ctl;                   // [1 + t] chain arrivals of token t ([0] unused)
  uint8_t *qx8;                    // [n][H] E4M3 codes of the quantised activation
  float *qxs;                      // [n][H/128] its scales
  float *ch, *zabs, *za;           // [n][E]: approximate choice, sum|w*x|, logit
  int *cand;                       // [n][E] candidate ids, ascending
  int *ncand;                      // [n]
  float *zx, *zc;                  // [n][E] exact score sqrt_softplus(z) and choice score + bias
                                   // per candidate position
  int *sel_e;                      // [n][K] routing, ascending id (moe_forward's idx)
  int *sel_pos;                    // [n][K] candidate position of each route
  float *sel_w;                    // [n][K] route weights (moe_forward's wt)
  float *sv;                       // [n][E + 1][I] SwiGLU t per candidate position; slot E = shared
  float *ro;                       // [n][K + 1][H] per-route outputs (BF16 values)
  int *idx_out;                    // optional copies of the routing
  float *wt_out;
  int n, H, I, E, K, maxc;
  int gu_tiles, dn_tiles;  // paired gate/up tiles (rows I, in H); down tiles (rows H, in I)
  int gu_nb;               // persistent routed gate/up workgroups per token
  float route_scale, limit;
  float gamma;  // gamma_{dec_par_depth(H)} + gamma_H, the candidates' bound factor
  int fast;  // routing from the parallel logits when the candidates are exactly top-k
};

// Expert e's matrix m (0 gate w1, 1 up w3, 2 down w2) in the reference slot
// layout [s1 | s2 | s3 | w1 | w2 | w3] (src/dsv4/dsv4_model.c:1584-1640).
__device__ __forceinline__ void expert_mat(const DecArgs &a, int e, int m, const uint8_t *&W,
                                           const uint8_t *&S) {
  const uint8_t *sc = a.experts + (size_t)e * a.expert_stride;
  const uint8_t *wt = sc + a.scale_run;
  const size_t w1 = (size_t)a.I * (a.H / 2), w2 = (size_t)a.H * (a.I / 2);
  const size_t s1 = (size_t)a.I * (a.H / 32), s2 = (size_t)a.H * (a.I / 32);
  if (m == 0) {
    W = wt;
    S = sc;
  } else if (m == 1) {
    W = wt + w1 + w2;
    S = sc + s1 + s2;
  } else {
    W = wt + w1;
    S = sc + s1;
  }
}

// The 4096 bytes of FP4 tile scales follow the tile's pairs in dynamic LDS.
__device__ __forceinline__ uint8_t *fp4_scale_lds(float *lds, const Fp4Geom &q) {
  return reinterpret_cast<uint8_t *>(lds) + (size_t)q.tr * pair_stride(q.G) * 8;
}

// One arrival on *cnt by the calling workgroup, after its global writes;
// true (workgroup-uniform) for the arrival that completes `total`, which then
// sees every other arrival's writes.
__device__ __forceinline__ bool dec_arrive_last(unsigned *cnt, unsigned total, int *s_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == total - 1u;
    if (last) __threadfence();
    *s_flag = last;
  }
  __syncthreads();
  return *s_flag != 0;
}

__device__ __forceinline__ void dec_select_finish(const DecArgs &a, int t, int my_e, float my_sc,
                                                  int my_pos);

// Rounding depth of a parallel logit of dec_logit_block: the product (one
// rounding), a lane's sequential sum of its 8-column pieces (at most
// 8 ceil(H / 2048) products), the 6-level wave butterfly, the 3 additions of
// the four waves' partials, and one more for the rounding of the computed
// sum|w*x| that the bound is scaled by.
__device__ __host__ __forceinline__ int dec_par_depth(int H) { return 8 * ((H / 4 + 511) / 512) + 11; }

// Candidates of token t in ascending expert id (whole calling wave) into
// cand[0 .. count) (LDS); returns the count. A hash layer's candidates are its
// tid2eid row. NPER = experts per lane (E <= 64 * NPER). One workgroup per
// token publishes: it also writes the list to a.cand / a.ncand and, in fast
// mode when the candidates are exactly the top-k, the routing, taken from
// the approximate choices (selection order) and the parallel logits (scores).
template <int NPER>
__device__ __forceinline__ int dec_candidates_t(const DecArgs &a, int t, int *cand, bool publish,
                                                const uint64_t *tab) {
  const int lane = threadIdx.x % 64;
  const size_t row = (size_t)t * a.E;
  const float ninf = -__builtin_inff();
  float v[NPER], z[NPER];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int e = lane + 64 * j;
    v[j] = ninf;
    z[j] = 0.0f;
    if (e < a.E) {
      const float c = a.ch[row + e];
      v[j] = c == c ? c : ninf;  // a NaN choice never wins a strict '>'
      amax = fmaxf(amax, a.zabs[row + e]);
      if (a.fast) z[j] = a.za[row + e];
    }
  }
  // k-th best approximate choice: k times remove one instance of the
  // maximum; lane k keeps the expert and logit of the k-th removal
  float kth = ninf, my_z = 0.0f;
  int my_e = -1;
  unsigned used = 0u;
  for (int k = 0; k < a.K; ++k) {
    float m = ninf, mz = 0.0f;
    int mj = -1;
#pragma unroll
    for (int j = 0; j < NPER; ++j)
      if (!((used >> j) & 1u) && v[j] > m) {
        m = v[j];
        mz = z[j];
        mj = j;
      }
    const float wm = wave_max_dpp(m);
    const unsigned long long bal = __ballot(mj >= 0 && m == wm);
    if (bal == 0ull) {  // fewer than k selectable experts
      kth = ninf;
      break;
    }
    const int wl = __builtin_ctzll(bal);
    if (lane == wl) used |= 1u << mj;
    const int we = wl + 64 * __builtin_amdgcn_readlane(mj, wl);
    const float wz = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mz), wl));
    if (lane == k) {
      my_e = we;
      my_z = wz;
    }
    kth = wm;
  }
  const float sum_abs = wave_max_dpp(amax);
  const float bound_z = a.gamma * sum_abs;  // gamma_{dec_par_depth(H)} + gamma_H
  const float thr = kth - 2.0f * (0.5f * bound_z + 1e-5f);
  int base = 0;
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int e = lane + 64 * j;
    const bool p = e < a.E && v[j] >= thr;
    const unsigned long long bal = __ballot(p);
    const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
    if (p) {
      cand[pos] = e;
      if (publish) a.cand[row + pos] = e;
    }
    base += __popcll(bal);
  }
  if (publish) {
    if (lane == 0) a.ncand[t] = base;
    if (a.fast && base == a.K) {  // the same test as dec_chain_block's early exit
      // candidates == top-k: sel_pos is the rank by id (dec_select_finish)
      dec_select_finish(a, t, my_e, lane < a.K ? sqrt_softplus(my_z, tab) : 0.0f, -1);
    }
  }
  return base;
}

__device__ __forceinline__ int dec_candidates(const DecArgs &a, int t, int *cand, bool publish,
                                              const uint64_t *tab) {
  if (a.tid2eid) {
    // the tid2eid row (K <= 32 <= lanes), in row order
    const int lane = threadIdx.x % 64;
    const int64_t *row = a.tid2eid + (size_t)a.token_ids[t] * a.K;
    const int e = lane < a.K ? (int)row[lane] : -1;
    if (lane < a.K) {
      cand[lane] = e;
      if (publish) a.cand[(size_t)t * a.E + lane] = e;
    }
    if (publish) {
      if (lane == 0) a.ncand[t] = a.K;
      if (a.fast) {
        // the row routes; weights from the parallel logits (route k = lane k)
        const bool ok = e >= 0 && e < a.E;
        dec_select_finish(a, t, e, ok ? sqrt_softplus(a.za[(size_t)t * a.E + e], tab) : 0.0f,
                          lane);
      }
    }
    return a.K;
  }
  if (a.E <= 64) return dec_candidates_t<1>(a, t, cand, publish, tab);
  if (a.E <= 128) return dec_candidates_t<2>(a, t, cand, publish, tab);
  if (a.E <= 256) return dec_candidates_t<4>(a, t, cand, publish, tab);
  if (a.E <= 512) return dec_candidates_t<8>(a, t, cand, publish, tab);
  return dec_candidates_t<16>(a, t, cand, publish, tab);
}


// Exact top-k of token t from the candidates' exact scores and choices (one
// whole wave; the nc candidates ct in ascending id, from the caller's LDS):
// routes ascending by id with weights and candidate positions, written to
// sel_* (and idx_out / wt_out) (src/dsv4/dsv4_model.c:6615-6676). Lane k
// carries route k in selection order.
template <int NPER>
__device__ __forceinline__ void dec_select_t(const DecArgs &a, int t, int nc, const int *ct) {
  const int lane = threadIdx.x % 64;
  const int K = a.K;
  const float *zt = a.zx + (size_t)t * a.E, *zc = a.zc + (size_t)t * a.E;
  int my_e = -1, my_pos = -1;
  float my_sc = 0.0f;
  if (a.tid2eid) {
    if (lane < K) {
      my_e = ct[lane];
      my_pos = lane;
      my_sc = (my_e >= 0 && my_e < a.E) ? zt[lane] : 0.0f;
    }
  } else {
    const float ninf = -__builtin_inff();
    float sc[NPER], chv[NPER];
    int ce[NPER];
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
      const int pos = lane + 64 * j;
      sc[j] = 0.0f;
      chv[j] = ninf;
      ce[j] = -1;
      if (pos < nc) {
        ce[j] = ct[pos];
        sc[j] = zt[pos];
        chv[j] = zc[pos];
      }
    }
    unsigned used = 0u;
    for (int k = 0; k < K; ++k) {
      // strict '>' in ascending id: the lowest id (position) wins a tie
      float m = ninf;
      int mj = -1;
#pragma unroll
      for (int j = 0; j < NPER; ++j)
        if (!((used >> j) & 1u) && chv[j] > m) {
          m = chv[j];
          mj = j;
        }
      const float wm = wave_max_dpp(m);
      const int win = wave_min_dpp((mj >= 0 && m == wm) ? lane + 64 * mj : 0x7fffffff);
      if (win == 0x7fffffff) continue;  // nothing left: route k stays empty (-1)
      float wsc = 0.0f;
      int we = -1;
#pragma unroll
      for (int j = 0; j < NPER; ++j)
        if (j == mj) {
          wsc = sc[j];
          we = ce[j];
        }
      const int wl = win % 64;
      if (lane == wl) used |= 1u << mj;
      const float bsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsc), wl));
      const int be = __builtin_amdgcn_readlane(we, wl);
      if (lane == k) {
        my_e = be;
        my_sc = bsc;
        my_pos = win;
      }
    }
  }
  dec_select_finish(a, t, my_e, my_sc, my_pos);
}

// Route weights from the unbiased scores, summed in selection order, then the
// routes sorted by id (src/dsv4/dsv4_model.c:6650-6674; equal ids carry
// equal weights, so any order among them matches the exchange sort). Lane k
// holds route k in selection order.
__device__ __forceinline__ void dec_select_finish(const DecArgs &a, int t, int my_e, float my_sc, int my_pos) {
  const int lane = threadIdx.x % 64;
  const int K = a.K;
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int ek = __builtin_amdgcn_readlane(my_e, k);
    const float sk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sc), k));
    sum += ek >= 0 ? sk : 0.0f;
  }
  const float rs = sum > 0.0f ? a.route_scale / sum : 0.0f;
  const float my_w = (sum > 0.0f && my_e >= 0) ? my_sc * rs : 0.0f;
  int rank = 0;
  for (int k = 0; k < K; ++k) {
    const int ek = __builtin_amdgcn_readlane(my_e, k);
    rank += (ek < my_e || (ek == my_e && k < lane)) ? 1 : 0;
  }
  if (lane < K) {
    const size_t o = (size_t)t * K + rank;
    a.sel_e[o] = my_e;
    a.sel_w[o] = my_w;
    a.sel_pos[o] = my_pos >= 0 ? my_pos : rank;  // fast path: candidates == routes
    if (a.idx_out) a.idx_out[o] = my_e;
    if (a.wt_out) a.wt_out[o] = my_w;
  }
}

// More than 256 candidates (near-ties or large expert counts): scores in
// LDS (2 * nc floats, nc <= 1024), scanned with plain loops.
__device__ __forceinline__ void dec_select_big(const DecArgs &a, int t, int nc, const int *ct,
                                               float *lds) {
  const int lane = threadIdx.x % 64;
  const float *zt = a.zx + (size_t)t * a.E, *zc = a.zc + (size_t)t * a.E;
  const float ninf = -__builtin_inff();
  float *sc = lds, *chv = lds + nc;
  for (int pos = lane; pos < nc; pos += 64) {
    sc[pos] = zt[pos];
    chv[pos] = zc[pos];
  }
  __builtin_amdgcn_wave_barrier();
  int my_e = -1, my_pos = -1;
  float my_sc = 0.0f;
  for (int k = 0; k < a.K; ++k) {
    float m = ninf;
    int mp = 0x7fffffff;
    for (int pos = lane; pos < nc; pos += 64)
      if (chv[pos] > m) {  // ascending positions: the lowest wins a tie
        m = chv[pos];
        mp = pos;
      }
    const float wm = wave_max_dpp(m);
    const int win = wave_min_dpp((mp != 0x7fffffff && m == wm) ? mp : 0x7fffffff);
    if (win == 0x7fffffff) continue;
    if (lane == k) {
      my_e = ct[win];
      my_sc = sc[win];
      my_pos = win;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) chv[win] = ninf;  // taken
    __builtin_amdgcn_wave_barrier();
  }
  dec_select_finish(a, t, my_e, my_sc, my_pos);
}

__device__ __forceinline__ void dec_select(const DecArgs &a, int t, int nc, const int *ct,
                                           float *lds) {
  if (a.tid2eid || nc <= 64) return dec_select_t<1>(a, t, nc, ct);
  if (nc <= 128) return dec_select_t<2>(a, t, nc, ct);
  if (nc <= 256) return dec_select_t<4>(a, t, nc, ct);
  dec_select_big(a, t, nc, ct, lds);
}

// ------------------------------------------------------------ router ----
// Router logit of expert e for every token, one workgroup: wave wv takes the
// columns [wv H/4, (wv + 1) H/4), lane l its 8-column pieces l, l + 64, ...
// (the gate row stays in registers, x is read directly); approximate choice
// sqrt_softplus(z) + bias, sum|w*x| and z (rounding depth: dec_par_depth).
__device__ __forceinline__ void dec_logit_block(const DecArgs &a, int e, float *s_part,
                                                uint64_t *s_tab) {
  const int tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
  const int H = a.H, Q = H / 4;
  const BufRsrc rg = buf_rsrc(a.gate + (size_t)e * H + (size_t)wv * Q, 2u * (uint32_t)Q);
  uint4 w[4];  // Q <= 2048: at most 4 pieces per lane; pieces past Q read zeros
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = buf_load16(rg, 16u * (uint32_t)(lane + 64 * i));
  const uint64_t tabv = libm_table_load();
  for (int t = 0; t < a.n; ++t) {
    const BufRsrc rx = buf_rsrc(a.x + (size_t)t * H + (size_t)wv * Q, 4u * (uint32_t)Q);
    uint4 xv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xv[2 * i] = buf_load16(rx, 32u * (uint32_t)(lane + 64 * i));
      xv[2 * i + 1] = buf_load16(rx, 32u * (uint32_t)(lane + 64 * i) + 16u);
    }
    float acc = 0.0f, aabs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
      const uint32_t xd[8] = {xv[2 * i].x,     xv[2 * i].y,     xv[2 * i].z,     xv[2 * i].w,
                              xv[2 * i + 1].x, xv[2 * i + 1].y, xv[2 * i + 1].z, xv[2 * i + 1].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float p0 = u2f(wd[d] << 16) * u2f(xd[2 * d]);
        const float p1 = u2f(wd[d] & 0xFFFF0000u) * u2f(xd[2 * d + 1]);
        acc += p0;
        acc += p1;
        aabs += fabsf(p0);
        aabs += fabsf(p1);
      }
    }
    acc = wave_sum(acc);
    aabs = wave_sum(aabs);
    if (t == 0) libm_table_store(s_tab, tabv);
    if (lane == 0) {
      s_part[2 * wv] = acc;
      s_part[2 * wv + 1] = aabs;
    }
    __syncthreads();
    if (tid == 0) {
      const float z = ((s_part[0] + s_part[2]) + s_part[4]) + s_part[6];
      const float zs = ((s_part[1] + s_part[3]) + s_part[5]) + s_part[7];
      const size_t o = (size_t)t * a.E + e;
      a.ch[o] = sqrt_softplus(z, s_tab) + (a.bias ? a.bias[e] : 0.0f);
      a.zabs[o] = zs;
      a.za[o] = z;
    }
    __syncthreads();  // s_part is reused by the next token
  }
}

// quant_fp8_act (src/dsv4/dsv4_ops.c:96-121) of one 128-group per wave, for
// the routed experts' gate/up tiles.
__device__ __forceinline__ void dec_quant_block(const DecArgs &a, int b) {
  const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int H = a.H, gpt = H / 128, gi = b * 4 + wv;
  if (gi >= a.n * gpt) return;
  const int t = gi / gpt, g = gi % gpt;
  const float *xr = a.x + (size_t)t * H + g * 128;
  const float v0 = xr[lane], v1 = xr[lane + 64];
  const float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  const float scale = act_scale(amax);
  const float inv = 1.0f / scale;
  uint8_t *q = a.qx8 + (size_t)t * H + g * 128;
  q[lane] = (uint8_t)e4m3_code(quant_e4m3(v0, inv));
  q[lane + 64] = (uint8_t)e4m3_code(quant_e4m3(v1, inv));
  if (lane == 0) a.qxs[(size_t)t * gpt + g] = scale;
}

// Shared expert gate/up, rows [r0, r0 + 8) of both, from the quantised x
// (E4M3 codes and per-128 scales, loaded ahead of the weights, decoded into
// LDS padded to 132 per group): t = silu(bf16 gate) * bf16 up for the 8 rows
// (src/dsv4/dsv4_model.c:6264-6268) into the shared slot of sv.
__device__ __forceinline__ void dec_shared_gateup(const DecArgs &a, int t, int tile, float *lds,
                                                  float *s_y, uint64_t *s_tab) {
  const int tid = threadIdx.x;
  {
    // the shared expert's weight stream starts 2 us into the kernel: at
    // launch the routed path's critical loads (the candidates' choices, the
    // chains' staging) are served about twice as fast by an otherwise idle
    // memory system, and the shared expert is needed only by k_dec_down
    const long long t0 = wall_clock64();  // 100 MHz
    while (wall_clock64() - t0 < 200) __builtin_amdgcn_s_sleep(8);
  }
  const int H = a.H, I = a.I, r0 = tile * (FP8_TR / 2);
  // the activation codes (at most 8192: 8 words per thread) and its
  // per-128 scales ahead of the weights
  const BufRsrc rq = buf_rsrc(a.qx8 + (size_t)t * H, (uint32_t)H);
  const BufRsrc rqs = buf_rsrc(a.qxs + (size_t)t * (H / 128), (uint32_t)(H / 128) * 4u);
  uint32_t xr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xr[j] = buf_load4(rq, 4u * (tid + 256 * j));
  const float qsv = buf_loadf(rqs, 4u * tid);
  __builtin_amdgcn_sched_barrier(0);  // issued before the weights
  Fp8Regs R;
  fp8_pair_load(R, a.sh[0], a.sh_s[0], a.sh[1], a.sh_s[1], H, I, r0);
  const uint64_t tabv = libm_table_load();
  float *xs = lds, *qs = lds + (H / 128) * 132;
  float2 *ps = reinterpret_cast<float2 *>(qs + ((H / 128 + 3) & ~3));
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = 4 * (tid + 256 * j);
    if (i < H) {
      const float2 lo = fp8x2<false>(xr[j]), hi = fp8x2<true>(xr[j]);
      *reinterpret_cast<float4 *>(xs + (i / 128) * 132 + (i % 128)) =
          make_float4(lo.x, lo.y, hi.x, hi.y);
    }
  }
  if (tid < H / 128) qs[tid] = qsv;
  __syncthreads();
  fp8_pair_finish(R, s_y, xs, qs, a.sh[0], a.sh_s[0], a.sh[1], a.sh_s[1], H, I, r0, ps);
  libm_table_store(s_tab, tabv);
  __syncthreads();
  if (tid < FP8_TR / 2 && r0 + tid < I)
    a.sv[((size_t)t * (a.E + 1) + a.E) * I + r0 + tid] =
        swiglu_t(s_y[tid], s_y[tid + FP8_TR / 2], a.limit, s_tab);
}

// Blocks: [E router logits][quant of x].
__global__ __launch_bounds__(256) void k_dec_router(DecArgs a) {
  __shared__ uint64_t s_tab[32];
  __shared__ float s_part[8];
  if ((int)blockIdx.x < a.E) return dec_logit_block(a, blockIdx.x, s_part, s_tab);
  dec_quant_block(a, blockIdx.x - a.E);
}

// ------------------------------------------------------------ chains ----
// Exact logits of candidate positions c, c + maxc, ... of token t: the whole
// block stages x and the candidate's gate row (widened to fp32) into LDS in
// one shot, then lane 0 of wave 0 runs the reference's fmaf chain in column
// order (dsv4_gemv_bf16, src/dsv4/dsv4_model.c:298-303) from LDS alone.
// The chain workgroup of position 0 publishes the candidates (and, in fast
// mode, the routing); the last chain workgroup of the token selects the
// routes.
__device__ __forceinline__ void dec_chain_block(const DecArgs &a, int t, int c, float *lds,
                                                uint64_t *s_tab, int *s_cand, int *s_nc,
                                                int *s_flag) {
  const int tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
  const int H = a.H;
  float *xs = lds, *gs = lds + H;  // H floats each
  const uint64_t tabv = libm_table_load();
  // x is issued before the candidates are known
  const BufRsrc rx = buf_rsrc(a.x + (size_t)t * H, 4u * (uint32_t)H);
  uint4 xv[8];  // H <= 8192: 8 pieces per thread
#pragma unroll
  for (int j = 0; j < 8; ++j) xv[j] = buf_load16(rx, 16u * (uint32_t)(tid + 256 * j));
  libm_table_store(s_tab, tabv);
  if (wv == 0) {
    __builtin_amdgcn_wave_barrier();  // the table, for the publishing fast path
    const int n = dec_candidates(a, t, s_cand, c == 0, s_tab);
    if (lane == 0) *s_nc = n;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (4 * (tid + 256 * j) < H) reinterpret_cast<uint4 *>(xs)[tid + 256 * j] = xv[j];
  __syncthreads();
  const int nc = *s_nc;
  if (a.fast && nc == a.K) return;  // routed by the publishing workgroup already
  for (int pos = c; pos < nc; pos += a.maxc) {
    const int e = s_cand[pos];
    const bool ok = e >= 0 && e < a.E;
    const float be = ok && a.bias ? a.bias[e] : 0.0f;  // in flight during the chain
    float acc = 0.0f;
    if (ok) {
      const BufRsrc rg = buf_rsrc(a.gate + (size_t)e * H, 2u * (uint32_t)H);
      uint4 gv[4];  // H / 8 <= 1024 pieces: 4 per thread
#pragma unroll
      for (int j = 0; j < 4; ++j) gv[j] = buf_load16(rg, 16u * (uint32_t)(tid + 256 * j));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = tid + 256 * j;
        if (8 * i < H) {
          float4 *gp = reinterpret_cast<float4 *>(gs) + 2 * i;
          gp[0] = make_float4(u2f(gv[j].x << 16), u2f(gv[j].x & 0xFFFF0000u),
                              u2f(gv[j].y << 16), u2f(gv[j].y & 0xFFFF0000u));
          gp[1] = make_float4(u2f(gv[j].z << 16), u2f(gv[j].z & 0xFFFF0000u),
                              u2f(gv[j].w << 16), u2f(gv[j].w & 0xFFFF0000u));
        }
      }
      __syncthreads();
      if (wv == 0 && lane == 0) {
        __builtin_amdgcn_s_setprio(3);
        const float4 *g = reinterpret_cast<const float4 *>(gs);
        const float4 *x = reinterpret_cast<const float4 *>(xs);
        if (H % 256 == 0)
          for (int cc = 0; cc < H / 4; cc += 64) acc = chain_cols<32>(g + cc, x + cc, acc);
        else
          for (int cc = 0; cc < H / 4; cc += 32) acc = chain_cols<16>(g + cc, x + cc, acc);
        __builtin_amdgcn_s_setprio(0);
      }
      __syncthreads();  // the next candidate restages the gate row
    }
    if (tid == 0) {
      // the reference's score and choice (src/dsv4/dsv4_model.c:5827-5831,
      // 6627-6634), here so that the selection after the hand-off only reads
      const float sc = ok ? sqrt_softplus(acc, s_tab) : 0.0f;
      a.zx[(size_t)t * a.E + pos] = sc;
      a.zc[(size_t)t * a.E + pos] = sc + be;
    }
  }
  if (!dec_arrive_last(&a.ctl[1 + t], (unsigned)a.maxc, s_flag)) return;
  // the candidates are this workgroup's own (LDS); nc > 256 uses lds
  // (2 nc floats) for the scores, past the x and gate rows no longer needed
  if (wv == 0) dec_select(a, t, nc, s_cand, lds);
  if (tid == 0) a.ctl[1 + t] = 0u;
}

// --------------------------------------------------------- gate / up ----
// Routed gate/up item j of token t: candidate position c = j / gu_tiles, rows
// [r0, r0 + tr / 2) of its gate and up matrices (tile j % gu_tiles). Loads
// the activation codes and the pair into R; an item past the end (or a
// malformed tid2eid entry) loads zero-length ranges, which read zeros without
// touching memory, so every load is issued unconditionally.
__device__ __forceinline__ void dec_gu_load(const DecArgs &a, Fp4RegsT<DEC_NP> &R, int t, int j,
                                            int nitems, const int *s_cand, const Fp4Geom &q,
                                            int &c, int &r0, bool &live) {
  const int H = a.H, I = a.I;
  c = j / a.gu_tiles;
  r0 = (j - c * a.gu_tiles) * (q.tr / 2);
  const int e = __builtin_amdgcn_readfirstlane(j < nitems ? s_cand[min(c, a.E - 1)] : -1);
  live = e >= 0 && e < a.E;
  const uint8_t *W0, *S0, *W1, *S1;
  expert_mat(a, live ? e : 0, 0, W0, S0);
  expert_mat(a, live ? e : 0, 1, W1, S1);
  fp4_tile_x(R, a.qx8 + (size_t)t * H, a.qxs + (size_t)t * (H / 128), q);
  fp4_pair_load_near(R, W0, S0, W1, S1, H, live ? I : 0, r0, q);  // S1 after S0 in the slot
}

// The item's group chains, then t = silu(bf16 gate) * bf16 up for its rows
// (src/dsv4/dsv4_model.c:6264-6268) into the candidate's slot of sv.
__device__ __forceinline__ void dec_gu_finish(const DecArgs &a, const Fp4RegsT<DEC_NP> &R, int t,
                                              int c, int r0, const Fp4Geom &q, float *lds,
                                              float *s_y, const uint64_t *s_tab) {
  const int tid = threadIdx.x, I = a.I, half = q.tr / 2;
  fp4_pair_finish(R, s_y, I, r0, q, reinterpret_cast<float2 *>(lds), fp4_scale_lds(lds, q));
  __syncthreads();
  if (tid < half && r0 + tid < I)
    a.sv[((size_t)t * (a.E + 1) + c) * I + r0 + tid] =
        swiglu_t(s_y[tid], s_y[tid + half], a.limit, s_tab);
}

// Persistent routed gate/up of token t, workgroup bb of gu_nb: items
// bb, bb + nb, ... of the token's ncand * gu_tiles, in two register tiles
// used in turn: the next item's loads are issued before an item is computed,
// so weights stream while the workgroup computes.
__device__ __forceinline__ void dec_gu_routed(const DecArgs &a, int t, int bb, float *lds,
                                              float *s_y, uint64_t *s_tab, int *s_cand,
                                              int *s_nc) {
  const int tid = threadIdx.x;
  const Fp4Geom q = fp4_geom_np(a.H, DEC_NP);
  const uint64_t tabv = libm_table_load();
  if (tid < 64) {
    const int n = dec_candidates(a, t, s_cand, false, s_tab);
    if (tid == 0) *s_nc = n;
  }
  libm_table_store(s_tab, tabv);
  __syncthreads();
  const int nitems = __builtin_amdgcn_readfirstlane(*s_nc) * a.gu_tiles;
  const int nb = a.gu_nb;
  if (bb >= nitems) return;
  if (!a.fast) {
    // exact mode: the chains bound the kernel and this stream has slack; it
    // starts 1 us later so that the chains' gate rows are staged first
    const long long t0 = wall_clock64();  // 100 MHz
    while (wall_clock64() - t0 < 100) __builtin_amdgcn_s_sleep(8);
  }
  // two register tiles used in turn, unrolled over the first four items (a
  // loop would carry loads in flight across its back edge, which the
  // compiler drains); more items (many candidates) run one at a time
  Fp4RegsT<DEC_NP> A, B;
  int cA, rA, cB, rB;
  bool lA, lB;
  int j = bb;
  dec_gu_load(a, A, t, j, nitems, s_cand, q, cA, rA, lA);
  dec_gu_load(a, B, t, j + nb, nitems, s_cand, q, cB, rB, lB);
  if (lA) dec_gu_finish(a, A, t, cA, rA, q, lds, s_y, s_tab);
  j += nb;
  dec_gu_load(a, A, t, j + nb, nitems, s_cand, q, cA, rA, lA);
  if (j < nitems && lB) dec_gu_finish(a, B, t, cB, rB, q, lds, s_y, s_tab);
  j += nb;
  dec_gu_load(a, B, t, j + nb, nitems, s_cand, q, cB, rB, lB);
  if (j < nitems && lA) dec_gu_finish(a, A, t, cA, rA, q, lds, s_y, s_tab);
  j += nb;
  if (j < nitems && lB) dec_gu_finish(a, B, t, cB, rB, q, lds, s_y, s_tab);
  for (j += nb; j < nitems; j += nb) {
    dec_gu_load(a, A, t, j, nitems, s_cand, q, cA, rA, lA);
    if (lA) dec_gu_finish(a, A, t, cA, rA, q, lds, s_y, s_tab);
  }
}

// Blocks: [n*maxc chain workgroups][n*gu_nb persistent routed FP4
// workgroups][n*(I/8) shared FP8 gate/up pairs]. Workgroups are dispatched in
// index order, so the small loads that gate the critical path (the
// candidates' choices, the chains' gate rows) are issued before the shared
// expert's weight stream.
__global__ __launch_bounds__(256) void k_dec_gateup(DecArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ uint64_t s_tab[32];
  __shared__ float s_y[256];
  __shared__ int s_cand[ROUTER_MAX_EXPERTS];
  __shared__ int s_nc, s_flag;
  const int I = a.I;
  const int nchain = a.n * a.maxc;
  const int t8 = (I + FP8_TR / 2 - 1) / (FP8_TR / 2);
  const int nshared = a.n * t8;
  int b = blockIdx.x;
  if (b < nchain) {
    dec_chain_block(a, b / a.maxc, b % a.maxc, lds, s_tab, s_cand, &s_nc, &s_flag);
    return;
  }
  b -= nchain;
  if (b < a.n * a.gu_nb) {
    dec_gu_routed(a, b / a.gu_nb, b % a.gu_nb, lds, s_y, s_tab, s_cand, &s_nc);
    return;
  }
  b -= a.n * a.gu_nb;
  if (b < nshared) dec_shared_gateup(a, b / t8, b % t8, lds, s_y, s_tab);
}

// -------------------------------------------------------------- down ----
// y = bf16(t * w), then per-128 E4M3 requant into LDS (all threads):
// qy[i + pad * (i / 128)], qys[i / 128] (src/dsv4/dsv4_model.c:6268-6287).
// Wave wv takes groups wv, wv + 4, ...; the t values of its first eight
// groups (all of them for inter <= 4096) are loaded ahead of the weights by
// dec_tv_load.
struct TvRegs {
  float v[16];
};

__device__ __forceinline__ void dec_tv_load(TvRegs &T, const float *tv, int I) {
  const uint32_t wv = threadIdx.x / 64, lane = threadIdx.x % 64;
  const BufRsrc r = buf_rsrc(tv, 4u * (uint32_t)I);  // groups past I / 128 read zeros
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t g = wv + 4u * j;
    T.v[2 * j] = buf_loadf(r, 4u * (g * 128u + lane));
    T.v[2 * j + 1] = buf_loadf(r, 4u * (g * 128u + 64u + lane));
  }
  // t has arrived before this workgroup's weights are requested: issued at
  // the same time, the few t lines would queue in the memory channels
  // behind the whole kernel's weight stream (about 5 us)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// CODES: qy receives E4M3 codes as bytes (the FP4 down tile), otherwise the
// grid values as floats, padded by 4 per 128 (the FP8 tile).
template <bool CODES>
__device__ void dec_requant(void *qyv, float *qys, const TvRegs &T, const float *tv, float w,
                            int I) {
  const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int g = wv + 4 * j;
    if (g >= I / 128) break;
    const int i0 = g * 128 + lane, i1 = i0 + 64;
    const float t0 = j < 8 ? T.v[(2 * j) & 15] : tv[i0];
    const float t1 = j < 8 ? T.v[(2 * j + 1) & 15] : tv[i1];
    const float y0 = bf16_round(t0 * w);
    const float y1 = bf16_round(t1 * w);
    const float amax = wave_max_dpp(fmaxf(fabsf(y0), fabsf(y1)));
    const float scale = act_scale(amax);
    const float inv = 1.0f / scale;
    if (CODES) {
      uint8_t *q = reinterpret_cast<uint8_t *>(qyv) + g * 128;
      q[lane] = (uint8_t)e4m3_code(quant_e4m3(y0, inv));
      q[lane + 64] = (uint8_t)e4m3_code(quant_e4m3(y1, inv));
    } else {
      float *q = reinterpret_cast<float *>(qyv) + g * 132;
      q[lane] = quant_e4m3(y0, inv);
      q[lane + 64] = quant_e4m3(y1, inv);
    }
    if (lane == 0) qys[g] = scale;
  }
  __syncthreads();
}

// Shared expert down, rows [16 tile, 16 tile + 16): its t (weight 1)
// requantised into LDS, then the FP8 tile into route slot K of ro.
__device__ __forceinline__ void dec_shared_down(const DecArgs &a, int t, int tile, float *lds) {
  const int H = a.H, I = a.I, K = a.K;
  const float *tv = a.sv + ((size_t)t * (a.E + 1) + a.E) * I;
  TvRegs T;
  dec_tv_load(T, tv, I);
  Fp8Regs R;
  fp8_tile_load(R, a.sh[2], a.sh_s[2], I, H, tile * FP8_TR);
  float *xs = lds, *qys = lds + (I / 128) * 132;
  float2 *ps = reinterpret_cast<float2 *>(qys + ((I / 128 + 3) & ~3));
  dec_requant<false>(xs, qys, T, tv, 1.0f, I);
  fp8_tile_finish(R, a.ro + ((size_t)t * (K + 1) + K) * H, xs, qys, a.sh[2], a.sh_s[2], I, H,
                  tile * FP8_TR, 1, ps);
}

// Blocks: [n*K*dn_tiles routed FP4 down tiles][n*(H/16) shared FP8 down].
__global__ __launch_bounds__(256) void k_dec_down(DecArgs a) {
  extern __shared__ __align__(16) float lds[];
  const int tid = threadIdx.x;
  const int H = a.H, I = a.I, K = a.K;
  const int nrouted = a.n * K * a.dn_tiles;
  int b = blockIdx.x;
  if (b < nrouted) {
    const int tile = b % a.dn_tiles;
    b /= a.dn_tiles;
    const int k = b % K, t = b / K;
    const size_t o = (size_t)t * K + k;
    const int e = a.sel_e[o], pos = a.sel_pos[o];
    const float w = a.sel_w[o];
    const Fp4Geom q = fp4_geom_np(I, DEC_NP);
    const int r0 = tile * q.tr;
    float *ro = a.ro + ((size_t)t * (K + 1) + k) * H;
    if (e < 0 || e >= a.E) {  // no expert: the route adds zeros
      for (int r = r0 + tid; r < min(H, r0 + q.tr); r += 256) ro[r] = 0.0f;
      return;
    }
    const float *tv = a.sv + ((size_t)t * (a.E + 1) + pos) * I;
    const uint8_t *W, *S;
    expert_mat(a, e, 2, W, S);
    TvRegs T;
    dec_tv_load(T, tv, I);
    Fp4RegsT<DEC_NP> R;
    fp4_tile_load(R, W, S, I, H, r0, q);
    // E4M3 codes and scales of y, read into registers before the pairs
    // overwrite them
    uint8_t *qy8 = reinterpret_cast<uint8_t *>(lds);  // I + I/32 bytes: within the pairs
    float *qys = lds + I / 4;
    dec_requant<true>(qy8, qys, T, tv, w, I);
    fp4_tile_x_lds(R, qy8, qys, q);
    fp4_tile_finish(R, ro, H, r0, q, reinterpret_cast<float2 *>(lds), fp4_scale_lds(lds, q));
    return;
  }
  b -= nrouted;
  const int t16 = (H + FP8_TR - 1) / FP8_TR;
  dec_shared_down(a, b / t16, b % t16, lds);
}

// out[t][i] = bf16(((0 + ro[t][0][i]) + ... + ro[t][K-1][i]) + ro[t][K][i]):
// routes in ascending expert id, then the shared expert
// (src/dsv4/dsv4_model.c:6795-6805).
__global__ __launch_bounds__(256) void k_dec_combine(DecArgs a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n * a.H) return;
  const int t = i / a.H, c = i % a.H;
  const float *r = a.ro + (size_t)t * (a.K + 1) * a.H + c;
  float acc = 0.0f;
  for (int k = 0; k < a.K; ++k) acc += r[(size_t)k * a.H];
  acc += r[(size_t)a.K * a.H];
  a.out[i] = bf16_round(acc);
}

__global__ void k_fill_zero_u32(unsigned *p, size_t n) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace dsv4

// ============================================================ C-ABI =====
using namespace dsv4;

namespace {

struct DecWs {
  unsigned *ctl;
  uint8_t *qx8;
  float *qxs, *ch, *zabs, *za, *zx, *zc, *sel_w, *sv, *ro;
  int *cand, *ncand, *sel_e, *sel_pos;
  size_t bytes;
};

int dec_maxc(const DSV4GLayer *L) {
  int m = L->topk + 10;
  if (m < 16) m = 16;
  return m < L->n_experts ? m : L->n_experts;
}

// The control words come first (offset 0 for every layer shape), then the
// rest, each piece 256-byte aligned.
DecWs dec_ws_layout(const DSV4GLayer *L, int n_tokens, void *base) {
  const size_t n = (size_t)n_tokens, K = (size_t)L->topk, E = (size_t)L->n_experts;
  const size_t H = (size_t)L->hidden, I = (size_t)L->inter;
  DecWs w = {};
  uintptr_t p = (uintptr_t)base;
  auto take = [&](size_t bytes) {
    void *r = (void *)p;
    p += (bytes + 255) & ~(size_t)255;
    return r;
  };
  w.ctl = (unsigned *)take(DEC_CTL_BYTES);
  w.qx8 = (uint8_t *)take(n * H);
  w.qxs = (float *)take(n * (H / 128) * 4);
  w.ch = (float *)take(n * E * 4);
  w.zabs = (float *)take(n * E * 4);
  w.za = (float *)take(n * E * 4);
  w.cand = (int *)take(n * E * 4);
  w.ncand = (int *)take(n * 4);
  w.zx = (float *)take(n * E * 4);
  w.zc = (float *)take(n * E * 4);
  w.sel_e = (int *)take(n * K * 4);
  w.sel_w = (float *)take(n * K * 4);
  w.sel_pos = (int *)take(n * K * 4);
  w.sv = (float *)take(n * (E + 1) * I * 4);
  w.ro = (float *)take(n * (K + 1) * H * 4);
  w.bytes = (size_t)(p - (uintptr_t)base);
  return w;
}

size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

// Workgroups of k_dec_gateup resident at once on the current device (its
// occupancy times the CU count), cached per device and LDS size.
int gateup_slots(size_t lds, int *slots) {
  static int cache_slots[64];
  static size_t cache_lds[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return dsv4g_fail(DSV4G_EHIP, "moe_decode: hipGetDevice failed");
  if (dev < 64 && cache_slots[dev] > 0 && cache_lds[dev] == lds) {
    *slots = cache_slots[dev];
    return DSV4G_OK;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_dec_gateup, 256, lds) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return dsv4g_fail(DSV4G_EHIP, "moe_decode: occupancy query failed");
  *slots = max(1, per_cu) * max(1, cus);
  if (dev < 64) {
    cache_lds[dev] = lds;
    cache_slots[dev] = *slots;
  }
  return DSV4G_OK;
}

int dec_launch(int phase, float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
               int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
               float *wt_out, hipStream_t st, int fast) {
  DSV4G_TRY(dsv4g_layer_ok(L, "moe_decode"));
  if (n_tokens <= 0) return dsv4g_fail(DSV4G_EINVAL, "moe_decode: n_tokens must be > 0");
  if (L->tid2eid && !token_ids)
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: hash layer needs token_ids");
  if (((uintptr_t)workspace & 255) || ((uintptr_t)x & 15) || ((uintptr_t)out & 15))
    return dsv4g_fail(DSV4G_EINVAL,
                      "moe_decode: workspace must be 256-byte aligned, x and out 16-byte aligned");
  const DecWs w = dec_ws_layout(L, n_tokens, workspace);
  if (!workspace || workspace_bytes < w.bytes)
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: workspace too small (%zu < %zu)",
                      workspace_bytes, w.bytes);
  DecArgs a = {};
  a.x = x;
  a.out = out;
  a.gate = L->gate_w;
  a.bias = L->bias;
  a.tid2eid = L->tid2eid;
  a.token_ids = token_ids;
  a.experts = L->experts;
  a.expert_stride = L->expert_stride;
  a.scale_run = L->scale_run;
  a.sh[0] = L->sh1;
  a.sh[1] = L->sh3;
  a.sh[2] = L->sh2;
  a.sh_s[0] = L->sh1_s;
  a.sh_s[1] = L->sh3_s;
  a.sh_s[2] = L->sh2_s;
  a.ctl = w.ctl;
  a.qx8 = w.qx8;
  a.qxs = w.qxs;
  a.ch = w.ch;
  a.zabs = w.zabs;
  a.za = w.za;
  a.cand = w.cand;
  a.ncand = w.ncand;
  a.zx = w.zx;
  a.zc = w.zc;
  a.sel_e = w.sel_e;
  a.sel_w = w.sel_w;
  a.sel_pos = w.sel_pos;
  a.sv = w.sv;
  a.ro = w.ro;
  a.idx_out = idx_out;
  a.wt_out = wt_out;
  a.n = n_tokens;
  a.H = L->hidden;
  a.I = L->inter;
  a.E = L->n_experts;
  a.K = L->topk;
  a.maxc = dec_maxc(L);
  const Fp4Geom qg = fp4_geom_np(a.H, DEC_NP), qd = fp4_geom_np(a.I, DEC_NP);
  a.gu_tiles = (a.I + qg.tr / 2 - 1) / (qg.tr / 2);
  a.dn_tiles = (a.H + qd.tr - 1) / qd.tr;

  a.route_scale = L->route_scale;
  {
    const double d = dec_par_depth(a.H) * 0x1p-24, h = a.H * 0x1p-24;
    a.gamma = (float)(d / (1.0 - d) + h / (1.0 - h));
  }
  a.limit = (float)(int)L->swiglu_limit;  // the reference passes the limit as int
  a.fast = fast;
  const int n = n_tokens, H = a.H, I = a.I;
  if (n > DEC_CTL_BYTES / 4 - 1)
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: at most %d tokens per call",
                      DEC_CTL_BYTES / 4 - 1);
  const size_t lds_fp8_gu = (size_t)(H / 128) * 132 * 4 + (size_t)((H / 128 + 3) & ~3) * 4 +
                            (size_t)FP8_TR * pair_stride(H / 128) * 8;
  const size_t lds_fp8_dn = (size_t)(I / 128) * 132 * 4 + (size_t)((I / 128 + 3) & ~3) * 4 +
                            (size_t)FP8_TR * pair_stride(I / 128) * 8;
  if (phase == 0) {
    const int blocks = a.E + (n * (H / 128) + 3) / 4;
    hipLaunchKernelGGL(k_dec_router, dim3(blocks), dim3(256), 0, st, a);
    return dsv4g_check_launch("dec_router");
  }
  if (phase == 1) {
    // routed pairs: the tile's pairs and scales; chains: x and a gate row
    const size_t lds_fp4 = (size_t)qg.tr * pair_stride(qg.G) * 8 + 4096;
    const size_t lds = max_sz(max_sz(lds_fp4, (size_t)H * 8), lds_fp8_gu);
    // persistent routed workgroups: the resident slots left beside the chain
    // and shared workgroups, split over the tokens (at least 128 each)
    const int fixed = n * (a.maxc + (I + FP8_TR / 2 - 1) / (FP8_TR / 2));
    int slots = 0;
    DSV4G_TRY(gateup_slots(lds, &slots));
    a.gu_nb = max(128, (slots - fixed) / n);
    const long blocks = (long)fixed + (long)n * a.gu_nb;
    hipLaunchKernelGGL(k_dec_gateup, dim3((unsigned)blocks), dim3(256), lds, st, a);
    return dsv4g_check_launch("dec_gateup");
  }
  if (phase == 2) {
    const size_t lds = max_sz(max_sz((size_t)qd.tr * pair_stride(qd.G) * 8 + 4096,
                                     (size_t)I + (size_t)I / 32 + 64),
                              lds_fp8_dn);
    const long blocks = (long)n * a.K * a.dn_tiles + (long)n * ((H + FP8_TR - 1) / FP8_TR);
    hipLaunchKernelGGL(k_dec_down, dim3((unsigned)blocks), dim3(256), lds, st, a);
    return dsv4g_check_launch("dec_down");
  }
  if (phase == 3) {
    hipLaunchKernelGGL(k_dec_combine, dim3((unsigned)((n * H + 255) / 256)), dim3(256), 0, st, a);
    return dsv4g_check_launch("dec_combine");
  }
  return dsv4g_fail(DSV4G_EINVAL, "moe_decode: bad phase %d", phase);
}

// The no-allocation entry's workspace: one array per device, held until the
// process ends. In host code `scratch` names a host-side stand-in, not device
// memory: kernels and fills take the device address that hipGetSymbolAddress
// returns for the current device, kept in g_scratch_ptr.
#define DEC_SCRATCH_BYTES ((size_t)16 << 20)
static __device__ __align__(256) uint8_t scratch[DEC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void *g_scratch_ptr[64];

// The current device's scratch address, resolved once per device. Device
// globals start zeroed when the code object loads; a first call that is not
// being captured also clears the control words with the fill kernel (no
// memset: the call may be captured into a graph).
int scratch_ptr(hipStream_t st, void **out) {
  int dev = 0;
  DSV4G_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return dsv4g_fail(DSV4G_EINVAL, "moe_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return dsv4g_fail(DSV4G_EHIP, "moe_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                        hipGetErrorString(e));
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    DSV4G_HIP(hipStreamIsCapturing(st, &cs));
    if (cs == hipStreamCaptureStatusNone) {
      const size_t words = DEC_CTL_BYTES / 4;
      hipLaunchKernelGGL(k_fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                         st, (unsigned *)p, words);
      DSV4G_TRY(dsv4g_check_launch("moe_noalloc_init"));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

size_t dsv4g_moe_workspace_bytes(const DSV4GLayer *L, int n_tokens) {
  return dec_ws_layout(L, n_tokens, nullptr).bytes;
}

int dsv4g_moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
  if (!workspace || ((uintptr_t)workspace & 255) || workspace_bytes < DEC_CTL_BYTES)
    return dsv4g_fail(DSV4G_EINVAL, "moe_workspace_init: bad workspace");
  const size_t words = workspace_bytes / 4;
  hipLaunchKernelGGL(k_fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (unsigned *)workspace, words);
  return dsv4g_check_launch("moe_workspace_init");
}

int dsv4g_moe_decode_phase(int phase, float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, void *stream) {
  const int fast = (phase & DSV4G_DECODE_FAST) != 0;
  return dec_launch(phase & ~DSV4G_DECODE_FAST, out, x, L, token_ids, n_tokens, workspace,
                    workspace_bytes, nullptr, nullptr, (hipStream_t)stream, fast);
}

int dsv4g_moe_decode_routing(int *idx_out, float *wt_out, const DSV4GLayer *L, int n_tokens,
                             void *workspace, void *stream) {
  const DecWs w = dec_ws_layout(L, n_tokens, workspace);
  hipStream_t st = (hipStream_t)stream;
  if (idx_out)
    DSV4G_HIP(hipMemcpyAsync(idx_out, w.sel_e, (size_t)n_tokens * L->topk * sizeof(int),
                             hipMemcpyDeviceToDevice, st));
  if (wt_out)
    DSV4G_HIP(hipMemcpyAsync(wt_out, w.sel_w, (size_t)n_tokens * L->topk * sizeof(float),
                             hipMemcpyDeviceToDevice, st));
  return 0;
}

int dsv4g_moe_forward(float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
                      int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
                      float *wt_out, void *stream) {
  for (int phase = 0; phase < 4; ++phase)
    DSV4G_TRY(dec_launch(phase, out, x, L, token_ids, n_tokens, workspace, workspace_bytes,
                         idx_out, wt_out, (hipStream_t)stream, 0));
  return 0;
}

int dsv4g_moe_forward_fast(float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, int *idx_out, float *wt_out, void *stream) {
  for (int phase = 0; phase < 4; ++phase)
    DSV4G_TRY(dec_launch(phase, out, x, L, token_ids, n_tokens, workspace, workspace_bytes,
                         idx_out, wt_out, (hipStream_t)stream, 1));
  return 0;
}

}  // extern "C"

extern "C" int dsv4g_moe_forward_noalloc(float *out, const float *x, const DSV4GLayer *L,
                                         const int *token_ids, int n_tokens, int *idx_out,
                                         float *wt_out, void *stream) {
  DSV4G_TRY(dsv4g_layer_ok(L, "moe_noalloc"));
  if (n_tokens <= 0) return dsv4g_fail(DSV4G_EINVAL, "moe_noalloc: n_tokens must be > 0");
  const size_t need = dsv4g_moe_workspace_bytes(L, n_tokens);
  if (need > DEC_SCRATCH_BYTES)
    return dsv4g_fail(DSV4G_EINVAL,
                      "moe_noalloc: %d tokens of this layer need %zu bytes of workspace, more "
                      "than the %zu bytes of the library's scratch; pass fewer tokens per call",
                      n_tokens, need, DEC_SCRATCH_BYTES);
  void *ws = nullptr;
  DSV4G_TRY(scratch_ptr((hipStream_t)stream, &ws));
  return dsv4g_moe_forward(out, x, L, token_ids, n_tokens, ws, need, idx_out, wt_out, stream);
}
