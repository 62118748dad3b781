// dsv4_decode.hip - the decode MoE layer on gfx950: moe_forward
// (src/dsv4/dsv4_model.c:6599-6807) for a few tokens, bit for bit, as three
// kernels per layer (workgroups are dispatched in index order; a wait inside
// a launch only ever holds a workgroup whose producers were dispatched
// before it and never wait on it):
//
//   k_dec_route    E router workgroups (expert e: the approximate logits z
//                  and sum|w*x| of every token and the approximate choice
//                  sqrt_softplus(z) + bias, published as self-marked 64-bit
//                  records); the shared FP8 expert's gate/up tiles (tile 0
//                  also writes the token's E4M3 activation codes); last, one
//                  candidate workgroup per token, which waits for the
//                  records and writes the token's candidate list (below).
//   k_dec_front    chain workgroups, a few per token: for the candidate
//                  positions c, c + maxc, ... the reference's exact
//                  sequential logit chain (dsv4_gemv_bf16,
//                  src/dsv4/dsv4_model.c:298-303); the last of them waits
//                  for the others and takes the exact top-k and route
//                  weights (src/dsv4/dsv4_model.c:6615-6676). Then the
//                  streaming workgroups: one register tile at a time, the
//                  FP4 gate/up items of the candidates, t = silu(bf16 gate)
//                  * bf16 up into the candidate's slot
//                  (src/dsv4/dsv4_model.c:6264-6268), then the shared
//                  expert's down rows.
//   k_dec_back     one requant workgroup per route first: y = bf16(t * w)
//                  and the per-128 E4M3 requant
//                  (src/dsv4/dsv4_model.c:6239-6287), published as codes and
//                  a flag; then one workgroup per 8 output rows: the FP4 down
//                  rows of every route (issued before the wait for the
//                  codes), then the routes in ascending expert id and the
//                  shared expert, rounded to BF16
//                  (src/dsv4/dsv4_model.c:6795-6805).
//
// Memory round trips that one launch's workgroups need before their weights
// can stream (the candidates, the route ids) are cut to one each: under the
// weight stream every dependent round trip queues behind the whole stream.
//
// Candidates. A parallel logit differs from the sequential fmaf chain by at
// most gamma_d + gamma_H times sum|w*x| (d: the parallel sum's rounding
// depth, dec_par_depth). Mapped through |d score / dz| <= 1/2 plus slack for
// the score's own rounding, and doubled for both sides, that gives delta: an
// expert whose approximate choice is below (k-th best approximate choice) -
// delta has k experts surely above it and cannot be selected. The others are
// the candidates, in ascending expert id; gate/up runs for every candidate
// while their exact chains run. Near-ties (a constant gate) only make more
// candidates: more chains in parallel and more gate/up items.
//
// Hand-offs inside a launch. On this part every XCD has its own L2, and a
// device-scope release fence writes back a whole L2; atomics on one address
// from many workgroups are serialised at about 170 ns each, and under full
// memory traffic every dependent round trip costs microseconds. So data that
// crosses workgroups inside a launch is stored and loaded with agent-scope
// relaxed atomics (write-through stores, loads of the coherent copy: ld_dev /
// st_dev) and is either self-marked (the router records: one 64-bit store
// carries the value and its mark, polled directly) or followed by a flag,
// one word per producer on a line of its own: a producer waits for its own
// stores (vmcnt), then sets its flag; the waiter polls all the flags with
// one wave. Every wait is bounded: one that runs out sets a sticky error
// word (dsv4g_moe_decode_status) and the workgroup leaves, so a broken
// hand-off ends as an error, never as a hang. Records and flags live in the
// workspace, zero before the first call (dsv4g_moe_workspace_init); every
// call leaves them zero. Data that crosses the launch boundary uses plain
// loads and stores.
#include <mutex>
#include <type_traits>

#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"
#include "dsv4_tiles.h"

namespace dsv4 {

#define DEC_CTL_BYTES 4096  // control words
#define DEC_NP 8            // passes per FP4 gate/up tile
// control word indices
#define DEC_ERR 0   // sticky error bits (DEC_ERR_*)
#define DEC_FS 16   // words between two producer flags (one 64-byte line each)
#define DEC_MAX_TOKENS 1020
#define DEC_ERR_TIMEOUT 1u
// polls of a wait before it gives up (each at least one memory round trip,
// about a microsecond: on the order of a second)
#define DEC_SPIN_LIMIT (1u << 20)
#define DB_RC 6  // routes per chunk of k_dec_back
#define DEC_PHASES 3  // launches per layer: route, front, back
// set in the high word of a router record once it is written (the low 31
// bits hold sum|w*x|, whose sign bit is always clear)
#define DEC_REC_SET 0x80000000u

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
  unsigned *ctl;  // control words (DEC_*)
  // per-token pieces of the workspace: token t's piece is tb bytes past
  // token 0's (dec_tok)
  uint64_t *rec;   // [E] router record: choice | (sum|w*x| + DEC_REC_SET) << 32
  uint64_t *zrec;  // [E] router logit z | DEC_REC_SET << 32
  unsigned *cf;    // [E] exact chain done flags per candidate position
  uint32_t *qc;    // [K][I/4] E4M3 codes of the requantised routes
  float *qcs;      // [K][I/128] their scales
  uint8_t *xq;     // [H] E4M3 codes of the token's activation (route launch)
  float *xqs;      // [H/128] their per-128 scales
  float *zx, *zc;  // [E] exact score sqrt_softplus(z) and choice score + bias per
                   // candidate position
  unsigned *qf;    // [K] route requant done flags (DEC_FS apart)
  int *cl;         // [1 + E + K] the candidates (route launch): count, ids, then the
                   // K best approximate choices in selection order
  int *sel_e;      // [K] routing, ascending id (moe_forward's idx)
  int *sel_pos;    // [K] candidate position of each route
  float *sel_w;    // [K] route weights (moe_forward's wt)
  float *sv;       // [E + 1][I] SwiGLU t per candidate position; slot E = shared
  float *ro;       // [H] the shared expert's down output (fp32)
  size_t tb;       // bytes between two tokens' pieces
  float *route_out;                // optional [n][K + 1][H]: route outputs before BF16
  int *idx_out;                    // optional copies of the routing
  float *wt_out;
  int n, H, I, E, K;
  int gu_tiles;    // paired gate/up tiles (rows I, in H)
  int maxc;        // chain workgroups per token
  int n_stream;    // streaming workgroups
  float route_scale, limit;
  float gamma;  // gamma_{dec_par_depth(H)} + gamma_H, the candidates' bound factor
  int fast;     // routing from the parallel logits when the candidates are exactly top-k
};

// Token t's piece of a per-token workspace array.
// (Byte-pointer arithmetic, not an integer round trip: the compiler then
// still sees a pointer into device memory and emits global loads and
// stores, not FLAT ones, whose pending state makes it drain every load.)
template <typename T>
__device__ __forceinline__ T *dec_tok(T *p, const DecArgs &a, int t) {
  using B = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T *>(reinterpret_cast<B *>(p) + (size_t)t * a.tb);
}

// ------------------------------------------------- agent-scope hand-off ----
// Through global-address-space pointers (every hand-off word lives in device
// memory): a generic pointer would make these FLAT operations, and one FLAT
// operation in flight makes the compiler wait for every load of the wave
// before any later use (it cannot order FLAT against other loads).
template <typename T>
__device__ __forceinline__ T ld_dev(const T *p) {
  return __hip_atomic_load((__attribute__((address_space(1))) T *)(const_cast<T *>(p)),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_dev(T *p, T v) {
  __hip_atomic_store((__attribute__((address_space(1))) T *)p, v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Sets the calling workgroup's flag once every thread's agent-scope stores
// are complete.
__device__ __forceinline__ void dec_signal(unsigned *flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) st_dev(flag, 1u);
}

// Raises the sticky error bit (the calling wave's lane 0).
__device__ __forceinline__ void dec_fail(unsigned *ctl) {
  if (threadIdx.x % 64 == 0)
    __hip_atomic_fetch_or(ctl + DEC_ERR, DEC_ERR_TIMEOUT, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
}

// Ends one poll of a bounded wait: false once the wait has run out or another
// workgroup has reported an error (the error word is then set), else a short
// sleep before the next poll (the calling wave).
__device__ __forceinline__ bool dec_spin(unsigned it, unsigned *ctl) {
  if (it >= DEC_SPIN_LIMIT || ((it & 63u) == 63u && ld_dev(ctl + DEC_ERR) != 0u)) {
    dec_fail(ctl);
    return false;
  }
  __builtin_amdgcn_s_sleep(2);
  return true;
}

// Waits (wave 0 polls, the others at the barrier) until flag f[i * stride] is
// set for every i < count with use(i) (use: nullptr = all); false if the wait
// ran out or another workgroup reported an error.
__device__ __forceinline__ bool dec_wait_flags(const unsigned *f, int count, int stride,
                                               const int *use, unsigned *ctl, int *s_i) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int ok = 1;
    for (unsigned it = 0;; ++it) {
      int mine = 1;
      for (int i = lane; i < count; i += 64)
        if (!use || use[i]) mine &= ld_dev(f + (size_t)i * stride) != 0u;
      if (__all(mine)) break;
      if (!dec_spin(it, ctl)) {
        ok = 0;
        break;
      }
    }
    if (lane == 0) *s_i = ok;
  }
  __syncthreads();
  return *s_i != 0;
}

// Expert e's matrix m (0 gate w1, 1 up w3, 2 down w2) in the reference slot
// layout [s1 | s2 | s3 | w1 | w2 | w3] (src/dsv4/dsv4_model.c:6298-6305).
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

// Rounding depth of a parallel logit of dec_router_block: the product (one
// rounding), a lane's sequential sum of its 8-column pieces (at most
// 8 ceil(H / 2048) products), the 6-level wave butterfly, the 3 additions of
// the four waves' partials, and one more for the rounding of the computed
// sum|w*x| that the bound is scaled by.
__device__ __host__ __forceinline__ int dec_par_depth(int H) { return 8 * ((H / 4 + 511) / 512) + 11; }

// ------------------------------------------------------- activation ----
// quant_fp8_act (src/dsv4/dsv4_ops.c:96-121) of 16 consecutive values v of a
// token row, columns [base, base + 16), into LDS: E4M3 codes into q8 (H
// bytes) and/or grid values into xf (padded to 132 floats per 128-group),
// the per-128 scale into qs. A group's 8 threads are neighbouring lanes of
// one wave (all threads of the wave call it; base past H stores nothing).
__device__ __forceinline__ void dec_quant16(const float (&v)[16], int base, int H, uint8_t *q8,
                                            float *xf, float *qs) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  m = fmaxf(m, __shfl_xor(m, 4, 64));
  if (base < H) {
    const float scale = act_scale(m);
    const float inv = 1.0f / scale;
    float g[16];
    uint32_t k[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) g[i] = quant_e4m3_code(v[i], inv, k[i]);
    if (q8) {
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        c[i] = k[4 * i] | (k[4 * i + 1] << 8) | (k[4 * i + 2] << 16) | (k[4 * i + 3] << 24);
      *reinterpret_cast<uint4 *>(q8 + base) = make_uint4(c[0], c[1], c[2], c[3]);
    }
    if (xf) {
      float *d = xf + (base / 128) * 132 + base % 128;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4 *>(d + 4 * i) =
            make_float4(g[4 * i], g[4 * i + 1], g[4 * i + 2], g[4 * i + 3]);
    }
    if ((threadIdx.x & 7) == 0) qs[base / 128] = scale;
  }
}

// Thread i's 16 values of token row xt (columns 16 i .. 16 i + 15; zeros past
// H), for rows of at most 4096: loaded once, at the start of a workgroup,
// before any weight load, so that they return first (loads complete in
// order) and the quantisation never waits on a memory round trip under the
// weight stream.
struct XRegs {
  uint4 v[4];
};
__device__ __forceinline__ void dec_x_load(XRegs &X, const float *xt, int H) {
  const BufRsrc rx = buf_rsrc(xt, H <= 4096 ? 4u * (uint32_t)H : 0u);
#pragma unroll
  for (int i = 0; i < 4; ++i) X.v[i] = buf_load16(rx, 4u * (uint32_t)(16 * threadIdx.x + 4 * i));
}
__device__ __forceinline__ void dec_quant_regs(const XRegs &X, int H, uint8_t *q8, float *xf,
                                               float *qs) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[4 * i] = u2f(X.v[i].x);
    v[4 * i + 1] = u2f(X.v[i].y);
    v[4 * i + 2] = u2f(X.v[i].z);
    v[4 * i + 3] = u2f(X.v[i].w);
  }
  dec_quant16(v, 16 * threadIdx.x, H, q8, xf, qs);
}

// The same straight from memory, for any row width (all threads).
__device__ __forceinline__ void dec_quant_x(const float *xt, int H, uint8_t *q8, float *xf,
                                            float *qs) {
  const int tid = threadIdx.x;
  const BufRsrc rx = buf_rsrc(xt, 4u * (uint32_t)H);
  const int span = (H + 4095) / 4096 * 4096;  // wave-uniform trip count
  for (int base = 16 * tid; base < span; base += 4096) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 u = buf_load16(rx, 4u * (uint32_t)(base + 4 * i));  // past H: zeros
      v[4 * i] = u2f(u.x);
      v[4 * i + 1] = u2f(u.y);
      v[4 * i + 2] = u2f(u.z);
      v[4 * i + 3] = u2f(u.w);
    }
    dec_quant16(v, base, H, q8, xf, qs);
  }
}

// Token 0's quantised activation: from X when it holds the row (H <= 4096),
// else loaded.
__device__ __forceinline__ void dec_quant_t0(const DecArgs &a, const XRegs &X, uint8_t *q8,
                                             float *xf, float *qs) {
  if (a.H <= 4096)
    dec_quant_regs(X, a.H, q8, xf, qs);
  else
    dec_quant_x(a.x, a.H, q8, xf, qs);
}

// Token t's activation codes and per-128 scales (written by the route launch)
// into LDS (all threads; read after the caller's next barrier).
__device__ __forceinline__ void dec_x_codes(const DecArgs &a, int t, uint8_t *q8, float *qs) {
  const int H = a.H;
  const uint4 *gq = reinterpret_cast<const uint4 *>(dec_tok(a.xq, a, t));
  const float *gs = dec_tok(a.xqs, a, t);
  for (int i = threadIdx.x; i < H / 16; i += 256) reinterpret_cast<uint4 *>(q8)[i] = gq[i];
  for (int i = threadIdx.x; i < (H + 127) / 128; i += 256) qs[i] = gs[i];
}

// ------------------------------------------------------------ routing ----
// Route weights from the unbiased scores, summed in selection order, then the
// routes sorted by id (src/dsv4/dsv4_model.c:6650-6674; equal ids carry
// equal weights, so any order among them matches the exchange sort). Lane k
// holds route k in selection order (whole wave).
__device__ __forceinline__ void dec_select_finish(const DecArgs &a, int t, int my_e, float my_sc,
                                                  int my_pos) {
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
    dec_tok(a.sel_e, a, t)[rank] = my_e;
    dec_tok(a.sel_w, a, t)[rank] = my_w;
    dec_tok(a.sel_pos, a, t)[rank] = my_pos >= 0 ? my_pos : rank;  // candidates == routes
    const size_t o = (size_t)t * K + rank;
    if (a.idx_out) a.idx_out[o] = my_e;
    if (a.wt_out) a.wt_out[o] = my_w;
  }
}

// Candidates of token t (one whole wave), from the router records: ct[0, nc)
// the candidate ids in ascending order, sel[0, K) the K best approximate
// choices in selection order (-1 past the selectable experts), both in LDS.
// Returns nc, or -1 if the wait for the records ran out. Every workgroup that
// calls it for a token derives the same candidates from the same records.
// The records come from the previous launch (k_dec_route), so plain cached
// loads see them (agent-scope loads of 256 records by every workgroup cost
// microseconds of fabric round trips); the mark check stays as a bounded
// guard. NPER = experts per lane (E <= 64 * NPER).
template <int NPER, bool COH>
__device__ __forceinline__ int dec_candidates_t(const DecArgs &a, int t, int *ct, int *sel) {
  const int lane = threadIdx.x % 64;
  const float ninf = -__builtin_inff();
  const uint64_t *rec = dec_tok(a.rec, a, t);
  float v[NPER];
  float amax;
  for (unsigned it = 0;; ++it) {  // until every record carries its mark
    uint64_t r[NPER];
    int ready = 1;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
      const int e = lane + 64 * j;
      r[j] = e < a.E ? (COH ? ld_dev(rec + e) : rec[e]) : ((uint64_t)DEC_REC_SET << 32);
    }
    amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NPER; ++j) {
      const float c = __uint_as_float((uint32_t)r[j]);
      const bool in = lane + 64 * j < a.E;
      ready &= (int)(r[j] >> 63);
      v[j] = (in && c == c) ? c : ninf;  // a NaN choice never wins a strict '>'
      if (in) amax = fmaxf(amax, __uint_as_float((uint32_t)(r[j] >> 32) & ~DEC_REC_SET));
    }
    if (__all(ready)) break;
    if (!dec_spin(it, a.ctl)) return -1;
  }
  // k-th best approximate choice: k times remove one instance of the
  // maximum
  if (lane < a.K) sel[lane] = -1;
  float kth = ninf;
  unsigned used = 0u;
  for (int k = 0; k < a.K; ++k) {
    float m = ninf;
    int mj = -1;
#pragma unroll
    for (int j = 0; j < NPER; ++j)
      if (!((used >> j) & 1u) && v[j] > m) {
        m = v[j];
        mj = j;
      }
    const float wm = wave_max_dpp(m);
    const unsigned long long bal = __ballot(mj >= 0 && m == wm);
    if (bal == 0ull) {  // fewer than k selectable experts
      kth = ninf;
      break;
    }
    const int wl = __builtin_ctzll(bal);
    if (lane == wl) {
      used |= 1u << mj;
      sel[k] = wl + 64 * mj;
    }
    kth = wm;
  }
  const float sum_abs = wave_max_dpp(amax);
  const float bound_z = a.gamma * sum_abs;
  const float thr = cand_threshold(kth, 2.0f * (0.5f * bound_z + 1e-5f));
  int base = 0;
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int e = lane + 64 * j;
    const bool p = e < a.E && v[j] >= thr;
    const unsigned long long bal = __ballot(p);
    if (p) ct[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
    base += __popcll(bal);
  }
  return base;
}

// The same for more than 256 experts, with the choices in LDS (v: E floats)
// and plain loops over a lane's experts e = lane + 64 j in ascending j, so
// that every step takes the same expert as dec_candidates_t; a taken expert
// is marked -inf in v (no strict '>' takes it again) and set back to the
// k-th best choice afterwards (it is a candidate either way).
template <bool COH>
__device__ __forceinline__ int dec_candidates_lds(const DecArgs &a, int t, int *ct, int *sel,
                                               float *v) {
  const int lane = threadIdx.x % 64;
  const float ninf = -__builtin_inff();
  const uint64_t *rec = dec_tok(a.rec, a, t);
  float amax;
  for (unsigned it = 0;; ++it) {  // until every record carries its mark
    int ready = 1;
    amax = 0.0f;
    for (int e = lane; e < a.E; e += 64) {
      const uint64_t r = COH ? ld_dev(rec + e) : rec[e];
      const float c = __uint_as_float((uint32_t)r);
      ready &= (int)(r >> 63);
      v[e] = c == c ? c : ninf;
      amax = fmaxf(amax, __uint_as_float((uint32_t)(r >> 32) & ~DEC_REC_SET));
    }
    if (__all(ready)) break;
    if (!dec_spin(it, a.ctl)) return -1;
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < a.K) sel[lane] = -1;
  float kth = ninf;
  for (int k = 0; k < a.K; ++k) {
    float m = ninf;
    int me = -1;
    for (int e = lane; e < a.E; e += 64)
      if (v[e] > m) {
        m = v[e];
        me = e;
      }
    const float wm = wave_max_dpp(m);
    const unsigned long long bal = __ballot(me >= 0 && m == wm);
    if (bal == 0ull) {
      kth = ninf;
      break;
    }
    const int wl = __builtin_ctzll(bal);
    __builtin_amdgcn_wave_barrier();
    if (lane == wl) {
      v[me] = ninf;
      sel[k] = me;
    }
    __builtin_amdgcn_wave_barrier();
    kth = wm;
  }
  if (lane < a.K && sel[lane] >= 0) v[sel[lane]] = kth;
  __builtin_amdgcn_wave_barrier();
  const float sum_abs = wave_max_dpp(amax);
  const float thr = cand_threshold(kth, 2.0f * (0.5f * (a.gamma * sum_abs) + 1e-5f));
  int base = 0;
  for (int e0 = 0; e0 < a.E; e0 += 64) {
    const int e = e0 + lane;
    const bool p = e < a.E && v[e] >= thr;
    const unsigned long long bal = __ballot(p);
    if (p) ct[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
    base += __popcll(bal);
  }
  return base;
}

// The candidates of token t into LDS (ct, nc, and sel: the selection order of
// the approximate top-k; a hash layer: the tid2eid row, K positions), wave 0
// deriving them while the others wait (s_v: E floats of LDS for more than 256
// experts). Returns nc (all threads), -1 if the wait for the router records
// ran out.
template <bool COH>
__device__ __forceinline__ int dec_candidates(const DecArgs &a, int t, int *ct, int *sel,
                                              float *s_v, int *s_i) {
  __syncthreads();  // ct, sel and s_i of the previous token have been read
  if (threadIdx.x < 64) {
    int nc;
    if (a.tid2eid) {
      const int lane = threadIdx.x;
      const int64_t *row = a.tid2eid + (size_t)a.token_ids[t] * a.K;
      if (lane < a.K) ct[lane] = sel[lane] = (int)row[lane];
      nc = a.K;
    } else if (a.E <= 64) {
      nc = dec_candidates_t<1, COH>(a, t, ct, sel);
    } else if (a.E <= 128) {
      nc = dec_candidates_t<2, COH>(a, t, ct, sel);
    } else if (a.E <= 256) {
      nc = dec_candidates_t<4, COH>(a, t, ct, sel);
    } else {
      nc = dec_candidates_lds<COH>(a, t, ct, sel, s_v);
    }
    if (threadIdx.x == 0) *s_i = nc;
  }
  __syncthreads();
  return *s_i;
}

// Candidate workgroup of token t in the route launch (dispatched after every
// router workgroup, whose records it waits for: coherent loads, since they
// are written in this launch): the candidates, once, into the token's list
// for the next launch, whose workgroups read it in one memory round trip
// instead of each deriving it from the 256 records (about 4 us of every
// front workgroup's start, with no weight in flight). A wait that runs out
// writes a count of -1.
__device__ __forceinline__ void dec_cand_block(const DecArgs &a, int t, float *lds) {
  int *ct = reinterpret_cast<int *>(lds), *sel = ct + ROUTER_MAX_EXPERTS;
  float *sv = reinterpret_cast<float *>(sel + 32);
  int *si = reinterpret_cast<int *>(sv + ROUTER_MAX_EXPERTS);
  const int nc = dec_candidates<true>(a, t, ct, sel, sv, si);
  int *cl = dec_tok(a.cl, a, t);
  if (threadIdx.x == 0) cl[0] = nc;
  for (int i = threadIdx.x; i < nc; i += 256) cl[1 + i] = ct[i];
  if (threadIdx.x < a.K) cl[1 + a.E + threadIdx.x] = sel[threadIdx.x];
}

// The token's candidates from the route launch's list into LDS (all
// threads): ct[0, nc) the candidate ids in ascending order, sel[0, K) the K
// best approximate choices in selection order; returns nc (-1: the route
// launch's wait ran out). Every entry is loaded at once (entries past nc
// unused), one memory round trip.
__device__ __forceinline__ int dec_candidates_read(const DecArgs &a, int t, int *ct, int *sel,
                                                   int *s_i) {
  __syncthreads();  // ct, sel and s_i of the previous token have been read
  const int *cl = dec_tok(a.cl, a, t);
  const int tid = threadIdx.x, E = a.E;
  int v[ROUTER_MAX_EXPERTS / 256];
#pragma unroll
  for (int j = 0; j < ROUTER_MAX_EXPERTS / 256; ++j)
    v[j] = tid + 256 * j < E ? cl[1 + tid + 256 * j] : 0;
  const int sv = tid < a.K ? cl[1 + E + tid] : 0;
  const int nc = tid == 0 ? cl[0] : 0;
#pragma unroll
  for (int j = 0; j < ROUTER_MAX_EXPERTS / 256; ++j)
    if (tid + 256 * j < E) ct[tid + 256 * j] = v[j];
  if (tid < a.K) sel[tid] = sv;
  if (tid == 0) *s_i = nc;
  __syncthreads();
  return *s_i;
}

// Whether the exact chains route token t: not in fast mode when the
// candidates are exactly the top-k, nor for a hash row in fast mode or
// without a valid entry (all threads; ct from dec_candidates).
__device__ __forceinline__ bool dec_need_chain(const DecArgs &a, int nc, const int *ct) {
  if (!a.tid2eid) return !(a.fast && nc == a.K);
  if (a.fast) return false;
  for (int p = 0; p < a.K; ++p)
    if (ct[p] >= 0 && ct[p] < a.E) return true;
  return false;
}

// Routing of a token that needs no chain (wave 0): fast mode: the approximate
// top-k in selection order, weighted from the parallel logits; a hash row:
// the tid2eid row, weighted from the parallel logits in fast mode, else
// (no valid entry) with weights 0. False if the wait for the logits ran out.
__device__ __forceinline__ bool dec_route_direct(const DecArgs &a, int t, const int *sel,
                                                 const uint64_t *tab) {
  const int lane = threadIdx.x % 64;
  const int e = lane < a.K ? sel[lane] : -1;
  const bool ok = e >= 0 && e < a.E;
  const bool use = a.fast && ok;
  const uint64_t *zr = dec_tok(a.zrec, a, t) + (use ? e : 0);
  uint64_t r = (uint64_t)DEC_REC_SET << 32;
  for (unsigned it = 0;; ++it) {
    if (use) r = *zr;
    if (__all((int)(r >> 63))) break;
    if (!dec_spin(it, a.ctl)) return false;
  }
  const float sc = use ? sqrt_softplus(__uint_as_float((uint32_t)r), tab) : 0.0f;
  dec_select_finish(a, t, e, sc, a.tid2eid ? lane : -1);
  return true;
}

// Exact top-k of token t from the candidates' exact scores and choices (one
// whole wave; the nc candidates ct in ascending id, from the caller's LDS):
// routes ascending by id with weights and candidate positions
// (src/dsv4/dsv4_model.c:6615-6676). Lane k carries route k in selection
// order.
template <int NPER>
__device__ __forceinline__ void dec_select_t(const DecArgs &a, int t, int nc, const int *ct) {
  const int lane = threadIdx.x % 64;
  const int K = a.K;
  const float *zt = dec_tok(a.zx, a, t), *zc = dec_tok(a.zc, a, t);
  int my_e = -1, my_pos = -1;
  float my_sc = 0.0f;
  if (a.tid2eid) {
    if (lane < K) {
      my_e = ct[lane];
      my_pos = lane;
      my_sc = (my_e >= 0 && my_e < a.E) ? ld_dev(zt + lane) : 0.0f;
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
        sc[j] = ld_dev(zt + pos);
        chv[j] = ld_dev(zc + pos);
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

// More than 256 candidates (near-ties or large expert counts): scores in
// LDS (2 * nc floats, nc <= 1024), scanned with plain loops.
__device__ __forceinline__ void dec_select_big(const DecArgs &a, int t, int nc, const int *ct,
                                               float *lds) {
  const int lane = threadIdx.x % 64;
  const float *zt = dec_tok(a.zx, a, t), *zc = dec_tok(a.zc, a, t);
  const float ninf = -__builtin_inff();
  float *sc = lds, *chv = lds + nc;
  for (int pos = lane; pos < nc; pos += 64) {
    sc[pos] = ld_dev(zt + pos);
    chv[pos] = ld_dev(zc + pos);
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
// Router workgroup of expert e: wave wv takes the columns [wv H/4,
// (wv + 1) H/4), lane l its 8-column pieces l, l + 64, ... (gate row and x
// read directly); for every token the approximate choice sqrt_softplus(z) +
// bias with sum|w*x| (rounding depth: dec_par_depth) and z, each published as
// one 64-bit record that carries its own DEC_REC_SET mark. Workgroup 0 also
// clears the previous call's requant flags.
__device__ __forceinline__ void dec_router_block(const DecArgs &a, int e, uint64_t tabv,
                                                 uint64_t *s_tab, float *s_part) {
  const int tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
  const int H = a.H, Q = H / 4;
  if (e == 0)
    for (int i = tid; i < a.n * a.K; i += 256)
      stg(dec_tok(a.qf, a, i / a.K) + (size_t)(i % a.K) * DEC_FS, 0u);
  const BufRsrc rg = buf_rsrc(a.gate + (size_t)e * H + (size_t)wv * Q, 2u * (uint32_t)Q);
  uint4 w[4];  // Q <= 2048: at most 4 pieces per lane; pieces past Q read zeros
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = buf_load16(rg, 16u * (uint32_t)(lane + 64 * i));
  const float be = a.bias ? a.bias[e] : 0.0f;
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
      const float c = sqrt_softplus(z, s_tab) + be;
      st_dev(dec_tok(a.zrec, a, t) + e, (uint64_t)__float_as_uint(z) | ((uint64_t)DEC_REC_SET << 32));
      st_dev(dec_tok(a.rec, a, t) + e,
             (uint64_t)__float_as_uint(c) | ((uint64_t)(__float_as_uint(zs) | DEC_REC_SET) << 32));
    }
    __syncthreads();  // s_part is reused by the next token
  }
}

// ------------------------------------------------------------ chains ----
// The exact logit z = ((0 + g0 x0) + g1 x1) + ... (one fmaf per column,
// dsv4_gemv_bf16's order, src/dsv4/dsv4_model.c:298-303) is a 4096-step
// dependent chain, about 20 us under the weight stream. When every product g[c] x[c] is exact in fp32 (BF16 gate
// times the BF16-valued activation: at most 16 significant bits; checked per
// column as fmaf(g, x, -p) == 0), each step is acc = fl(acc + p[c]), so the
// chain can be cut:
//  * the prefix sums P_b (fp32 partial sums: only a guess) locate, near H/4,
//    H/2 and 3H/4, the boundary b where |P_b| is largest (there the fp32
//    running sum s_b has the coarsest spacing, so it lies fewest floats from
//    fl(P_b); sampled over random gates and activations: within 75 floats,
//    mostly a few);
//  * wave 0 runs the first segment from +0; wave k runs segment k from the
//    64 consecutive floats around the guess of P_b (lane j: 32 below to 31
//    above), all in parallel;
//  * the true start of segment k is the end of segment k - 1 from its true
//    start: one lane of wave k started there (bit-equal), and its end is
//    the true end; otherwise segment k runs again from the true start.
// Every step is the reference's own addition in the reference's order, so
// the result is the sequential chain's, bit for bit, however good the
// guesses. Needs H a multiple of 256, at least 1024; gs (fp32 gate row) is
// overwritten with the products.
#define SPLIT_SEGS 4
struct SplitLds {
  float wtot[4];                        // per-wave sums
  unsigned long long key[SPLIT_SEGS];   // per window: |P_b| bits, then ~b
  int b[SPLIT_SEGS + 1];                // segment boundaries
  float p0[SPLIT_SEGS];                 // the guess of P_b at each boundary
  float st[SPLIT_SEGS][64], en[SPLIT_SEGS][64];  // starts and ends per lane
  int exact;
};

__device__ __forceinline__ int ord_f(float f) {
  const int b = (int)f2u(f);
  return b >= 0 ? b : -(b & 0x7FFFFFFF);
}
__device__ __forceinline__ float ord_inv(int o) {
  return o >= 0 ? u2f((uint32_t)o) : u2f((uint32_t)(-o) | 0x80000000u);
}

// acc + p[lo] + ... + p[hi - 1] in order (fp32 adds; p in LDS, read as a
// broadcast by every lane). The main loop takes 64 columns an iteration in two
// halves of 8 float4 reads, each half's reads issued a half ahead, with no
// condition on a read: the last reads may pass hi by up to 64 floats, which
// stay inside the workgroup's LDS (the callers' arrays past p), and are not
// added.
__device__ __forceinline__ float split_run(const float *p, int lo, int hi, float acc) {
  int c = lo;
  for (; c < hi && (c & 3); ++c) acc = acc + p[c];
  const float4 *q = reinterpret_cast<const float4 *>(p + c);
  const int nb = (hi - c) / 64;  // whole 64-column iterations
  float4 ra[8], rb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) ra[k] = q[k];
  for (int it = 0; it < nb; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) rb[k] = q[16 * it + 8 + k];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      acc = acc + ra[k].x;
      acc = acc + ra[k].y;
      acc = acc + ra[k].z;
      acc = acc + ra[k].w;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) ra[k] = q[16 * it + 16 + k];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      acc = acc + rb[k].x;
      acc = acc + rb[k].y;
      acc = acc + rb[k].z;
      acc = acc + rb[k].w;
    }
  }
  for (c += 64 * nb; c < hi; ++c) acc = acc + p[c];
  return acc;
}

// z in wave 0 (the other waves return an unspecified value), or false in
// *ok when a product is inexact (then nothing is computed and the caller
// runs the fmaf chain).
__device__ __forceinline__ float dec_chain_split(float *gs, const float *xs, int H, SplitLds *L,
                                                 bool *ok) {
  const int tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
  const int npt = H / 256, c0 = tid * npt, seg = H / SPLIT_SEGS;
  if (tid == 0) L->exact = 1;
  if (tid < SPLIT_SEGS) L->key[tid] = 0ull;
  __syncthreads();
  // products in place, their exactness, and the thread's sum
  float tsum = 0.0f;
  int ex = 1;
  for (int i = 0; i < npt; ++i) {
    const float g = gs[c0 + i], x = xs[c0 + i];
    const float pr = g * x;
    ex &= fmaf(g, x, -pr) == 0.0f;
    gs[c0 + i] = pr;
    tsum += pr;
  }
  if (!__all(ex) && lane == 0) L->exact = 0;
  // exclusive prefix of the thread sums (wave scan, then the wave sums)
  float inc = tsum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(inc, o, 64);
    if (lane >= o) inc += u;
  }
  if (lane == 63) L->wtot[wv] = inc;
  __syncthreads();
  *ok = L->exact != 0;
  if (!*ok) return 0.0f;
  float pre = inc - tsum;
  for (int w = 0; w < wv; ++w) pre += L->wtot[w];
  // the window [nom - wd, nom + wd] around boundary k's nominal column nom
  // (wd <= seg / 4 and npt <= seg / 4: only the window nearest c0 can meet a
  // thread's columns): the column b with the largest |P_b|, lowest b on
  // ties, by a 64-bit LDS max over (|P_b| bits, ~b)
  const int wd = min(128, H / 16);
  const int k = (c0 + seg / 2) / seg, nom = k * seg;
  float pb = 0.0f;
  unsigned long long best = 0ull;
  if (k >= 1 && k < SPLIT_SEGS && c0 <= nom + wd && c0 + npt > nom - wd) {
    float run = pre;
    for (int i = 0; i < npt; ++i) {
      const int c = c0 + i;  // run = P_c
      if (c >= nom - wd && c <= nom + wd) {
        const unsigned long long key =
            ((unsigned long long)f2u(fabsf(run)) << 32) | (uint32_t)~(uint32_t)c;
        if (key > best) {
          best = key;
          pb = run;
        }
      }
      run += gs[c];
    }
    if (best) atomicMax(&L->key[k], best);
  }
  if (tid == 0) {
    L->b[0] = 0;
    L->b[SPLIT_SEGS] = H;
    L->p0[0] = 0.0f;
  }
  __syncthreads();
  if (best && L->key[k] == best) {  // this thread holds the boundary
    L->b[k] = (int)~(uint32_t)best;
    L->p0[k] = pb;
  }
  __syncthreads();
  // the segments, all at once: wave k takes segment k
  if (wv < SPLIT_SEGS) {
    const float st = wv == 0 ? 0.0f : ord_inv(ord_f(L->p0[wv]) + lane - 32);
    const float en = split_run(gs, L->b[wv], L->b[wv + 1], st);
    L->st[wv][lane] = st;
    L->en[wv][lane] = en;
  }
  __syncthreads();
  // the true chain through the segments (wave 0, from LDS)
  float cur = 0.0f;
  if (wv == 0) {
    cur = L->en[0][0];
    for (int s = 1; s < SPLIT_SEGS; ++s) {
      const unsigned long long m = __ballot(f2u(L->st[s][lane]) == f2u(cur));
      if (m)
        cur = L->en[s][__builtin_ctzll(m)];
      else  // not covered: the segment again from the true start
        cur = split_run(gs, L->b[s], L->b[s + 1], cur);
    }
  }
  return cur;
}

// Exact logits of candidate positions c, c + maxc, ... of token t: x and the
// candidate's gate row widened to fp32 in LDS, then lane 0 of wave 0 runs
// the reference's fmaf chain in column order (dsv4_gemv_bf16,
// src/dsv4/dsv4_model.c:298-303); the score and choice go to the position,
// then its flag. The token's last chain workgroup (dispatched after the
// others, so its wait cannot hold a slot they need) then waits for every
// chain of the token, clears the flags and selects the routes; for a token
// that needs no chain it routes directly (dec_route_direct).
__device__ __forceinline__ void dec_chain_block(const DecArgs &a, int t, int c, float *lds,
                                                uint64_t *s_tab, int *s_cand, int *s_sel,
                                                int *s_i) {
  const int tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
  const int H = a.H;
  float *xs = lds, *gs = lds + H;
  // the split chain's scratch, past x, the gate row and the E choices
  SplitLds *sl = reinterpret_cast<SplitLds *>(lds + 2 * H + ((a.E + 3) & ~3));
  const uint64_t tabv = libm_table_load();
  // x is staged before the candidates are known
  const BufRsrc rx = buf_rsrc(a.x + (size_t)t * H, 4u * (uint32_t)H);
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // H <= 8192: 8 pieces per thread
    const uint32_t i4 = (uint32_t)(tid + 256 * j);
    if (4u * i4 < (uint32_t)H) reinterpret_cast<uint4 *>(xs)[i4] = buf_load16(rx, 16u * i4);
  }
  libm_table_store(s_tab, tabv);
  const int nc = dec_candidates_read(a, t, s_cand, s_sel, s_i);
  if (nc < 0) return;
  if (!dec_need_chain(a, nc, s_cand)) {
    if (c == a.maxc - 1 && wv == 0) dec_route_direct(a, t, s_sel, s_tab);
    return;
  }
  for (int pos = c; pos < nc; pos += a.maxc) {
    const int e = s_cand[pos];
    if (e < 0 || e >= a.E) continue;  // a malformed tid2eid entry has no chain
    const float be = a.bias ? a.bias[e] : 0.0f;
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
    bool split = false;
    float zsplit = 0.0f;
    if (H % 256 == 0 && H >= 1024) {
      // the token's critical path: ahead of the streaming workgroups' VALU
      // work on the SIMD
      __builtin_amdgcn_s_setprio(3);
      zsplit = dec_chain_split(gs, xs, H, sl, &split);
      __builtin_amdgcn_s_setprio(0);
    }
    if (wv == 0 && lane == 0) {
      float acc = zsplit;
      if (!split) {
        __builtin_amdgcn_s_setprio(3);
        acc = 0.0f;
        const float4 *g = reinterpret_cast<const float4 *>(gs);
        const float4 *x = reinterpret_cast<const float4 *>(xs);
        if (H % 256 == 0)
          for (int cc = 0; cc < H / 4; cc += 64) acc = chain_cols<32>(g + cc, x + cc, acc);
        else
          for (int cc = 0; cc < H / 4; cc += 32) acc = chain_cols<16>(g + cc, x + cc, acc);
        __builtin_amdgcn_s_setprio(0);
      }
      // the reference's score and choice (src/dsv4/dsv4_model.c:5827-5831,
      // 6627-6634)
      const float sc = sqrt_softplus(acc, s_tab);
      st_dev(dec_tok(a.zx, a, t) + pos, sc);
      st_dev(dec_tok(a.zc, a, t) + pos, sc + be);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the scores before the flag
      st_dev(dec_tok(a.cf, a, t) + pos, 1u);
    }
    __syncthreads();  // the next candidate restages the gate row
  }
  if (c != a.maxc - 1) return;
  // the selector: every position with an expert in range has a chain
  int *use = reinterpret_cast<int *>(lds + 2 * H);  // nc ints
  for (int p = tid; p < nc; p += 256) use[p] = s_cand[p] >= 0 && s_cand[p] < a.E;
  __syncthreads();
  unsigned *cf = dec_tok(a.cf, a, t);
  if (!dec_wait_flags(cf, nc, 1, use, a.ctl, s_i)) return;
  for (int p = tid; p < nc; p += 256) st_dev(cf + p, 0u);
  // more than 256 candidates select from 2 nc floats of LDS past x and the
  // gate row
  if (wv == 0) dec_select(a, t, nc, s_cand, lds + 2 * H);
}

// ---------------------------------------------------- shared expert ----
// Rows of each shared matrix per gate/up tile: a staged FP8 tile holds
// fp8s_rows(H) / 2 rows of gate and of up, a register tile FP8_TR / 2.
__device__ __host__ __forceinline__ bool dec_sh_gu_staged(int H) {
  return fp8s_ok(H) && H >= 1024 && H <= 4096;
}
__device__ __host__ __forceinline__ int dec_sh_gu_rows(int H) {
  return dec_sh_gu_staged(H) ? fp8s_rows(H) / 2 : FP8_TR / 2;
}
__device__ __host__ __forceinline__ int dec_sh_dn_rows(int I) {
  return fp8s_ok(I) ? fp8s_rows(I) : FP8_TR;
}

// Shared expert gate/up tile `tile` of token t (rows [r0, r0 + dec_sh_gu_rows)
// of both matrices), from the quantised x (quant_fp8_act,
// src/dsv4/dsv4_model.c:5580-5606; grid values in LDS, padded to 132 per
// group): t for its rows into the shared slot of sv (read by the next
// launch). Tile 0 also writes the token's activation codes and per-128
// scales (xq, xqs) for the next launch's routed items. ST (dec_sh_gu_staged(H)): the token's x row and the weights come
// by direct-to-LDS loads, x first, so the quantisation runs while the
// weights stream; otherwise a register tile, and x loaded here.
template <bool ST>
__device__ __forceinline__ void dec_shared_gu(const DecArgs &a, int t, int tile, float *lds,
                                              float *s_y, uint64_t *s_tab) {
  const int tid = threadIdx.x;
  const int H = a.H, I = a.I, hr = dec_sh_gu_rows(H), r0 = tile * hr;
  const uint64_t tabv = libm_table_load();
  if (ST) {
    // [32 KB tile][x: H raw floats, then 132 floats per group][scales]
    // [pairs]; the scale codes in s_y (free until the rows are chained), so
    // that three workgroups fit a CU's LDS. Every load below is a
    // direct-to-LDS load the compiler does not track, so its only wait (for
    // tabv) comes after fp8s_wait().
    uint8_t *tl = reinterpret_cast<uint8_t *>(lds);
    float *xs = lds + 8192, *qs = xs + (H / 128) * 132;
    float2 *ps = reinterpret_cast<float2 *>(qs + ((H / 128 + 3) & ~3));
    uint32_t *codes = reinterpret_cast<uint32_t *>(s_y);
    fp8s_code_dma(codes, a.sh_s[0], a.sh_s[1], H, I, r0, true);
    {
      // the row: H / 256 pieces of 1 KB, a quarter per wave
      const int l = tid % 64, wv = __builtin_amdgcn_readfirstlane(tid / 64);
      const int nd = H / 1024;
      const DmaRsrc rx = dma_rsrc(a.x + (size_t)t * H, 4u * (uint32_t)H);
      const uint32_t wb = (uint32_t)(wv * nd) * 1024u;
      for (int d = 0; d < nd; ++d)
        dma_load16(rx, wb + (uint32_t)d * 1024u + 16u * (uint32_t)l,
                   lds_addr(xs) + wb + (uint32_t)d * 1024u);
    }
    fp8s_dma(tl, a.sh[0], a.sh[1], H, I, r0, true);
    vm_wait_n<8>();  // codes and x have landed (the tile's 8 loads may be in flight)
    __syncthreads();
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 f = 16 * tid < H ? reinterpret_cast<const float4 *>(xs)[4 * tid + i]
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
    __syncthreads();  // every raw value read before the padded rows overwrite them
    dec_quant16(v, 16 * tid, H, tile == 0 ? dec_tok(a.xq, a, t) : nullptr, xs, qs);
    const uint32_t code = fp8s_code(codes, H, I, r0, true);
    fp8s_wait();
    __syncthreads();  // also: every code read before s_y takes the rows
    if (tile == 0 && tid < H / 128) dec_tok(a.xqs, a, t)[tid] = qs[tid];
    libm_table_store(s_tab, tabv);
    const float y = fp8s_rows_dot(tl, xs, qs, code, H, ps);
    if (tid < 2 * hr) s_y[tid] = bf16_round(y);
  } else {
    Fp8Regs R;
    fp8_pair_load(R, a.sh[0], a.sh_s[0], a.sh[1], a.sh_s[1], H, I, r0);
    float *xs = lds, *qs = lds + (H / 128) * 132;
    float2 *ps = reinterpret_cast<float2 *>(qs + ((H / 128 + 3) & ~3));
    libm_table_store(s_tab, tabv);  // after the weight loads are issued
    dec_quant_x(a.x + (size_t)t * H, H, tile == 0 ? dec_tok(a.xq, a, t) : nullptr, xs, qs);
    __syncthreads();
    if (tile == 0)
      for (int i = tid; i < H / 128; i += 256) dec_tok(a.xqs, a, t)[i] = qs[i];
    fp8_pair_finish(R, s_y, xs, qs, a.sh[0], a.sh_s[0], a.sh[1], a.sh_s[1], H, I, r0, ps);
  }
  __syncthreads();
  if (tid < hr && r0 + tid < I)
    dec_tok(a.sv, a, t)[(size_t)a.E * I + r0 + tid] =
        swiglu_t(s_y[tid], s_y[tid + hr], a.limit, s_tab);
}

// y = bf16(t * w), then per-128 E4M3 requant into LDS (all threads):
// qy[i + pad * (i / 128)], qys[i / 128] (src/dsv4/dsv4_model.c:6268-6287).
// Wave wv takes groups wv, wv + 4, ...; t comes through agent-scope loads
// (written by other workgroups of the launch), those of the first eight
// groups (all of them for inter <= 4096) loaded together ahead.
struct TvRegs {
  float v[16];
};

__device__ __forceinline__ void dec_tv_load_dev(TvRegs &T, const float *tv, int I) {
  const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int g = wv + 4 * j;
    T.v[2 * j] = g * 128 < I ? ld_dev(tv + g * 128 + lane) : 0.0f;
    T.v[2 * j + 1] = g * 128 < I ? ld_dev(tv + g * 128 + 64 + lane) : 0.0f;
  }
}

__device__ void dec_requant_f(float *qy, float *qys, const TvRegs &T, const float *tv, float w,
                              int I) {
  const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int g = wv + 4 * j;
    if (g >= I / 128) break;
    const int i0 = g * 128 + lane, i1 = i0 + 64;
    const float t0 = j < 8 ? T.v[(2 * j) & 15] : ld_dev(tv + i0);
    const float t1 = j < 8 ? T.v[(2 * j + 1) & 15] : ld_dev(tv + i1);
    const float y0 = bf16_round(t0 * w);
    const float y1 = bf16_round(t1 * w);
    const float amax = wave_max_dpp(fmaxf(fabsf(y0), fabsf(y1)));
    const float scale = act_scale(amax);
    const float inv = 1.0f / scale;
    float *q = qy + g * 132;
    q[lane] = quant_e4m3(y0, inv);
    q[lane + 64] = quant_e4m3(y1, inv);
    if (lane == 0) qys[g] = scale;
  }
  __syncthreads();
}

// Shared expert down tile `tile` of token t (rows [r0, r0 + dec_sh_dn_rows)):
// the token's shared t (written by the route launch) is loaded first, then
// the weights, so t returns first and is requantised (weight 1) into LDS
// while the weights stream; then the FP8 rows into ro (fp32; k_dec_back
// rounds them). ST: the tile is staged (fp8s_ok(I)).
template <bool ST>
__device__ __forceinline__ void dec_shared_dn(const DecArgs &a, int t, int tile, float *lds) {
  const int H = a.H, I = a.I, nr = dec_sh_dn_rows(I), r0 = tile * nr;
  const float *tv = dec_tok(a.sv, a, t) + (size_t)a.E * I;
  if (ST) {
    // [32 KB tile][t: I raw floats, then 132 floats per group][scales]
    // [pairs][scale codes], all by direct-to-LDS loads (none the compiler
    // tracks): t and the codes first, so they land while the weights stream
    uint8_t *tl = reinterpret_cast<uint8_t *>(lds);
    float *xs = lds + 8192, *qys = xs + (I / 128) * 132;
    float2 *ps = reinterpret_cast<float2 *>(qys + ((I / 128 + 3) & ~3));
    uint32_t *codes = reinterpret_cast<uint32_t *>(ps + fp8s_rows(I) * pair_stride(I / 128));
    const int tid = threadIdx.x, l = tid % 64, wv = __builtin_amdgcn_readfirstlane(tid / 64);
    fp8s_code_dma(codes, a.sh_s[2], a.sh_s[2], I, H, r0, false);
    {
      const int nd = I / 1024;  // 1 KB pieces per wave
      const DmaRsrc rt = dma_rsrc(tv, 4u * (uint32_t)I);
      const uint32_t wb = (uint32_t)(wv * nd) * 1024u;
      for (int d = 0; d < nd; ++d)
        dma_load16(rt, wb + (uint32_t)d * 1024u + 16u * (uint32_t)l,
                   lds_addr(xs) + wb + (uint32_t)d * 1024u);
    }
    fp8s_dma(tl, a.sh[2], a.sh[2], I, H, r0, false);
    vm_wait_n<8>();  // codes and t have landed
    __syncthreads();
    // requant (weight 1, src/dsv4/dsv4_model.c:6268-6287) of the raw t in
    // place: wave w takes groups w, w + 4, ..., lane l columns l, l + 64
    float tvv[2 * 16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int g = wv + 4 * j;
      tvv[2 * j] = g * 128 < I ? xs[g * 128 + l] : 0.0f;
      tvv[2 * j + 1] = g * 128 < I ? xs[g * 128 + 64 + l] : 0.0f;
    }
    __syncthreads();  // every raw value read before the padded rows overwrite them
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int g = wv + 4 * j;
      if (g >= I / 128) break;
      const float y0 = bf16_round(tvv[2 * j]), y1 = bf16_round(tvv[2 * j + 1]);
      const float amax = wave_max_dpp(fmaxf(fabsf(y0), fabsf(y1)));
      const float scale = act_scale(amax);
      const float inv = 1.0f / scale;
      xs[g * 132 + l] = quant_e4m3(y0, inv);
      xs[g * 132 + 64 + l] = quant_e4m3(y1, inv);
      if (l == 0) qys[g] = scale;
    }
    const uint32_t code = fp8s_code(codes, I, H, r0, false);
    fp8s_wait();
    __syncthreads();
    const float v = fp8s_rows_dot(tl, xs, qys, code, I, ps);
    if (tid < nr && r0 + tid < H) dec_tok(a.ro, a, t)[r0 + tid] = v;
  } else {
    TvRegs T;
    dec_tv_load_dev(T, tv, I);
    Fp8Regs R;
    fp8_tile_load(R, a.sh[2], a.sh_s[2], I, H, r0);
    float *xs = lds, *qys = lds + (I / 128) * 132;
    float2 *ps = reinterpret_cast<float2 *>(qys + ((I / 128 + 3) & ~3));
    dec_requant_f(xs, qys, T, tv, 1.0f, I);
    fp8_tile_finish(R, dec_tok(a.ro, a, t), xs, qys, a.sh[2], a.sh_s[2], I, H, r0, 0, ps);
  }
}

// --------------------------------------------------- routed gate/up ----
// Routed gate/up item l of token t: candidate position c = l / gu_tiles, rows
// [r0, r0 + tr / 2) of its gate and up matrices (tile l % gu_tiles). An item
// past the end (or a malformed tid2eid entry) loads zero-length ranges,
// which read zeros without touching memory, so every load is issued
// unconditionally. The activation codes in R stay as set.
__device__ __forceinline__ void dec_gu_load(const DecArgs &a, Fp4RegsT<DEC_NP> &R, int l,
                                            int nitems, const int *s_cand, const Fp4Geom &q,
                                            int &c, int &r0, bool &live) {
  const int H = a.H, I = a.I;
  c = l / a.gu_tiles;
  r0 = (l - c * a.gu_tiles) * (q.tr / 2);
  const int e = __builtin_amdgcn_readfirstlane(l < nitems ? s_cand[min(c, a.E - 1)] : -1);
  live = e >= 0 && e < a.E;
  const uint8_t *W0, *S0, *W1, *S1;
  expert_mat(a, live ? e : 0, 0, W0, S0);
  expert_mat(a, live ? e : 0, 1, W1, S1);
  fp4_pair_load_near(R, W0, S0, W1, S1, H, live ? I : 0, r0, q);  // S1 after S0 in the slot
}

// Dynamic LDS of a streaming workgroup for the FP4 items: the pairs of a
// tile (tr rows, pair_stride(G) apart) and 4096 bytes of its scales, the
// token's activation codes (H bytes) and per-128 scales, then E floats for
// the candidates (dec_candidates).
struct DecLds {
  float2 *ps;
  uint8_t *cl;
  uint8_t *xq8;
  float *xqs;
  float *aux;
};

__device__ __host__ __forceinline__ size_t dec_lds_pairs(const Fp4Geom &q) {
  return (size_t)q.tr * pair_stride(q.G) * 8;
}
__device__ __host__ __forceinline__ size_t dec_lds_x(int H) {
  return ((size_t)H + (size_t)H / 32 + 15) & ~(size_t)15;
}
__device__ __host__ __forceinline__ size_t dec_lds_fp4(const Fp4Geom &q, int H, int E) {
  return dec_lds_pairs(q) + 4096 + dec_lds_x(H) + 4 * (size_t)E;
}

__device__ __forceinline__ DecLds dec_lds(float *lds, const Fp4Geom &q, int H) {
  uint8_t *b = reinterpret_cast<uint8_t *>(lds);
  const size_t P = dec_lds_pairs(q);
  DecLds L;
  L.ps = reinterpret_cast<float2 *>(b);
  L.cl = b + P;
  L.xq8 = b + P + 4096;
  L.xqs = reinterpret_cast<float *>(L.xq8 + H);
  L.aux = reinterpret_cast<float *>(L.xq8 + dec_lds_x(H));
  return L;
}

// The item's group chains over its partials (one lane per tile row,
// pair_chain, src/dsv4/dsv4_model.c:1049-1074), then t = silu(bf16 gate) *
// bf16 up for its rows (src/dsv4/dsv4_model.c:6264-6268) into candidate
// slot c of sv.
__device__ __forceinline__ void dec_gu_chain(const DecArgs &a, int t, int c, int r0,
                                             const Fp4Geom &q, const DecLds &L, float *s_y,
                                             const uint64_t *s_tab) {
  const int tid = threadIdx.x, I = a.I, half = q.tr / 2;
  // the chain lanes' wave ahead of the other waves' partials on its SIMD:
  // at the usual priority its 128 dependent steps took about 2 us
  __builtin_amdgcn_s_setprio(3);
  const float v = fp4_tile_chain(q, L.ps);
  __builtin_amdgcn_s_setprio(0);
  if (tid < q.tr) s_y[tid] = v;
  __syncthreads();
  if (tid < half && r0 + tid < I)
    dec_tok(a.sv, a, t)[(size_t)c * I + r0 + tid] =
        swiglu_t(s_y[tid], s_y[tid + half], a.limit, s_tab);
}

// Routed gate/up items l0, l0 + S, ... (below le) of token t (of nc *
// gu_tiles; nc candidates s_cand in LDS), from the token's quantised
// activation (in LDS already if have_x, else quantised here), one register
// tile at a time: a workgroup holding one tile leaves registers for more
// workgroups per CU, whose loads overlap each other's compute (measured:
// more bandwidth than two tiles in turn in fewer workgroups).
__device__ __forceinline__ void dec_routed_items(const DecArgs &a, int t, int l0, int le, int nc,
                                                 bool have_x, const DecLds &L, float *s_y,
                                                 uint64_t *s_tab, uint64_t tabv,
                                                 const int *s_cand) {
  const int H = a.H, S = a.n_stream;
  const Fp4Geom q = fp4_geom_np(H, DEC_NP);
  const int nitems = nc * a.gu_tiles;
  if (l0 >= le) return;
  if (!have_x) {
    dec_quant_x(a.x + (size_t)t * H, H, L.xq8, nullptr, L.xqs);
    __syncthreads();
  }
  Fp4RegsT<DEC_NP> A;
  fp4_tile_x_lds(A, L.xq8, L.xqs, q);  // the lane's activation group: the same for every item
  // the expf table for SwiGLU (loaded at the workgroup's start; read after
  // the first chain's barrier)
  libm_table_store(s_tab, tabv);
  // the next item's loads go out as soon as this item's partials are in LDS
  // (its weight registers are free then), so they are in flight while this
  // item's group chains and SwiGLU run
  int c, r0;
  bool live;
  dec_gu_load(a, A, l0, nitems, s_cand, q, c, r0, live);
  for (int l = l0; l < le; l += S) {
    const int cc = c, rr = r0;
    const bool lv = live;
    if (lv) fp4_tile_partials(A, a.I, rr, q, L.ps, L.cl, true);
    if (l + S < le) dec_gu_load(a, A, l + S, nitems, s_cand, q, c, r0, live);
    if (lv) dec_gu_chain(a, t, cc, rr, q, L, s_y, s_tab);
  }
  __syncthreads();  // LDS (candidates, activation) is rewritten by the next token
}

// Streaming workgroup j of n_stream (k_dec_front): first its tiles of the
// shared expert's down rows (their input, the shared t, is complete when the
// launch starts, so their loads fill the time the candidates take to
// arrive), then per token its quantised activation (codes and per-128
// scales, written by the route launch) into LDS, the candidates
// (dec_candidates_read) and its routed gate/up items. The units (a shared
// down tile: 16 FP8 rows, 32 KB; a routed item: 16 FP4 rows, 32 KB) are
// dealt round-robin over the streaming workgroups in the order [the shared
// down tiles, token 0's items, token 1's items, ...], so no workgroup has
// more than one unit above the mean. ST: the shared down tiles are staged
// (fp8s_ok(I)).
template <bool ST>
__device__ __forceinline__ void dec_stream_block(const DecArgs &a, int j, float *lds, float *s_y, uint64_t *s_tab,
                                                 uint64_t tabv, int *s_cand, int *s_sel, int *s_i) {
  const int S = a.n_stream;
  const DecLds L = dec_lds(lds, fp4_geom_np(a.H, DEC_NP), a.H);
  const int t16 = (a.H + dec_sh_dn_rows(a.I) - 1) / dec_sh_dn_rows(a.I);
  int done = a.n * t16;  // units dealt so far: the shared down tiles first
  for (int i = j; i < done; i += S) {
    __syncthreads();  // LDS of the previous unit
    dec_shared_dn<ST>(a, i / t16, i % t16, lds);
  }
  __syncthreads();  // the tiles' LDS before the activation codes take it
  for (int t = 0; t < a.n; ++t) {
    dec_x_codes(a, t, L.xq8, L.xqs);  // read after dec_candidates_read's first barrier
    const int nc = dec_candidates_read(a, t, s_cand, s_sel, s_i);
    if (nc < 0) return;
    const int nitems = nc * a.gu_tiles;
    const int l0 = (j + S - done % S) % S;
    if (l0 < nitems) dec_routed_items(a, t, l0, nitems, nc, true, L, s_y, s_tab, tabv, s_cand);
    done += nitems;
  }
}

// Route launch: blocks [E router][n * (I / rows) shared gate/up tiles]
// (768 at the model's shape: one round of resident workgroups). Router
// workgroup e: the approximate logits of expert e for every token, published
// as records (dec_router_block). Shared workgroup: one tile of the shared
// expert's gate/up for one token (tile 0 also the token's activation codes).
// Nothing here waits on another workgroup: the next launch reads both
// results. ST: dec_sh_gu_staged(H).
template <bool ST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_dec_route(
    DecArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ uint64_t s_tab[32];
  __shared__ float s_y[256];
  __shared__ float s_part[8];
  const int b = blockIdx.x;
  if (b < a.E) {
    const uint64_t tabv = libm_table_load();
    return dec_router_block(a, b, tabv, s_tab, s_part);
  }
  const int hr = dec_sh_gu_rows(a.H), t8 = (a.I + hr - 1) / hr, i = b - a.E;
  if (i >= a.n * t8) {
    if (i - a.n * t8 < a.n) dec_cand_block(a, i - a.n * t8, lds);
    return;
  }
  dec_shared_gu<ST>(a, i / t8, i % t8, lds, s_y, s_tab);
}

// Front launch: blocks [n maxc chain][n_stream streaming]. The chain
// workgroups come first, so their loads (x and the candidates' gate rows)
// are ahead of the weight streams; the token's last chain workgroup waits
// only on the token's other chain workgroups, dispatched before it. A
// streaming workgroup's first loads are token 0's activation and the expf
// table. ST: fp8s_ok(I).
template <bool ST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_dec_front(
    DecArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ uint64_t s_tab[32];
  __shared__ float s_y[256];
  __shared__ int s_cand[ROUTER_MAX_EXPERTS];
  __shared__ int s_sel[32];
  __shared__ int s_i;
  const int b = blockIdx.x;
  if (b < a.n * a.maxc)
    return dec_chain_block(a, b / a.maxc, b % a.maxc, lds, s_tab, s_cand, s_sel, &s_i);
  const int j = b - a.n * a.maxc;
  if (j >= a.n_stream) return;
  // the expf table's load goes first, but its LDS store (which waits for
  // it) only when the first routed item needs it, not ahead of the first
  // weight loads: a memory round trip at the start of every workgroup
  const uint64_t tabv = libm_table_load();
  dec_stream_block<ST>(a, j, lds, s_y, s_tab, tabv, s_cand, s_sel, &s_i);
}

// ------------------------------------------------------- down + combine ----
// E4M3 codes of four values already scaled and clamped to +-448 (quant_e4m3's
// q, src/dsv4/dsv4_model.c:5598-5604), packed little-endian: the hardware
// conversion (v_cvt_pk_fp8_f32, OCP E4M3, round to nearest even) equals
// round_e4m3's code for every |q| <= 448 of either sign except q = -0, which
// the reference codes as +0 (q + 0 gives +0 there and changes nothing
// else); checked exhaustively on the device. A NaN q takes the frexp form.
__device__ __forceinline__ uint32_t e4m3_codes4(const float (&q)[4]) {
  uint32_t c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0] + 0.0f, q[1] + 0.0f, 0, false);
  c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2] + 0.0f, q[3] + 0.0f, (int)c, true);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (!(fabsf(q[i]) <= 448.0f))
      c = (c & ~(0xFFu << (8 * i))) | (e4m3_code(round_e4m3_frexp(q[i])) << (8 * i));
  return c;
}

// 16 bytes of a buffer with the agent-scope coherent load (sc1: data written
// by another workgroup of the launch through st_dev, as ld_dev reads it;
// past the range: zeros).
__device__ __forceinline__ uint4 buf_load16_dev(BufRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Requant workgroup of route (t, k) (the first n K workgroups of the back
// launch): y = bf16(t * w) and the per-128 E4M3 requant
// (src/dsv4/dsv4_model.c:6261-6287), published as codes and scales
// (write-through stores), then its flag. Thread i takes 8 consecutive
// values; a 128-group is 16 neighbouring lanes. t comes from the front
// launch; a route without an expert, or with a position outside the
// candidate slots (the routing of a front launch whose waits ran out), reads
// zeros. (Every down workgroup requantising for itself made the routes' t,
// 48 KB read by 512 workgroups, an L2 hot spot; a launch of its own cost a
// launch gap more than the flag hand-off.)
__device__ __forceinline__ void dec_route_requant(const DecArgs &a, int t, int k) {
  const int tid = threadIdx.x;
  const int I = a.I, E = a.E;
  const int e = ldg(dec_tok(a.sel_e, a, t) + k), pos = ldg(dec_tok(a.sel_pos, a, t) + k);
  const float w = ldg(dec_tok(a.sel_w, a, t) + k);
  const bool ok = e >= 0 && e < E && pos >= 0 && pos < E;
  const BufRsrc rt = buf_rsrc(dec_tok(a.sv, a, t) + (size_t)(ok ? pos : 0) * I,
                              ok ? 4u * (uint32_t)I : 0u);
  uint32_t *qc = dec_tok(a.qc, a, t) + (size_t)k * (I / 4);
  float *qcs = dec_tok(a.qcs, a, t) + (size_t)k * (I / 128);
  const int span = (I + 2047) / 2048 * 2048;  // wave-uniform trip count
  for (int base = 8 * tid; base < span; base += 2048) {
    const uint4 u0 = buf_load16(rt, 4u * (uint32_t)base);  // past I: zeros
    const uint4 u1 = buf_load16(rt, 4u * (uint32_t)base + 16u);
    const float v[8] = {u2f(u0.x), u2f(u0.y), u2f(u0.z), u2f(u0.w),
                        u2f(u1.x), u2f(u1.y), u2f(u1.z), u2f(u1.w)};
    float y[8], m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = bf16_round(v[i] * w);
      m = fmaxf(m, fabsf(y[i]));
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    if (base < I) {
      const float scale = act_scale(m);
      const float inv = 1.0f / scale;
      uint32_t c[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          q[i] = y[4 * h + i] * inv;
          if (q[i] > 448.0f) q[i] = 448.0f;
          else if (q[i] < -448.0f) q[i] = -448.0f;
        }
        c[h] = e4m3_codes4(q);
      }
      st_dev(qc + base / 4, c[0]);
      st_dev(qc + base / 4 + 1, c[1]);
      if ((tid & 15) == 0) st_dev(qcs + base / 128, scale);
    }
  }
  dec_signal(dec_tok(a.qf, a, t) + (size_t)k * DEC_FS);
}

// Down workgroup (token t, rows [r0, r0 + 8)): the routes' ids first; then
// the FP4 down rows of every route, all in flight together; then wave 0
// polls the chunk's requant flags (its first poll returns behind its own rows,
// when the requant has normally long finished, so hundreds of workgroups do
// not keep polling the flag lines while the weights stream) and every thread
// copies the routes' E4M3 codes and scales with coherent loads (one memory
// round trip); then the partials route by route: lane: group g of 32
// columns of tile row h rpp + lane / GP,
// a sequential fmaf partial per group; one lane per (route, row) chains the
// groups in order (src/dsv4/dsv4_model.c:1049-1074), y_route = bf16(acc);
// then out = bf16(((0 + y_0) + ... + y_{K-1}) + shared) in ascending expert id
// (src/dsv4/dsv4_model.c:6795-6805). A route without an expert adds zeros.
// NPR: passes per route (inter <= 1024 NPR); routes go in chunks of RC.
template <int NPR>
__device__ __forceinline__ void dec_route_down(const DecArgs &a, int t, int r0, float *lds,
                                               int *s_e, float *s_r, int *s_i) {
  constexpr int RC = NPR <= 2 ? DB_RC : DB_RC / 2;  // routes per chunk
  const int tid = threadIdx.x;
  const int H = a.H, I = a.I, K = a.K, E = a.E;
  const int G = I / 32;
  int GP = 1;
  while (GP < G) GP <<= 1;
  const int rpp = 256 / GP, g = tid % GP, rsub = tid / GP;
  if (tid < K) s_e[tid] = ldg(dec_tok(a.sel_e, a, t) + tid);
  const float ysh = tid < 8 ? ldg(dec_tok(a.ro, a, t) + r0 + tid) : 0.0f;
  __syncthreads();
  uint32_t *qy = reinterpret_cast<uint32_t *>(lds);      // [DB_RC][I / 4] codes
  float *qys = reinterpret_cast<float *>(qy + DB_RC * (I / 4));  // [DB_RC][32]
  float2 *ps = reinterpret_cast<float2 *>(qys + DB_RC * 32);       // [DB_RC * 8][stride]
  const int stride = pair_stride(G);
  // one chunk of routes (k0 .. k0 + nk - 1)
  auto chunk = [&](int k0) {
    const int nk = min(RC, K - k0);
    // every route id of the chunk before the first load (an LDS read between
    // two routes' loads made the compiler drain the earlier loads first)
    int es[RC];
    bool ok[RC];
#pragma unroll
    for (int kk = 0; kk < RC; ++kk) {
      es[kk] = __builtin_amdgcn_readfirstlane(s_e[min(k0 + kk, K - 1)]);
      ok[kk] = kk < nk && es[kk] >= 0 && es[kk] < E;
    }
    uint4 w[RC][NPR];
    uint32_t code[RC][NPR];
#pragma unroll
    for (int kk = 0; kk < RC; ++kk) {
      const uint8_t *W, *S;
      expert_mat(a, ok[kk] ? es[kk] : 0, 2, W, S);
      const BufRsrc rw =
          buf_rsrc(uptr(W + (size_t)r0 * (I / 2)), ok[kk] ? 8u * (uint32_t)(I / 2) : 0u);
      const BufRsrc rs = buf_rsrc(uptr(S + (size_t)r0 * G), ok[kk] ? 8u * (uint32_t)G : 0u);
#pragma unroll
      for (int h = 0; h < NPR; ++h) {
        const int lr = h * rpp + rsub;
        const bool in = lr < 8 && g < G;
        w[kk][h] = buf_load16(rw, in ? (uint32_t)lr * (uint32_t)(I / 2) + 16u * g : 0xFFFFFFF0u);
        code[kk][h] = __builtin_amdgcn_raw_buffer_load_b8(
            rs, in ? (uint32_t)(lr * G + g) : 0xFFFFFFF0u, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the rows are issued before the poll
    if (!dec_wait_flags(dec_tok(a.qf, a, t) + (size_t)k0 * DEC_FS, nk, DEC_FS, nullptr, a.ctl,
                        s_i))
      return;
    {
      // the chunk's codes: nk I bytes as 16-byte pieces (at most 3 per
      // thread for inter <= 1024 NPR) and nk I / 128 scales (at most one per
      // thread), coherent loads (written in this launch)
      const uint32_t nb = (uint32_t)nk * (uint32_t)I;
      const BufRsrc rq = buf_rsrc(uptr(dec_tok(a.qc, a, t) + (size_t)k0 * (I / 4)), nb);
      const BufRsrc rqs = buf_rsrc(uptr(dec_tok(a.qcs, a, t) + (size_t)k0 * (I / 128)),
                                   4u * (uint32_t)(nk * (I / 128)));
      constexpr int NC = (RC * 1024 * NPR + 4095) / 4096;
      uint4 cv[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j)
        cv[j] = buf_load16_dev(rq, 4096u * (uint32_t)j + 16u * (uint32_t)tid);
      const float sc = u2f(__builtin_amdgcn_raw_buffer_load_b32(rqs, 4u * (uint32_t)tid, 0, 16));
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const uint32_t o = 4096u * (uint32_t)j + 16u * (uint32_t)tid;
        if (o < nb) reinterpret_cast<uint4 *>(qy)[o / 16] = cv[j];
      }
      if (tid < nk * (I / 128)) qys[(tid / (I / 128)) * 32 + tid % (I / 128)] = sc;
    }
    __syncthreads();
    // partials: a route's passes share the lane's activation group
#pragma unroll
    for (int kk = 0; kk < RC; ++kk) {
      if (kk >= nk) break;
      const int gc = min(g, G - 1);
      const uint4 c0 = *reinterpret_cast<const uint4 *>(qy + kk * (I / 4) + 8 * gc);
      const uint4 c1 = *reinterpret_cast<const uint4 *>(qy + kk * (I / 4) + 8 * gc + 4);
      const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      float xq[32];
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const float2 lo = fp8x2<false>(cw[d]), hi = fp8x2<true>(cw[d]);
        xq[4 * d] = lo.x;
        xq[4 * d + 1] = lo.y;
        xq[4 * d + 2] = hi.x;
        xq[4 * d + 3] = hi.y;
      }
      const float as = qys[kk * 32 + gc / 4];
#pragma unroll
      for (int h = 0; h < NPR; ++h) {
        const int lr = h * rpp + rsub;
        if (lr < 8 && g < G) {
          float part = fp4_group_partial(w[kk][h], xq);
          float s = as * e8m0(code[kk][h]);
          if (code[kk][h] == 255u) {  // NaN scale: the reference skips the group
            part = 0.0f;
            s = 0.0f;
          }
          ps[(kk * 8 + lr) * stride + g] = make_float2(part, s);
        }
      }
    }
    __syncthreads();
    if (tid < RC * 8) {
      const int kk = tid / 8, lr = tid % 8, k = k0 + kk;
      if (kk < nk) {
        const float acc = ok[kk] ? pair_chain(ps + tid * stride, G) : 0.0f;
        s_r[k * 8 + lr] = bf16_round(acc);  // no expert: the route adds zeros
        if (a.route_out) stg(a.route_out + ((size_t)t * (K + 1) + k) * H + r0 + lr, acc);
      }
    }
    __syncthreads();  // qy, qys and ps are rewritten by the next chunk
  };
  // the model's top-k fits one chunk: no loop, so no loads that the compiler
  // sees carried across a back edge (it drains every load at such a loop's
  // head, the shared expert's row among them, before the first code load)
  if (K <= RC)
    chunk(0);
  else
    for (int k0 = 0; k0 < K; k0 += RC) chunk(k0);
  if (tid < 8) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc += s_r[k * 8 + tid];
    acc += bf16_round(ysh);
    stg(a.out + (size_t)t * H + r0 + tid, bf16_round(acc));
    if (a.route_out) stg(a.route_out + ((size_t)t * (K + 1) + K) * H + r0 + tid, ysh);
  }
}

// Back launch: [n K requant workgroups][n (H / 8) down row tiles], all
// resident at once at the model's shape; the requant workgroups come first in
// dispatch order (the down workgroups wait for them). Requant workgroup 0
// also clears the front launch's records (that launch has ended).
template <int NPR>
__global__ __launch_bounds__(256) void k_dec_back(DecArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_e[32];
  __shared__ float s_r[32 * 8];
  __shared__ int s_i;
  const int nq = a.n * a.K, nt = a.H / 8;
  int b = blockIdx.x;
  if (b < nq) {
    if (b == 0)
      for (int i = threadIdx.x; i < a.n * a.E; i += 256) {
        stg(dec_tok(a.rec, a, i / a.E) + i % a.E, (uint64_t)0);
        stg(dec_tok(a.zrec, a, i / a.E) + i % a.E, (uint64_t)0);
      }
    return dec_route_requant(a, b / a.K, b % a.K);
  }
  b -= nq;
  dec_route_down<NPR>(a, b / nt, (b % nt) * 8, lds, s_e, s_r, &s_i);
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
  unsigned *ctl, *cf, *qf;
  uint64_t *rec, *zrec;
  uint32_t *qc;
  float *qcs, *zx, *zc, *sel_w, *sv, *ro, *xqs;
  uint8_t *xq;
  int *sel_e, *sel_pos, *cl;
  size_t tb;  // bytes of one token's piece
  size_t bytes;
};

// The control words first, then one piece per token, each holding every
// per-token array (256-byte aligned): a token's arrays sit at the same
// offsets whatever the token count of the call, so a workspace serves calls
// with any token count up to its size without stale words in its flags.
DecWs dec_ws_layout(const DSV4GLayer *L, int n_tokens, void *base) {
  const size_t K = (size_t)L->topk, E = (size_t)L->n_experts;
  const size_t H = (size_t)L->hidden, I = (size_t)L->inter;
  DecWs w = {};
  uintptr_t p = (uintptr_t)base;
  auto take = [&](size_t bytes) {
    void *r = (void *)p;
    p += (bytes + 255) & ~(size_t)255;
    return r;
  };
  w.ctl = (unsigned *)take(DEC_CTL_BYTES);
  const uintptr_t t0 = p;
  w.rec = (uint64_t *)take(E * 8);
  w.zrec = (uint64_t *)take(E * 8);
  w.cf = (unsigned *)take(E * 4);
  w.qf = (unsigned *)take(K * DEC_FS * 4);
  w.zx = (float *)take(E * 4);
  w.zc = (float *)take(E * 4);
  w.cl = (int *)take((1 + E + K) * 4);
  w.sel_e = (int *)take(K * 4);
  w.sel_w = (float *)take(K * 4);
  w.sel_pos = (int *)take(K * 4);
  w.sv = (float *)take((E + 1) * I * 4);
  w.ro = (float *)take(H * 4);
  w.qc = (uint32_t *)take(K * I);
  w.qcs = (float *)take(K * (I / 128) * 4);
  w.xq = (uint8_t *)take(H);
  w.xqs = (float *)take(((H + 127) / 128) * 4);
  w.tb = (size_t)(p - t0);
  w.bytes = DEC_CTL_BYTES + (size_t)n_tokens * w.tb;
  return w;
}

size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

// Workgroups of k_dec_front resident at once on the current device (its
// occupancy times the CU count), cached per device and LDS size.
int front_slots(size_t lds, bool st, int *slots) {
  static std::mutex mu;
  static int cache_slots[64];
  static size_t cache_lds[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return dsv4g_fail(DSV4G_EHIP, "moe_decode: hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  const size_t key = 2 * lds + (st ? 1 : 0);  // the kernel variant and its LDS
  if (dev < 64 && cache_slots[dev] > 0 && cache_lds[dev] == key) {
    *slots = cache_slots[dev];
    return DSV4G_OK;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, st ? k_dec_front<true> : k_dec_front<false>, 256, lds) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return dsv4g_fail(DSV4G_EHIP, "moe_decode: occupancy query failed");
  *slots = max(1, per_cu) * max(1, cus);
  if (dev < 64) {
    cache_lds[dev] = key;
    cache_slots[dev] = *slots;
  }
  return DSV4G_OK;
}

int dec_launch(int phase, float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
               int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
               float *wt_out, float *route_out, hipStream_t st, int fast) {
  DSV4G_TRY(dsv4g_layer_ok(L, "moe_decode"));
  if (n_tokens <= 0) return dsv4g_fail(DSV4G_EINVAL, "moe_decode: n_tokens must be > 0");
  if (n_tokens > DEC_MAX_TOKENS)
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: at most %d tokens per call", DEC_MAX_TOKENS);
  if (L->inter > 4096)
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: inter %d above 4096", L->inter);
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
  a.rec = w.rec;
  a.zrec = w.zrec;
  a.cf = w.cf;
  a.qf = w.qf;
  a.qc = w.qc;
  a.qcs = w.qcs;
  a.xq = w.xq;
  a.xqs = w.xqs;
  a.tb = w.tb;
  a.zx = w.zx;
  a.zc = w.zc;
  a.cl = w.cl;
  a.sel_e = w.sel_e;
  a.sel_w = w.sel_w;
  a.sel_pos = w.sel_pos;
  a.sv = w.sv;
  a.ro = w.ro;
  a.route_out = route_out;
  a.idx_out = idx_out;
  a.wt_out = wt_out;
  a.n = n_tokens;
  a.H = L->hidden;
  a.I = L->inter;
  a.E = L->n_experts;
  a.K = L->topk;
  const Fp4Geom qg = fp4_geom_np(a.H, DEC_NP);
  a.gu_tiles = (a.I + qg.tr / 2 - 1) / (qg.tr / 2);
  a.route_scale = L->route_scale;
  {
    const double d = dec_par_depth(a.H) * 0x1p-24, h = a.H * 0x1p-24;
    a.gamma = (float)(d / (1.0 - d) + h / (1.0 - h));
  }
  a.limit = (float)(int)L->swiglu_limit;  // the reference passes the limit as int
  a.fast = fast;
  const int n = n_tokens, H = a.H, I = a.I;
  // a shared FP8 tile: staged (32 KB of weights, then the activation, its
  // scales and the pairs) or in registers (the activation, scales, pairs)
  auto lds_fp8 = [](int in) {
    const size_t CB = (size_t)(in + 127) / 128;
    const size_t act = CB * 132 * 4 + ((CB + 3) & ~(size_t)3) * 4;
    return fp8s_ok(in) ? 32768 + act + (size_t)fp8s_rows(in) * pair_stride((int)CB) * 8 + 1024
                       : act + (size_t)FP8_TR * pair_stride((int)CB) * 8;
  };
  // the staged gate/up tile keeps its scale codes in static LDS
  const size_t lds_fp8_gu = lds_fp8(H) - (dec_sh_gu_staged(H) ? 1024 : 0);
  // the route launch's candidate workgroups: ids, choices and flags in LDS
  const size_t lds_cand = 4 * (2 * (size_t)ROUTER_MAX_EXPERTS + 40);
  if (phase == 0) {  // activation codes, router records and the shared expert's gate/up
    const int t8 = (I + dec_sh_gu_rows(H) - 1) / dec_sh_gu_rows(H);
    const dim3 grid((unsigned)((long)a.E + (long)n * t8 + n));  // + candidate workgroups
    if (dec_sh_gu_staged(H))
      hipLaunchKernelGGL(k_dec_route<true>, grid, dim3(256), max_sz(lds_fp8_gu, lds_cand), st, a);
    else
      hipLaunchKernelGGL(k_dec_route<false>, grid, dim3(256), max_sz(lds_fp8_gu, lds_cand), st, a);
    return dsv4g_check_launch("dec_route");
  }
  if (phase == 1) {
    // streaming: routed pairs and their scales, the activation codes and
    // scales, or a shared FP8 down tile; chains: x and the gate row in fp32,
    // then nc ints or 2 nc floats
    const size_t lds_fp4 = dec_lds_fp4(qg, H, a.E);
    const size_t lds_fp8_dn = lds_fp8(I);
    const size_t lds_chain = (size_t)8 * H + (size_t)4 * ((a.E + 3) & ~3) + sizeof(SplitLds);
    const size_t lds = max_sz(max_sz(lds_fp4, max_sz(lds_chain, (size_t)8 * H + (size_t)8 * a.E)),
                              lds_fp8_dn);
    int slots = 0;
    DSV4G_TRY(front_slots(lds, fp8s_ok(I), &slots));
    a.maxc = min(max(a.K + 10, 16), a.E);
    // streaming workgroups: the resident slots beside the chains
    a.n_stream = max(64, slots - n * a.maxc);
    const long blocks = (long)n * a.maxc + a.n_stream;
    if (fp8s_ok(I))
      hipLaunchKernelGGL(k_dec_front<true>, dim3((unsigned)blocks), dim3(256), lds, st, a);
    else
      hipLaunchKernelGGL(k_dec_front<false>, dim3((unsigned)blocks), dim3(256), lds, st, a);
    return dsv4g_check_launch("dec_front");
  }
  if (phase == 2) {
    const int G = I / 32;
    const size_t lds =
        (size_t)DB_RC * I + DB_RC * 32 * 4 + (size_t)DB_RC * 8 * pair_stride(G) * 8;
    const dim3 grid((unsigned)((long)n * a.K + (long)n * (H / 8)));
    if (I <= 1024)
      hipLaunchKernelGGL(k_dec_back<1>, grid, dim3(256), lds, st, a);
    else if (I <= 2048)
      hipLaunchKernelGGL(k_dec_back<2>, grid, dim3(256), lds, st, a);
    else
      hipLaunchKernelGGL(k_dec_back<4>, grid, dim3(256), lds, st, a);
    return dsv4g_check_launch("dec_back");
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
uint64_t g_scratch_shape[64];  // the layer shape of the last call per device

// The current device's scratch address, resolved once per device (device
// globals start zeroed when the code object loads).
int scratch_ptr(const DSV4GLayer *L, hipStream_t st, void **out) {
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
    g_scratch_ptr[dev] = p;
  }
  // the records and flags sit at offsets of the layer's shape: another
  // shape than the last call's finds stale words there, so the array is
  // cleared first (a fill kernel, which graph capture records as well)
  const uint64_t shape = (uint64_t)L->hidden ^ ((uint64_t)L->inter << 16) ^
                         ((uint64_t)L->n_experts << 32) ^ ((uint64_t)L->topk << 48);
  if (g_scratch_shape[dev] != 0 && g_scratch_shape[dev] != shape) {
    const size_t words = DEC_SCRATCH_BYTES / 4;
    hipLaunchKernelGGL(k_fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       (unsigned *)g_scratch_ptr[dev], words);
    DSV4G_TRY(dsv4g_check_launch("moe_noalloc_clear"));
  }
  g_scratch_shape[dev] = shape;
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

unsigned *dsv4g_decode_status_word(void *workspace) {
  return (unsigned *)workspace + DEC_ERR;
}

int dsv4g_moe_decode_status(unsigned *status, void *workspace, void *stream) {
  if (!status || !workspace || ((uintptr_t)workspace & 255))
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode_status: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  DSV4G_HIP(hipMemcpyAsync(status, (const unsigned *)workspace + DEC_ERR, sizeof(unsigned),
                           hipMemcpyDeviceToHost, st));
  DSV4G_HIP(hipStreamSynchronize(st));
  if (*status) {
    hipLaunchKernelGGL(k_fill_zero_u32, dim3(1), dim3(64), 0, st,
                       (unsigned *)workspace + DEC_ERR, (size_t)1);
    DSV4G_TRY(dsv4g_check_launch("moe_decode_status"));
  }
  return 0;
}

int dsv4g_moe_decode_phase(int phase, float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, void *stream) {
  const int fast = (phase & DSV4G_DECODE_FAST) != 0;
  return dec_launch(phase & ~DSV4G_DECODE_FAST, out, x, L, token_ids, n_tokens, workspace,
                    workspace_bytes, nullptr, nullptr, nullptr, (hipStream_t)stream, fast);
}

int dsv4g_moe_decode_routing(int *idx_out, float *wt_out, const DSV4GLayer *L, int n_tokens,
                             void *workspace, void *stream) {
  const DecWs w = dec_ws_layout(L, n_tokens, workspace);
  hipStream_t st = (hipStream_t)stream;
  const size_t row = (size_t)L->topk * 4;  // one token's routing, from its piece
  if (idx_out)
    DSV4G_HIP(hipMemcpy2DAsync(idx_out, row, w.sel_e, w.tb, row, (size_t)n_tokens,
                               hipMemcpyDeviceToDevice, st));
  if (wt_out)
    DSV4G_HIP(hipMemcpy2DAsync(wt_out, row, w.sel_w, w.tb, row, (size_t)n_tokens,
                               hipMemcpyDeviceToDevice, st));
  return 0;
}

int dsv4g_moe_forward(float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
                      int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
                      float *wt_out, void *stream) {
  for (int phase = 0; phase < DEC_PHASES; ++phase)
    DSV4G_TRY(dec_launch(phase, out, x, L, token_ids, n_tokens, workspace, workspace_bytes,
                         idx_out, wt_out, nullptr, (hipStream_t)stream, 0));
  return 0;
}

int dsv4g_moe_forward_fast(float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, int *idx_out, float *wt_out, void *stream) {
  for (int phase = 0; phase < DEC_PHASES; ++phase)
    DSV4G_TRY(dec_launch(phase, out, x, L, token_ids, n_tokens, workspace, workspace_bytes,
                         idx_out, wt_out, nullptr, (hipStream_t)stream, 1));
  return 0;
}

int dsv4g_moe_forward_routes(float *out, const float *x, const DSV4GLayer *L,
                             const int *token_ids, int n_tokens, void *workspace,
                             size_t workspace_bytes, int *idx_out, float *wt_out,
                             float *route_out, int fast, void *stream) {
  for (int phase = 0; phase < DEC_PHASES; ++phase)
    DSV4G_TRY(dec_launch(phase, out, x, L, token_ids, n_tokens, workspace, workspace_bytes,
                         idx_out, wt_out, route_out, (hipStream_t)stream, fast ? 1 : 0));
  return 0;
}

int dsv4g_moe_forward_noalloc(float *out, const float *x, const DSV4GLayer *L,
                              const int *token_ids, int n_tokens, int *idx_out, float *wt_out,
                              void *stream) {
  DSV4G_TRY(dsv4g_layer_ok(L, "moe_noalloc"));
  if (n_tokens <= 0) return dsv4g_fail(DSV4G_EINVAL, "moe_noalloc: n_tokens must be > 0");
  const size_t need = dsv4g_moe_workspace_bytes(L, n_tokens);
  if (need > DEC_SCRATCH_BYTES)
    return dsv4g_fail(DSV4G_EINVAL,
                      "moe_noalloc: %d tokens of this layer need %zu bytes of workspace, more "
                      "than the %zu bytes of the library's scratch; pass fewer tokens per call",
                      n_tokens, need, DEC_SCRATCH_BYTES);
  void *ws = nullptr;
  DSV4G_TRY(scratch_ptr(L, (hipStream_t)stream, &ws));
  return dsv4g_moe_forward(out, x, L, token_ids, n_tokens, ws, need, idx_out, wt_out, stream);
}

int dsv4g_moe_noalloc_status(unsigned *status, void *stream) {
  if (!status) return dsv4g_fail(DSV4G_EINVAL, "moe_noalloc_status: status is NULL");
  *status = 0u;
  int dev = 0;
  DSV4G_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return dsv4g_fail(DSV4G_EINVAL, "moe_noalloc_status: device %d", dev);
  void *p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev];
  }
  if (!p) return 0;  // no noalloc call on this device yet
  hipStream_t st = (hipStream_t)stream;
  DSV4G_HIP(hipMemcpyAsync(status, (const unsigned *)p + DEC_ERR, sizeof(unsigned),
                           hipMemcpyDeviceToHost, st));
  DSV4G_HIP(hipStreamSynchronize(st));
  if (*status) {
    // a wait that ran out leaves records and flags of its call set
    const size_t words = DEC_SCRATCH_BYTES / 4;
    hipLaunchKernelGGL(k_fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       (unsigned *)p, words);
    DSV4G_TRY(dsv4g_check_launch("moe_noalloc_status"));
  }
  return 0;
}

}  // extern "C"
