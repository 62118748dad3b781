// dsv4_moe.hip - MoE layer kernels for gfx950: router (logits, sqrt-softplus
// scoring, biased top-k, weights), SwiGLU + FP8 requant, multi-expert GEMV
// launches and the ordered combine. Together they reproduce moe_forward
// (src/dsv4/dsv4_model.c:6599-6807) bit for bit.
//
// Router exactness. The reference's logit z[e] is one 4096-long fmaf chain in
// column order (dsv4_gemv_bf16, src/dsv4/dsv4_model.c:298-303), and the route
// weights depend on z of the selected experts through sqrt-softplus. A
// parallel dot product is fast but differs in the last bits, which the
// SwiGLU requant can amplify. So: (1) all logits are computed in parallel
// together with sum|w*x|, which bounds the difference between any two
// summation orders; (2) every expert whose approximate choice lies within that
// bound of the k-th best is a candidate; (3) candidates get the exact
// sequential chain, one lane each, and selection and weights use only exact
// values. Scores use the bit-exact libm restatements (dsv4_libm.h).
#include "dsv4_device.h"
#include "dsv4_gpu_internal.h"
#include "dsv4_tiles.h"

using namespace dsv4;

namespace dsv4 {

#define ROUTER_MAX_EXPERTS 1024
// LDS of one k_expert_pass workgroup: the larger of the FP4 tile (float2 pairs)
// and the FP8 tile (padded qx plus float2 pairs).
#define EXPERT_LDS_BYTES (FP8_MAX_IN / 128 * 132 * 4 + FP8_TR * (FP8_MAX_IN / 128 + 1) * 8)

// ------------------------------------------------------------- router ----
// z and sum|bf16(g)*x| per (token, expert); one wave per expert row.
__global__ __launch_bounds__(256) void k_router_logits(float *__restrict__ z,
                                                       float *__restrict__ zabs,
                                                       const float *__restrict__ x,
                                                       const uint16_t *__restrict__ G,
                                                       int H, int E) {
  const int lane = threadIdx.x % 64;
  const int e = blockIdx.x * 4 + threadIdx.x / 64;
  const int t = blockIdx.y;
  if (e >= E) return;
  const float *xt = x + (size_t)t * H;
  const uint16_t *gr = G + (size_t)e * H;
  float acc = 0.0f, aabs = 0.0f;
  for (int c = 8 * lane; c < H; c += 512) {
    const uint4 w = *reinterpret_cast<const uint4 *>(gr + c);
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float p0 = u2f(wd[d] << 16) * xt[c + 2 * d];
      const float p1 = u2f(wd[d] & 0xFFFF0000u) * xt[c + 2 * d + 1];
      acc += p0;
      acc += p1;
      aabs += fabsf(p0);
      aabs += fabsf(p1);
    }
  }
  acc = wave_sum(acc);
  aabs = wave_sum(aabs);
  if (lane == 0) {
    z[(size_t)t * E + e] = acc;
    zabs[(size_t)t * E + e] = aabs;
  }
}

// gamma_n = n u / (1 - n u), u = 2^-24: the classic bound on the rounding
// error of any n-term summation order.
__device__ __forceinline__ float gamma_n(int n) {
  const double nu = (double)n * 0x1p-24;
  return (float)(nu / (1.0 - nu));
}

// One workgroup (256 threads) per token. Writes idx[K] ascending and wt[K].
__global__ __launch_bounds__(256) void k_router_select(
    int *__restrict__ idx_out, float *__restrict__ wt_out, const float *__restrict__ z_a,
    const float *__restrict__ zabs, const float *__restrict__ x,
    const uint16_t *__restrict__ G, const float *__restrict__ bias,
    const int64_t *__restrict__ tid2eid, const int *__restrict__ token_ids, int H, int E,
    int K, float route_scale, int public_mode) {
  __shared__ __align__(16) float xs[8192];
  __shared__ float choice_a[ROUTER_MAX_EXPERTS];
  __shared__ int cand[ROUTER_MAX_EXPERTS];
  __shared__ float csc[ROUTER_MAX_EXPERTS];  // exact score per candidate
  __shared__ float cch[ROUTER_MAX_EXPERTS];  // exact choice per candidate
  __shared__ unsigned char used[ROUTER_MAX_EXPERTS];
  __shared__ float dred[4];
  __shared__ int ncand_s;
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const float *xt = x + (size_t)t * H;
  for (int i = tid; i < H; i += 256) xs[i] = xt[i];
  const float *zt = z_a + (size_t)t * E;
  const float *at = zabs + (size_t)t * E;
  float dmax = 0.0f;
  for (int e = tid; e < E; e += 256) {
    choice_a[e] = sqrt_softplus(zt[e]) + (bias ? bias[e] : 0.0f);
    used[e] = 0;
    dmax = fmaxf(dmax, at[e]);
  }
  dmax = wave_max(dmax);
  if (tid % 64 == 0) dred[tid / 64] = dmax;
  __syncthreads();
  const bool hash = tid2eid != nullptr;
  if (tid == 0) {
    if (hash) {
      const int64_t *row = tid2eid + (size_t)token_ids[t] * K;
      for (int k = 0; k < K; ++k) cand[k] = (int)row[k];
      ncand_s = K;
    } else {
      // Bound on |z_parallel - z_sequential| (any two summation orders of the
      // same H products), mapped through |d score / dz| <= 1/2, plus slack for
      // the score evaluation's own rounding; doubled for both sides.
      const float sum_abs = fmaxf(fmaxf(dred[0], dred[1]), fmaxf(dred[2], dred[3]));
      const float bound_z = (gamma_n(H / 64 + 8) + gamma_n(H)) * sum_abs;
      const float delta = 2.0f * (0.5f * bound_z + 1e-5f);
      // k-th best approximate choice (repeated strict '>' maximum)
      float kth = -__builtin_inff();
      for (int k = 0; k < K; ++k) {
        int be = -1;
        float bv = -__builtin_inff();
        for (int e = 0; e < E; ++e)
          if (!used[e] && choice_a[e] > bv) {
            bv = choice_a[e];
            be = e;
          }
        if (be >= 0) used[be] = 1;
        kth = bv;
      }
      int n = 0;
      const float thr = kth - delta;
      for (int e = 0; e < E; ++e)
        if (choice_a[e] >= thr) cand[n++] = e;
      ncand_s = n;
    }
  }
  __syncthreads();
  const int nc = ncand_s;
  // exact sequential chains, one lane each: fmaf for moe_forward
  // (src/dsv4/dsv4_model.c:298-303), unfused z += w*x for the public router
  // (src/dsv4/dsv4_ops.c:502)
  for (int ci = tid; ci < nc; ci += 256) {
    const int e = cand[ci];
    if (e < 0 || e >= E) {  // malformed tid2eid entry: never read out of bounds
      csc[ci] = 0.0f;
      cch[ci] = -__builtin_inff();
      continue;
    }
    const uint16_t *gr = G + (size_t)e * H;
    float acc = 0.0f;
    if (public_mode) {
      for (int c = 0; c < H; c += 2) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(gr + c);
        const float p0 = u2f(w << 16) * xs[c];
        acc = acc + p0;
        const float p1 = u2f(w & 0xFFFF0000u) * xs[c + 1];
        acc = acc + p1;
      }
    } else for (int c = 0; c < H; c += 8) {
      const uint4 w = *reinterpret_cast<const uint4 *>(gr + c);
      const float4 xa = *reinterpret_cast<const float4 *>(xs + c);
      const float4 xb = *reinterpret_cast<const float4 *>(xs + c + 4);
      acc = fmaf(u2f(w.x << 16), xa.x, acc);
      acc = fmaf(u2f(w.x & 0xFFFF0000u), xa.y, acc);
      acc = fmaf(u2f(w.y << 16), xa.z, acc);
      acc = fmaf(u2f(w.y & 0xFFFF0000u), xa.w, acc);
      acc = fmaf(u2f(w.z << 16), xb.x, acc);
      acc = fmaf(u2f(w.z & 0xFFFF0000u), xb.y, acc);
      acc = fmaf(u2f(w.w << 16), xb.z, acc);
      acc = fmaf(u2f(w.w & 0xFFFF0000u), xb.w, acc);
    }
    const float sc = sqrt_softplus(acc);
    csc[ci] = sc;
    cch[ci] = sc + (bias ? bias[e] : 0.0f);
  }
  __syncthreads();
  if (tid == 0) {
    int order[32];
    float score_sel[32], wt[32];
    if (hash) {
      for (int k = 0; k < K; ++k) {
        order[k] = cand[k];
        score_sel[k] = csc[k];
      }
    } else {
      for (int i = 0; i < nc; ++i) used[i] = 0;  // reuse as per-candidate flags
      for (int k = 0; k < K; ++k) {
        int bi = -1;
        float bv = -__builtin_inff();
        for (int i = 0; i < nc; ++i)  // candidates are in ascending id
          if (!used[i] && cch[i] > bv) {
            bv = cch[i];
            bi = i;
          }
        if (bi >= 0) used[bi] = 1;
        order[k] = bi >= 0 ? cand[bi] : -1;
        score_sel[k] = bi >= 0 ? csc[bi] : 0.0f;
      }
    }
    // weights from the unbiased scores (src/dsv4/dsv4_model.c:6650-6658;
    // the public router multiplies by 1/sum, src/dsv4/dsv4_ops.c:528-531)
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum += score_sel[k];
    if (public_mode) {
      const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
      for (int k = 0; k < K; ++k) {
        const float tmp = score_sel[k] * inv;
        wt[k] = tmp * route_scale;
      }
    } else if (sum > 0.0f) {
      const float rs = route_scale / sum;
      for (int k = 0; k < K; ++k) wt[k] = score_sel[k] * rs;
    } else {
      for (int k = 0; k < K; ++k) wt[k] = 0.0f;
    }
    // exchange sort ascending by id (src/dsv4/dsv4_model.c:6666-6674)
    for (int i = 0; i < K; ++i)
      for (int j = i + 1; j < K; ++j)
        if (order[j] < order[i]) {
          const int ti = order[i];
          order[i] = order[j];
          order[j] = ti;
          const float tw = wt[i];
          wt[i] = wt[j];
          wt[j] = tw;
        }
    for (int k = 0; k < K; ++k) {
      idx_out[(size_t)t * K + k] = order[k];
      wt_out[(size_t)t * K + k] = wt[k];
    }
  }
}

// ---------------------------------------------------------- SwiGLU -------
// routed_swiglu_quant (src/dsv4/dsv4_model.c:6239-6287) for one 128-group:
// y = bf16((silu(g)*u)*w), amax, E4M3 requant. One wave per group.
// grid = (I/128, nslots). Slot s has gate at gu + s*2*I and up at +I.
// Route weight: with K > 0 the slots are [token][K+1] and slot (t, k) uses
// wt[t*K + k] for k < K and 1 for the shared slot k == K; with K == 0 slot s
// uses wt[s]; wt == nullptr means weight 1.
__global__ __launch_bounds__(64) void k_swiglu_quant(float *__restrict__ qy,
                                                     float *__restrict__ qys,
                                                     const float *__restrict__ gu,
                                                     const float *__restrict__ wt, int K,
                                                     int I, float limit) {
  const int g = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const float *gate = gu + (size_t)s * 2 * I;
  const float *up = gate + I;
  float w = 1.0f;
  if (wt) {
    if (K > 0) {
      const int t = s / (K + 1), k = s % (K + 1);
      if (k < K) w = wt[(size_t)t * K + k];
    } else {
      w = wt[s];
    }
  }
  const int i0 = g * 128 + lane, i1 = i0 + 64;
  float y0 = 0.0f, y1 = 0.0f;
  if (i0 < I) y0 = bf16_round(swiglu_t(gate[i0], up[i0], limit) * w);
  if (i1 < I) y1 = bf16_round(swiglu_t(gate[i1], up[i1], limit) * w);
  const float amax = wave_max(fmaxf(fabsf(y0), fabsf(y1)));
  const float scale = act_scale(amax);
  const float inv = 1.0f / scale;
  float *q = qy + (size_t)s * I;
  if (lane == 0) qys[(size_t)s * ((I + 127) / 128) + g] = scale;
  if (i0 < I) q[i0] = quant_e4m3(y0, inv);
  if (i1 < I) q[i1] = quant_e4m3(y1, inv);
}

// ----------------------------------------------- multi-expert GEMVs ------
// Work slots: for token t and route k < K the routed expert idx[t][k]; slot
// K of each token is the shared FP8 expert. Phase 0 computes gate/up rows
// (gu[slot] = [gate | up]), phase 1 the down rows (ro[slot]).
struct ExpertPass {
  const int *idx;  // [n][K]
  const uint8_t *experts;
  size_t expert_stride, scale_run;
  const uint8_t *sh[3], *sh_s[3];  // gate, up, down
  const float *qx, *qxs;           // phase 0: [n][H], [n][H/128]
  const float *qy, *qys;           // phase 1: [n][K+1][I], [n][K+1][I/128]
  float *out;                      // phase 0: gu [n][K+1][2][I]; phase 1: ro [n][K+1][H]
  int n, K, H, I, E, phase;
  int fp4_tiles, fp8_tiles;  // row tiles per matrix
};

__global__ __launch_bounds__(256) void k_expert_pass(ExpertPass p) {
  __shared__ float4 lds[EXPERT_LDS_BYTES / 16];
  float2 *ps = reinterpret_cast<float2 *>(lds);
  const int nmat = p.phase == 0 ? 2 : 1;
  const int in = p.phase == 0 ? p.H : p.I;
  const int rows = p.phase == 0 ? p.I : p.H;
  const int routed_blocks = p.n * p.K * nmat * p.fp4_tiles;
  int b = blockIdx.x;
  if (b < routed_blocks) {
    const int tile = b % p.fp4_tiles;
    b /= p.fp4_tiles;
    const int m = b % nmat;
    b /= nmat;
    const int k = b % p.K, t = b / p.K;
    const int e = p.idx[t * p.K + k];
    const int slot = t * (p.K + 1) + k;
    const Fp4Geom q = fp4_geom(in);
    if (e < 0 || e >= p.E) {  // no expert selected (all choices NaN): zero rows
      float *y = p.phase == 0 ? p.out + ((size_t)slot * 2 + m) * p.I : p.out + (size_t)slot * p.H;
      for (int r = tile * q.tr + threadIdx.x; r < min(rows, (tile + 1) * q.tr); r += 256)
        y[r] = 0.0f;
      return;
    }
    const uint8_t *scales = p.experts + (size_t)e * p.expert_stride;
    const uint8_t *weights = scales + p.scale_run;
    const size_t w1 = (size_t)p.I * (p.H / 2), w2 = (size_t)p.H * (p.I / 2);
    const size_t s1 = (size_t)p.I * (p.H / 32), s2 = (size_t)p.H * (p.I / 32);
    const uint8_t *W, *S;
    if (p.phase == 0) {
      W = m == 0 ? weights : weights + w1 + w2;
      S = m == 0 ? scales : scales + s1 + s2;
    } else {
      W = weights + w1;
      S = scales + s1;
    }
    const float *qx = p.phase == 0 ? p.qx + (size_t)t * p.H : p.qy + (size_t)slot * p.I;
    const float *qs =
        p.phase == 0 ? p.qxs + (size_t)t * (p.H / 128) : p.qys + (size_t)slot * (p.I / 128);
    float *y = p.phase == 0 ? p.out + ((size_t)slot * 2 + m) * p.I : p.out + (size_t)slot * p.H;
    fp4_rows_exact(y, qx, qs, W, S, in, rows, tile * q.tr, ps);
    return;
  }
  b -= routed_blocks;
  const int tile = b % p.fp8_tiles;
  b /= p.fp8_tiles;
  const int m = b % nmat, t = b / nmat;
  const int slot = t * (p.K + 1) + p.K;
  const int mi = p.phase == 0 ? m : 2;
  const float *qx = p.phase == 0 ? p.qx + (size_t)t * p.H : p.qy + (size_t)slot * p.I;
  const float *qs =
      p.phase == 0 ? p.qxs + (size_t)t * (p.H / 128) : p.qys + (size_t)slot * (p.I / 128);
  float *y = p.phase == 0 ? p.out + ((size_t)slot * 2 + m) * p.I : p.out + (size_t)slot * p.H;
  float *xs = reinterpret_cast<float *>(lds);
  float2 *ps8 = reinterpret_cast<float2 *>(xs + FP8_MAX_IN / 128 * 132);
  fp8_rows_exact(y, qx, qs, p.sh[mi], p.sh_s[mi], in, rows, tile * FP8_TR, 1, xs, ps8);
}

// out[t][i] = bf16(((0 + ro[t][0][i]) + ... + ro[t][K-1][i]) + ro[t][K][i])
// (src/dsv4/dsv4_model.c:6795-6805).
__global__ void k_combine(float *__restrict__ out, const float *__restrict__ ro, int n, int K,
                          int H) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= (size_t)n * H) return;
  const size_t t = i / H, c = i % H;
  const float *r = ro + t * (size_t)(K + 1) * H + c;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc += r[(size_t)k * H];
  acc += r[(size_t)K * H];
  out[i] = bf16_round(acc);
}

}  // namespace dsv4

// ============================================================ C-ABI =====
using namespace dsv4;

static int layer_ok(const DSV4GLayer *L, const char *who) {
  if (!L || !L->gate_w || !L->experts || !L->sh1 || !L->sh3 || !L->sh2)
    return dsv4g_fail(DSV4G_EINVAL, "%s: layer descriptor incomplete", who);
  if (L->hidden <= 0 || L->hidden % 128 || L->hidden > 8192 || L->inter <= 0 ||
      L->inter % 128 || L->inter > 8192)
    return dsv4g_fail(DSV4G_EINVAL,
                      "%s: hidden/inter must be positive multiples of 128, at most 8192", who);
  if (L->n_experts <= 0 || L->n_experts > ROUTER_MAX_EXPERTS || L->topk <= 0 ||
      L->topk > 32 || L->topk > L->n_experts)
    return dsv4g_fail(DSV4G_EINVAL, "%s: n_experts %d / topk %d out of range", who,
                      L->n_experts, L->topk);
  return 0;
}

extern "C" {

// Decode workspace layout: 256-byte aligned pieces, in this order.
struct MoeWs {
  float *qx, *qxs, *z, *zabs, *wt, *gu, *qy, *qys, *ro;
  int *idx;
  size_t bytes;
};

static MoeWs moe_ws_layout(const DSV4GLayer *L, int n_tokens, void *base) {
  const size_t n = (size_t)n_tokens, K = (size_t)L->topk, E = (size_t)L->n_experts;
  const size_t H = (size_t)L->hidden, I = (size_t)L->inter;
  MoeWs w = {};
  uintptr_t p = ((uintptr_t)base + 255) & ~(uintptr_t)255;
  const uintptr_t p0 = (uintptr_t)base;
  auto take = [&](size_t bytes) {
    void *r = (void *)p;
    p += (bytes + 255) & ~(size_t)255;
    return r;
  };
  w.qx = (float *)take(n * H * 4);
  w.qxs = (float *)take(n * (H / 128) * 4);
  w.z = (float *)take(n * E * 4);
  w.zabs = (float *)take(n * E * 4);
  w.wt = (float *)take(n * K * 4);
  w.gu = (float *)take(n * (K + 1) * 2 * I * 4);
  w.qy = (float *)take(n * (K + 1) * I * 4);
  w.qys = (float *)take(n * (K + 1) * (I / 128) * 4);
  w.ro = (float *)take(n * (K + 1) * H * 4);
  w.idx = (int *)take(n * K * 4);
  w.bytes = (size_t)(p - p0) + 256;
  return w;
}

extern "C" size_t dsv4g_moe_workspace_bytes(const DSV4GLayer *L, int n_tokens) {
  return moe_ws_layout(L, n_tokens, nullptr).bytes;
}

int dsv4g_router(int *idx, float *wt, const float *x, const DSV4GLayer *L,
                 const int *token_ids, int n_tokens, float *z_ws, float *zabs_ws,
                 void *stream) {
  DSV4G_TRY(layer_ok(L, "router"));
  if (L->tid2eid && !token_ids)
    return dsv4g_fail(DSV4G_EINVAL, "router: hash layer needs token_ids");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_router_logits, dim3((L->n_experts + 3) / 4, n_tokens), dim3(256), 0, st,
                     z_ws, zabs_ws, x, L->gate_w, L->hidden, L->n_experts);
  DSV4G_TRY(dsv4g_check_launch("router_logits"));
  hipLaunchKernelGGL(k_router_select, dim3(n_tokens), dim3(256), 0, st, idx, wt, z_ws, zabs_ws,
                     x, L->gate_w, L->bias, L->tid2eid, token_ids, L->hidden, L->n_experts,
                     L->topk, L->route_scale, 0);
  return dsv4g_check_launch("router_select");
}

// Public dsv4_router semantics (src/dsv4/dsv4_ops.c:473-545) for one token.
// tid2eid, when hash_layer, points at that token's row and token_id at 0.
int dsv4g_router_public(int *idx, float *wt, const float *x, const uint16_t *gate,
                        const float *bias, const int64_t *tid2eid, const int *token_id,
                        int hidden, int n_experts, int topk, int hash_layer,
                        float route_scale, float *z_ws, float *zabs_ws, void *stream) {
  if (hidden <= 0 || hidden % 8 || hidden > 8192 || n_experts <= 0 ||
      n_experts > ROUTER_MAX_EXPERTS || topk <= 0 || topk > 32 || topk > n_experts)
    return dsv4g_fail(DSV4G_EINVAL, "router: unsupported shape");
  if (hash_layer && (!tid2eid || !token_id))
    return dsv4g_fail(DSV4G_EINVAL, "router: hash layer needs tid2eid");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_router_logits, dim3((n_experts + 3) / 4, 1), dim3(256), 0, st, z_ws,
                     zabs_ws, x, gate, hidden, n_experts);
  DSV4G_TRY(dsv4g_check_launch("router_logits"));
  hipLaunchKernelGGL(k_router_select, dim3(1), dim3(256), 0, st, idx, wt, z_ws, zabs_ws, x,
                     gate, bias, hash_layer ? tid2eid : nullptr, token_id, hidden, n_experts,
                     topk, route_scale, 1);
  return dsv4g_check_launch("router_select");
}

int dsv4g_swiglu_quant(float *qy, float *qys, const float *gate_up, const float *wt, int K,
                       int n_slots, int inter, float limit, void *stream) {
  if (inter <= 0 || inter % 128 || n_slots <= 0 || K < 0)
    return dsv4g_fail(DSV4G_EINVAL, "swiglu_quant: bad size");
  hipLaunchKernelGGL(k_swiglu_quant, dim3(inter / 128, n_slots), dim3(64), 0,
                     (hipStream_t)stream, qy, qys, gate_up, wt, K, inter, limit);
  return dsv4g_check_launch("swiglu_quant");
}

// One phase of the decode MoE layer (moe_forward per token, bit-exact):
//   0 activation quant + router, 1 gate/up GEMVs (6 FP4 routed + shared FP8),
//   2 SwiGLU + FP8 requant, 3 down GEMVs, 4 ordered combine into out.
// Phases run in order on one stream; dsv4g_moe_forward runs all five.
int dsv4g_moe_decode_phase(int phase, float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, void *stream) {
  DSV4G_TRY(layer_ok(L, "moe_decode"));
  if (n_tokens <= 0) return dsv4g_fail(DSV4G_EINVAL, "moe_decode: n_tokens must be > 0");
  if (workspace_bytes < dsv4g_moe_workspace_bytes(L, n_tokens))
    return dsv4g_fail(DSV4G_EINVAL, "moe_decode: workspace too small (%zu < %zu)",
                      workspace_bytes, dsv4g_moe_workspace_bytes(L, n_tokens));
  hipStream_t st = (hipStream_t)stream;
  const int n = n_tokens, K = L->topk, H = L->hidden, I = L->inter;
  const MoeWs w = moe_ws_layout(L, n, workspace);
  if (phase == 0) {
    DSV4G_TRY(dsv4g_quant_fp8_act(w.qx, w.qxs, x, H, n, stream));
    return dsv4g_router(w.idx, w.wt, x, L, token_ids, n, w.z, w.zabs, stream);
  }
  if (phase == 2)
    return dsv4g_swiglu_quant(w.qy, w.qys, w.gu, w.wt, K, n * (K + 1), I,
                              (float)(int)L->swiglu_limit, stream);
  if (phase == 4) {
    const size_t total = (size_t)n * H;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, out,
                       w.ro, n, K, H);
    return dsv4g_check_launch("combine");
  }
  if (phase != 1 && phase != 3) return dsv4g_fail(DSV4G_EINVAL, "moe_decode: bad phase %d", phase);
  ExpertPass p = {};
  p.idx = w.idx;
  p.experts = L->experts;
  p.expert_stride = L->expert_stride;
  p.scale_run = L->scale_run;
  p.sh[0] = L->sh1;
  p.sh[1] = L->sh3;
  p.sh[2] = L->sh2;
  p.sh_s[0] = L->sh1_s;
  p.sh_s[1] = L->sh3_s;
  p.sh_s[2] = L->sh2_s;
  p.qx = w.qx;
  p.qxs = w.qxs;
  p.qy = w.qy;
  p.qys = w.qys;
  p.n = n;
  p.K = K;
  p.H = H;
  p.I = I;
  p.E = L->n_experts;
  const int in = phase == 1 ? H : I, rows = phase == 1 ? I : H, nmat = phase == 1 ? 2 : 1;
  int G = in / 32, gp = 1;
  while (gp < G) gp <<= 1;
  int tr = FP4_LDS_ENTRIES / gp;
  if (tr > 256) tr = 256;
  p.phase = phase == 1 ? 0 : 1;
  p.out = phase == 1 ? w.gu : w.ro;
  p.fp4_tiles = (rows + tr - 1) / tr;
  p.fp8_tiles = (rows + FP8_TR - 1) / FP8_TR;
  const int blocks = n * K * nmat * p.fp4_tiles + n * nmat * p.fp8_tiles;
  hipLaunchKernelGGL(k_expert_pass, dim3(blocks), dim3(256), 0, st, p);
  return dsv4g_check_launch(phase == 1 ? "expert_pass(gate/up)" : "expert_pass(down)");
}

// Routing of the last decode call made with this workspace.
int dsv4g_moe_decode_routing(int *idx_out, float *wt_out, const DSV4GLayer *L, int n_tokens,
                             void *workspace, void *stream) {
  const MoeWs w = moe_ws_layout(L, n_tokens, workspace);
  hipStream_t st = (hipStream_t)stream;
  if (idx_out)
    DSV4G_HIP(hipMemcpyAsync(idx_out, w.idx, (size_t)n_tokens * L->topk * sizeof(int),
                             hipMemcpyDeviceToDevice, st));
  if (wt_out)
    DSV4G_HIP(hipMemcpyAsync(wt_out, w.wt, (size_t)n_tokens * L->topk * sizeof(float),
                             hipMemcpyDeviceToDevice, st));
  return 0;
}

// Decode-path MoE layer: moe_forward per token, bit-exact. idx/wt (optional,
// device) receive the routing.
int dsv4g_moe_forward(float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
                      int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
                      float *wt_out, void *stream) {
  for (int phase = 0; phase < 5; ++phase)
    DSV4G_TRY(dsv4g_moe_decode_phase(phase, out, x, L, token_ids, n_tokens, workspace,
                                     workspace_bytes, stream));
  return dsv4g_moe_decode_routing(idx_out, wt_out, L, n_tokens, workspace, stream);
}

}  // extern "C"
