// dsv4_moe.hip - router entry points for gfx950 (logits, sqrt-softplus
// scoring, biased top-k, weights; the moe_forward router of
// src/dsv4/dsv4_model.c:6615-6676 and the public dsv4_router of
// src/dsv4/dsv4_ops.c:473-545) and the standalone SwiGLU + FP8 requant
// (src/dsv4/dsv4_model.c:6239-6287), all bit for bit.
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

// ------------------------------------------------------------- router ----
// (The decode MoE layer itself is in dsv4_decode.hip; these kernels serve the
// standalone router entry points.)
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
      const float thr = cand_threshold(kth, delta);
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

// expert_forward's down projection (dsv4_gemv_fp4_q, src/dsv4/dsv4_model.c:
// 1049-1074 via :6336-6345) with the per-128 E4M3 requant of
// routed_swiglu_quant (:6269-6287) folded in. Workgroup: 8 output rows. y
// (the bf16-rounded silu * up * weight of the gate/up launch, inter floats)
// is loaded first, 8 consecutive values per thread of each 2048-column
// block, then the rows (lane: group g of 32 columns of tile row h rpp +
// lane / GP); the requant (amax over 16 neighbouring lanes) writes the E4M3
// grid values and scales into LDS while the rows stream; then each lane's
// sequential fmaf partial and one lane per row chains the groups in order;
// out[r] = bf16(acc). inter <= 4096, a multiple of 128.
template <int RPW>  // output rows per workgroup: 8 or 16
__global__ __launch_bounds__(256) void k_expert_down(float *__restrict__ out,
                                                     const float *__restrict__ y,
                                                     const uint8_t *__restrict__ W2,
                                                     const uint8_t *__restrict__ S2, int H,
                                                     int I) {
  __shared__ __align__(16) float xq[4096];
  __shared__ float xs[32];
  __shared__ __align__(16) float2 ps[RPW * 130];
  const int tid = threadIdx.x, r0 = blockIdx.x * RPW;
  const int G = I / 32;
  int GP = 1;
  while (GP < G) GP <<= 1;
  const int rpp = 256 / GP, g = tid % GP, rsub = tid / GP;
  const int stride = pair_stride(G);
  const BufRsrc ry = buf_rsrc(y, 4u * (uint32_t)I);
  uint4 yv[2][2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t base = 2048u * (uint32_t)b + 8u * (uint32_t)tid;
    yv[b][0] = buf_load16(ry, 4u * base);  // past I: zeros
    yv[b][1] = buf_load16(ry, 4u * base + 16u);
  }
  __builtin_amdgcn_sched_barrier(0);  // y ahead of the rows (loads return in order)
  const int nrow = max(0, min(RPW, H - r0));
  const BufRsrc rw = buf_rsrc(W2 + (size_t)r0 * (I / 2), (uint32_t)nrow * (uint32_t)(I / 2));
  const BufRsrc rs = buf_rsrc(S2 + (size_t)r0 * G, (uint32_t)nrow * (uint32_t)G);
  uint4 w[4];
  uint32_t code[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int lr = h * rpp + rsub;
    const bool in = lr < RPW && g < G;
    w[h] = buf_load16(rw, in ? (uint32_t)lr * (uint32_t)(I / 2) + 16u * g : 0xFFFFFFF0u);
    code[h] = __builtin_amdgcn_raw_buffer_load_b8(rs, in ? (uint32_t)(lr * G + g) : 0xFFFFFFF0u,
                                                  0, 0);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int base = 2048 * b + 8 * tid;
    const float v[8] = {u2f(yv[b][0].x), u2f(yv[b][0].y), u2f(yv[b][0].z), u2f(yv[b][0].w),
                        u2f(yv[b][1].x), u2f(yv[b][1].y), u2f(yv[b][1].z), u2f(yv[b][1].w)};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    if (base < I) {
      const float scale = act_scale(m);
      const float inv = 1.0f / scale;
#pragma unroll
      for (int i = 0; i < 8; ++i) xq[base + i] = quant_e4m3(v[i], inv);
      if ((tid & 15) == 0) xs[base / 128] = scale;
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int lr = h * rpp + rsub;
    if (lr < RPW && g < G) {
      float part = fp4_group_partial(w[h], xq + 32 * g);
      float s = xs[g / 4] * e8m0(code[h]);
      if (code[h] == 255u) {  // NaN scale: the reference skips the group
        part = 0.0f;
        s = 0.0f;
      }
      ps[lr * stride + g] = make_float2(part, s);
    }
  }
  __syncthreads();
  if (tid < nrow) out[r0 + tid] = bf16_round(pair_chain(ps + tid * stride, G));
}

}  // namespace dsv4

// ============================================================ C-ABI =====
using namespace dsv4;

extern "C" int dsv4g_layer_ok(const DSV4GLayer *L, const char *who) {
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

int dsv4g_router(int *idx, float *wt, const float *x, const DSV4GLayer *L,
                 const int *token_ids, int n_tokens, float *z_ws, float *zabs_ws,
                 void *stream) {
  DSV4G_TRY(dsv4g_layer_ok(L, "router"));
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

size_t dsv4g_expert_workspace_bytes(int inter) {
  return ((size_t)(3 * inter + (inter + 127) / 128) * 4 + 255) & ~(size_t)255;
}

// expert_forward (src/dsv4/dsv4_model.c:6289-6345) as the reference composes
// it: the paired FP4 gate/up GEMV, routed_swiglu_quant and the FP4 down GEMV,
// three launches on the stream; the slot layout of expert_forward_l1/_l2
// (scales [s1 | s2 | s3] at slot, weights [w1 | w2 | w3] at slot + scale_run).
int dsv4g_expert_forward(float *out, const float *qx, const float *qscale, const uint8_t *slot,
                         size_t scale_run, int hidden, int inter, float swiglu_limit,
                         const float *weight, void *workspace, size_t workspace_bytes,
                         void *stream) {
  if (!out || !qx || !qscale || !slot || hidden <= 0 || inter <= 0 || inter % 128 ||
      hidden % 32)
    return dsv4g_fail(DSV4G_EINVAL, "expert_forward: bad arguments");
  if (!workspace || workspace_bytes < dsv4g_expert_workspace_bytes(inter) ||
      ((uintptr_t)workspace & 255))
    return dsv4g_fail(DSV4G_EINVAL, "expert_forward: workspace too small or unaligned");
  const size_t H = (size_t)hidden, I = (size_t)inter;
  const uint8_t *sc = slot, *wt = slot + scale_run;
  const uint8_t *w1 = wt, *w2 = wt + I * (H / 2), *w3 = w2 + H * (I / 2);
  const uint8_t *s1 = sc, *s2 = sc + I * (H / 32), *s3 = s2 + H * (I / 32);
  float *ws = (float *)workspace;
  float *gate = ws, *up = ws + I, *qy = ws + 2 * I, *qys = ws + 3 * I;
  if (inter <= 4096 && hidden <= 8192) {
    // two launches: the paired gate/up tiles with the SwiGLU epilogue (y =
    // bf16(silu(gate) * up * weight) into the workspace), then the down rows
    // with the requant folded in (k_expert_down)
    GemvArgs a = {};
    a.W[0] = w1;
    a.S[0] = s1;
    a.W[1] = w3;
    a.S[1] = s3;
    a.qx = qx;
    a.qscale = qscale;
    a.in = hidden;
    a.rows = inter;
    a.y_stride = I;
    a.swi_y = ws;
    a.swi_w = weight;
    // the reference passes the limit as int (src/dsv4/dsv4_model.c:6297)
    a.swi_limit = (float)(int)swiglu_limit;
    a.np = 4;  // 4 rows of each matrix per tile: 512 tiles (measured: 14.0 us at the model's
               // shape, against 14.9 with 1024 tiles of 2 rows and 14.2 with 256 of 8)
    DSV4G_TRY(dsv4g_launch_gemv_fp4(&a, 1, 2, stream));
    // 16 rows per workgroup where a thread's four pieces cover them (inter <=
    // 2048): half the workgroups reading y
    if (inter <= 2048)
      hipLaunchKernelGGL(k_expert_down<16>, dim3((unsigned)((hidden + 15) / 16)), dim3(256), 0,
                         (hipStream_t)stream, out, ws, w2, s2, hidden, inter);
    else
      hipLaunchKernelGGL(k_expert_down<8>, dim3((unsigned)((hidden + 7) / 8)), dim3(256), 0,
                         (hipStream_t)stream, out, ws, w2, s2, hidden, inter);
    return dsv4g_check_launch("expert_down");
  }
  DSV4G_TRY(dsv4g_gemv_fp4_pair_q(gate, up, qx, qscale, w1, s1, w3, s3, hidden, inter, stream));
  // the reference passes the limit as int (src/dsv4/dsv4_model.c:6297)
  DSV4G_TRY(dsv4g_swiglu_quant(qy, qys, gate, weight, 0, 1, inter, (float)(int)swiglu_limit,
                               stream));
  return dsv4g_gemv_fp4_q(out, qy, qys, w2, s2, inter, hidden, stream);
}

int dsv4g_swiglu_quant(float *qy, float *qys, const float *gate_up, const float *wt, int K,
                       int n_slots, int inter, float limit, void *stream) {
  if (inter <= 0 || inter % 128 || n_slots <= 0 || K < 0)
    return dsv4g_fail(DSV4G_EINVAL, "swiglu_quant: bad size");
  hipLaunchKernelGGL(k_swiglu_quant, dim3(inter / 128, n_slots), dim3(64), 0,
                     (hipStream_t)stream, qy, qys, gate_up, wt, K, inter, limit);
  return dsv4g_check_launch("swiglu_quant");
}

}  // extern "C"
