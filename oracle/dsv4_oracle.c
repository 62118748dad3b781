/* dsv4_oracle.c - CPU oracle (checker) for the quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py; never linked into the product library.
 *
 * Each function restates one reference routine in its scalar loop order; the
 * citation above each function names the reference lines it follows. Build
 * with -ffp-contract=off (oracle/Makefile) so the explicit fmaf() calls are the
 * only fused operations, as in the reference build (GNUmakefile:48).
 * OpenMP only splits independent output rows; every row keeps its scalar
 * accumulation order, so results do not depend on the thread count
 * (src/dsv4/dsv4_model.c:584, 1106).
 */
#include "dsv4_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORC_FP8_BLOCK 128 /* src/dsv4/dsv4_internal.h:28 */
#define ORC_FP4_GROUP 32  /* src/dsv4/dsv4_internal.h:29 */
#define ORC_MAX_BATCH 33  /* DSV4_MAX_TOPK + 1, src/dsv4/dsv4_model.c:689 */

static void *orc_alloc(size_t bytes)
{
    void *p = malloc(bytes ? bytes : 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory (%zu bytes)\n", bytes);
        exit(1);
    }
    return p;
}

/* ------------------------------------------------------------- decode ---- */

/* RNE narrowing by integer bias, no NaN special case
 * (src/dsv4/dsv4_ops.c:35-44). */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t bits;
    memcpy(&bits, &f, 4);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

/* Widening is a shift (include/dsv4/dsv4.h:176-181). */
float orc_bf16_to_f32(uint16_t h)
{
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32bf(): narrow then widen (src/dsv4/dsv4_internal.h:254). */
float orc_bf16_round(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* OCP E4M3FN decode (src/dsv4/dsv4_ops.c:47-61): exponent field 0 is
 * man * 2^-9, S.1111.111 is NaN, otherwise (8 + man) * 2^(exp - 10). */
float orc_fp8_e4m3(uint8_t code)
{
    int e = (code >> 3) & 15, man = code & 7;
    float mag;
    if (e == 0)
        mag = ldexpf((float)man, -9);
    else if (e == 15 && man == 7)
        mag = NAN;
    else
        mag = ldexpf((float)(8 + man), e - 10);
    return (code & 0x80) ? -mag : mag;
}

/* E8M0 2^(code-127); 255 decodes to NaN (src/dsv4/dsv4_ops.c:63-67). */
float orc_e8m0(uint8_t code)
{
    return code == 255 ? NAN : ldexpf(1.0f, (int)code - 127);
}

/* E2M1 nibble: bit 3 is the sign, -0.0 kept (src/dsv4/dsv4_model.c:971-974). */
float orc_fp4_e2m1(uint8_t nibble)
{
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = mag[nibble & 7];
    return (nibble & 8) ? -v : v;
}

/* Ties-to-even on the integer grid (src/dsv4/dsv4_ops.c:81-90). */
static float orc_round_half_even(float x)
{
    float lo = floorf(x);
    float frac = x - lo;
    if (frac > 0.5f) return lo + 1.0f;
    if (frac < 0.5f) return lo;
    return fmodf(lo, 2.0f) == 0.0f ? lo : lo + 1.0f;
}

/* Nearest E4M3 grid value (src/dsv4/dsv4_ops.c:93-109): normal branch for
 * frexp exponent >= -5 with a 3-bit mantissa, overflow to +-448, subnormal
 * step 2^-9 that may carry into the smallest normal. */
float orc_round_e4m3(float v)
{
    if (v == 0.0f) return 0.0f;
    const float sign = v < 0 ? -1.0f : 1.0f;
    const float a = fabsf(v);
    int e;
    float m = frexpf(a, &e);
    if (e >= -5) {
        float mr = orc_round_half_even(m * 16.0f) / 16.0f;
        if (mr >= 1.0f) {
            mr = 0.5f;
            e++;
        }
        if (e - 1 > 8) return sign * 448.0f;
        return sign * mr * ldexpf(1.0f, e);
    }
    return sign * (orc_round_half_even(a * 512.0f) / 512.0f);
}

/* Power-of-two scale 2^ceil(log2(amax/448)) with the 1e-4 amax floor
 * (src/dsv4/dsv4_model.c:5590-5596). */
static float orc_act_scale(float amax)
{
    if (amax < 1e-4f) amax = 1e-4f;
    float r = amax * (1.0f / 448.0f);
    int e;
    float m = frexpf(r, &e);
    if (m == 0.5f) e--;
    return ldexpf(1.0f, e);
}

/* dsv4_quant_fp8_codes (src/dsv4/dsv4_model.c:5580-5606); identical to the
 * public dsv4_quant_fp8_act (src/dsv4/dsv4_ops.c:122-146). */
void orc_quant_fp8_act(float *qx, float *qscale, const float *x, int n)
{
    for (int base = 0; base < n; base += ORC_FP8_BLOCK) {
        int len = n - base < ORC_FP8_BLOCK ? n - base : ORC_FP8_BLOCK;
        float amax = 0.0f;
        for (int i = 0; i < len; i++)
            if (fabsf(x[base + i]) > amax) amax = fabsf(x[base + i]);
        float scale = orc_act_scale(amax);
        qscale[base / ORC_FP8_BLOCK] = scale;
        float inv = 1.0f / scale;
        for (int i = 0; i < len; i++) {
            float q = x[base + i] * inv;
            if (q > 448.0f) q = 448.0f;
            else if (q < -448.0f) q = -448.0f;
            qx[base + i] = orc_round_e4m3(q);
        }
    }
}

/* --------------------------------------------------------------- GEMVs ---- */

/* dsv4_gemv_bf16 scalar row (src/dsv4/dsv4_model.c:298-303): one fmaf chain
 * over the columns in order. */
static float orc_bf16_row(const uint16_t *wrow, const float *x, int in)
{
    float acc = 0.0f;
    for (int c = 0; c < in; c++) acc = fmaf(orc_bf16_to_f32(wrow[c]), x[c], acc);
    return acc;
}

void orc_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                   int round_out)
{
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < out; r++) {
        float acc = orc_bf16_row(W + (size_t)r * in, x, in);
        y[r] = round_out ? orc_bf16_round(acc) : acc;
    }
}

/* dsv4_gemv_bf16_batch is bit-identical to repeated single GEMVs
 * (src/dsv4/dsv4_model.c:348-366). */
void orc_gemv_bf16_batch(float *y, const float *x, int batch, const uint16_t *W,
                         int in, int out, int round_out)
{
    for (int t = 0; t < batch; t++)
        orc_gemv_bf16(y + (size_t)t * out, x + (size_t)t * in, W, in, out,
                      round_out);
}

/* One FP8 row (src/dsv4/dsv4_model.c:651-673): a 128-column fmaf partial,
 * then acc = fmaf(partial, qscale[cb] * e8m0(S[rb][cb]), acc); NaN scale
 * blocks are skipped. */
static float orc_fp8_row(const uint8_t *wrow, const uint8_t *srow,
                         const float *qx, const float *qscale, int in)
{
    const int cblocks = (in + ORC_FP8_BLOCK - 1) / ORC_FP8_BLOCK;
    float acc = 0.0f;
    for (int cb = 0; cb < cblocks; cb++) {
        int c0 = cb * ORC_FP8_BLOCK;
        int c1 = c0 + ORC_FP8_BLOCK < in ? c0 + ORC_FP8_BLOCK : in;
        float partial = 0.0f;
        for (int c = c0; c < c1; c++)
            partial = fmaf(orc_fp8_e4m3(wrow[c]), qx[c], partial);
        float ws = orc_e8m0(srow[cb]);
        if (!isnan(ws)) acc = fmaf(partial, qscale[cb] * ws, acc);
    }
    return acc;
}

void orc_gemv_fp8_q(float *y, const float *qx, const float *qscale,
                    const uint8_t *W, const uint8_t *S, int in, int out,
                    int round_out)
{
    const int cblocks = (in + ORC_FP8_BLOCK - 1) / ORC_FP8_BLOCK;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < out; r++) {
        float acc = orc_fp8_row(W + (size_t)r * in,
                                S + (size_t)(r / ORC_FP8_BLOCK) * cblocks,
                                qx, qscale, in);
        y[r] = round_out ? orc_bf16_round(acc) : acc;
    }
}

/* dsv4_gemv_fp8_batch_q (src/dsv4/dsv4_model.c:779-806): per-token partials
 * in the single-token order; exits above 33 tokens (:689-693). */
void orc_gemv_fp8_batch_q(float *y, const float *qx, const float *qscale,
                          int batch, const uint8_t *W, const uint8_t *S,
                          int in, int out, int round_out)
{
    if (batch > ORC_MAX_BATCH) {
        fprintf(stderr, "oracle: FP8 batch %d exceeds %d\n", batch, ORC_MAX_BATCH);
        exit(1);
    }
    const int qn = (in + ORC_FP8_BLOCK - 1) / ORC_FP8_BLOCK;
    for (int t = 0; t < batch; t++)
        orc_gemv_fp8_q(y + (size_t)t * out, qx + (size_t)t * in,
                       qscale + (size_t)t * qn, W, S, in, out, round_out);
}

/* dsv4_gemv_fp8_pair_q (src/dsv4/dsv4_model.c:938-961): two GEMVs sharing
 * qx, both BF16-rounded. */
void orc_gemv_fp8_pair_q(float *y0, float *y1, const float *qx,
                         const float *qscale, const uint8_t *W0,
                         const uint8_t *S0, const uint8_t *W1,
                         const uint8_t *S1, int in, int out)
{
    orc_gemv_fp8_q(y0, qx, qscale, W0, S0, in, out, 1);
    orc_gemv_fp8_q(y1, qx, qscale, W1, S1, in, out, 1);
}

/* One FP4 row (src/dsv4/dsv4_model.c:1049-1074): per 32-column group an
 * fmaf partial over decoded nibbles (low nibble = even column), then
 * acc = fmaf(partial, qscale[c0/128] * e8m0(S[r][g]), acc); output BF16. */
static float orc_fp4_row(const uint8_t *wrow, const uint8_t *srow,
                         const float *qx, const float *qscale, int in)
{
    float acc = 0.0f;
    for (int c0 = 0; c0 < in; c0 += ORC_FP4_GROUP) {
        int c1 = c0 + ORC_FP4_GROUP < in ? c0 + ORC_FP4_GROUP : in;
        float partial = 0.0f;
        for (int c = c0; c < c1; c++) {
            uint8_t b = wrow[c >> 1];
            uint8_t nib = (c & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
            partial = fmaf(orc_fp4_e2m1(nib), qx[c], partial);
        }
        float ws = orc_e8m0(srow[c0 / ORC_FP4_GROUP]);
        if (!isnan(ws)) acc = fmaf(partial, qscale[c0 / ORC_FP8_BLOCK] * ws, acc);
    }
    return acc;
}

void orc_gemv_fp4_q(float *y, const float *qx, const float *qscale,
                    const uint8_t *W, const uint8_t *S, int in, int rows)
{
    const size_t pcols = (size_t)(in + 1) / 2;
    const size_t gcols = (size_t)(in + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        y[r] = orc_bf16_round(
            orc_fp4_row(W + r * pcols, S + r * gcols, qx, qscale, in));
}

/* dsv4_gemv_fp4_batch_q (src/dsv4/dsv4_model.c:1188-1217). */
void orc_gemv_fp4_batch_q(float *y, const float *qx, const float *qscale,
                          int batch, const uint8_t *W, const uint8_t *S,
                          int in, int rows)
{
    if (batch > ORC_MAX_BATCH) {
        fprintf(stderr, "oracle: FP4 batch %d exceeds %d\n", batch, ORC_MAX_BATCH);
        exit(1);
    }
    const int qn = (in + ORC_FP8_BLOCK - 1) / ORC_FP8_BLOCK;
    for (int t = 0; t < batch; t++)
        orc_gemv_fp4_q(y + (size_t)t * rows, qx + (size_t)t * in,
                       qscale + (size_t)t * qn, W, S, in, rows);
}

/* dsv4_gemv_fp4_pair_q (src/dsv4/dsv4_model.c:1352-1380). */
void orc_gemv_fp4_pair_q(float *y0, float *y1, const float *qx,
                         const float *qscale, const uint8_t *W0,
                         const uint8_t *S0, const uint8_t *W1,
                         const uint8_t *S1, int in, int rows)
{
    orc_gemv_fp4_q(y0, qx, qscale, W0, S0, in, rows);
    orc_gemv_fp4_q(y1, qx, qscale, W1, S1, in, rows);
}

/* Public float-scale FP8 GEMV dsv4_gemv_fp8 (src/dsv4/dsv4_ops.c:176-207):
 * xs[c] = x[c] * s(rb, cb), then one unfused mul+add chain over all columns. */
void orc_gemv_fp8_legacy(float *y, const float *x, const uint8_t *W,
                         const float *wscale, int in, int rows, int block)
{
    const int rblocks = (rows + block - 1) / block;
    const int cblocks = (in + block - 1) / block;
    float *xs = (float *)orc_alloc((size_t)in * sizeof(float));
    for (int rb = 0; rb < rblocks; rb++) {
        for (int c = 0; c < in; c++)
            xs[c] = x[c] * wscale[(size_t)rb * cblocks + c / block];
        int r1 = (rb + 1) * block < rows ? (rb + 1) * block : rows;
        #pragma omp parallel for schedule(static)
        for (int r = rb * block; r < r1; r++) {
            const uint8_t *wrow = W + (size_t)r * in;
            float acc = 0.0f;
            for (int c = 0; c < in; c++) {
                float prod = orc_fp8_e4m3(wrow[c]) * xs[c];
                acc = acc + prod;
            }
            y[r] = acc;
        }
    }
    free(xs);
}

/* dsv4_gemv_fp8_tbl (src/dsv4/dsv4_ops.c:214-239): acc += (w * x) * s, left
 * to right, unfused. */
void orc_gemv_fp8_tbl(float *y, const float *x, const uint8_t *W,
                      const float *wscale, int in, int rows, int block)
{
    const int cblocks = (in + block - 1) / block;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const uint8_t *wrow = W + (size_t)r * in;
        const float *srow = wscale + (size_t)(r / block) * cblocks;
        float acc = 0.0f;
        for (int c = 0; c < in; c++) {
            float t = orc_fp8_e4m3(wrow[c]) * x[c];
            t = t * srow[c / block];
            acc = acc + t;
        }
        y[r] = acc;
    }
}

/* Public float-scale FP4 GEMV dsv4_gemv_fp4 (src/dsv4/dsv4_ops.c:249-284):
 * xd = qx * qscale once, then acc += (w * xd) * wscale, unfused. */
void orc_gemv_fp4_legacy(float *y, const float *qx, const float *qscale,
                         const uint8_t *W, const float *wscale, int in,
                         int rows, int group)
{
    const size_t pcols = (size_t)(in + 1) / 2;
    const size_t gcols = (size_t)(in + group - 1) / group;
    float *xd = (float *)orc_alloc((size_t)in * sizeof(float));
    for (int c = 0; c < in; c++) xd[c] = qx[c] * qscale[c / 128];
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const uint8_t *wrow = W + r * pcols;
        float acc = 0.0f;
        for (int c = 0; c < in; c++) {
            uint8_t b = wrow[c >> 1];
            uint8_t nib = (c & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
            float t = orc_fp4_e2m1(nib) * xd[c];
            t = t * wscale[r * gcols + c / group];
            acc = acc + t;
        }
        y[r] = acc;
    }
    free(xd);
}

/* -------------------------------------------------------------- router ---- */

/* src/dsv4/dsv4_model.c:5827-5831 (and src/dsv4/dsv4_ops.c:466-470). */
float orc_sqrt_softplus(float z)
{
    if (z > 20.0f) return sqrtf(z);
    return sqrtf(log1pf(expf(z)));
}

/* The exchange sort both routers use to order experts ascending while
 * carrying weights (src/dsv4/dsv4_model.c:6666-6674). */
static void orc_sort_routes(int *idx, float *wt, int topk)
{
    for (int i = 0; i < topk; i++)
        for (int j = i + 1; j < topk; j++)
            if (idx[j] < idx[i]) {
                int ti = idx[i];
                idx[i] = idx[j];
                idx[j] = ti;
                float tw = wt[i];
                wt[i] = wt[j];
                wt[j] = tw;
            }
}

/* Biased top-k by repeated strict-'>' maximum (lowest id wins ties), hash
 * lookup on hash layers, weights from the UNBIASED scores times
 * route_scale/sum, then ascending-id order (src/dsv4/dsv4_model.c:6627-6676). */
void orc_route(int *idx, float *wt, const float *z, const float *bias,
               const int64_t *tid2eid_row, int n_experts, int topk,
               float route_scale)
{
    float *score = (float *)orc_alloc((size_t)n_experts * sizeof(float));
    float *choice = (float *)orc_alloc((size_t)n_experts * sizeof(float));
    for (int e = 0; e < n_experts; e++) score[e] = orc_sqrt_softplus(z[e]);
    for (int e = 0; e < n_experts; e++)
        choice[e] = score[e] + (bias ? bias[e] : 0.0f);
    if (tid2eid_row) {
        for (int k = 0; k < topk; k++) idx[k] = (int)tid2eid_row[k];
    } else {
        for (int k = 0; k < topk; k++) {
            int best = -1;
            float bv = -INFINITY;
            for (int e = 0; e < n_experts; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++) taken |= idx[j] == e;
                if (!taken && choice[e] > bv) {
                    bv = choice[e];
                    best = e;
                }
            }
            idx[k] = best;
        }
    }
    float sum = 0.0f;
    for (int k = 0; k < topk; k++) sum += idx[k] >= 0 ? score[idx[k]] : 0.0f;
    if (sum > 0.0f) {
        float rs = route_scale / sum;
        for (int k = 0; k < topk; k++)
            wt[k] = idx[k] >= 0 ? score[idx[k]] * rs : 0.0f;
    } else {
        for (int k = 0; k < topk; k++) wt[k] = 0.0f;
    }
    orc_sort_routes(idx, wt, topk);
    free(score);
    free(choice);
}

/* Public dsv4_router (src/dsv4/dsv4_ops.c:473-545): z by unfused mul+add,
 * weights = (score * (1/sum)) * route_scale. On hash layers the expert list
 * is tid2eid's row and only those experts are scored. */
void orc_router_public(int *idx, float *wt, const float *x,
                       const uint16_t *gate, const float *bias,
                       const int64_t *tid2eid, int token_id, int hidden,
                       int n_experts, int topk, int hash_layer,
                       float route_scale)
{
    float *score = (float *)orc_alloc((size_t)n_experts * sizeof(float));
    float *choice = (float *)orc_alloc((size_t)n_experts * sizeof(float));
    int order[64];
    for (int e = 0; e < n_experts; e++) score[e] = choice[e] = 0.0f;
    for (int e = 0; e < n_experts; e++) {
        if (hash_layer) {
            int chosen = 0;
            for (int k = 0; k < topk; k++)
                chosen |= (int)tid2eid[(size_t)token_id * topk + k] == e;
            if (!chosen) continue;
        }
        const uint16_t *grow = gate + (size_t)e * hidden;
        float zz = 0.0f;
        for (int i = 0; i < hidden; i++) {
            float prod = orc_bf16_to_f32(grow[i]) * x[i];
            zz = zz + prod;
        }
        score[e] = orc_sqrt_softplus(zz);
        choice[e] = score[e] + (bias ? bias[e] : 0.0f);
    }
    if (hash_layer) {
        for (int k = 0; k < topk; k++)
            order[k] = (int)tid2eid[(size_t)token_id * topk + k];
    } else {
        for (int k = 0; k < topk; k++) {
            int best = -1;
            float bv = -INFINITY;
            for (int e = 0; e < n_experts; e++) {
                int taken = 0;
                for (int j = 0; j < k; j++) taken |= order[j] == e;
                if (!taken && choice[e] > bv) {
                    bv = choice[e];
                    best = e;
                }
            }
            order[k] = best;
        }
    }
    float sum = 0.0f;
    for (int k = 0; k < topk; k++) sum += order[k] >= 0 ? score[order[k]] : 0.0f;
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int k = 0; k < topk; k++) {
        float t = (order[k] >= 0 ? score[order[k]] : 0.0f) * inv;
        wt[k] = t * route_scale;
    }
    orc_sort_routes(order, wt, topk);
    for (int k = 0; k < topk; k++) idx[k] = order[k];
    free(score);
    free(choice);
}

/* -------------------------------------------------------------- expert ---- */

/* routed_swiglu_quant (src/dsv4/dsv4_model.c:6261-6287): clamp up to
 * [-limit, limit], gate to <= limit, y = bf16((silu(g) * u) * w), then the
 * per-128 FP8 requant of y. */
void orc_swiglu_quant(float *y, float *qy, float *qys, const float *gate,
                      const float *up, int n, int limit, float route_weight)
{
    for (int base = 0; base < n; base += ORC_FP8_BLOCK) {
        int len = n - base < ORC_FP8_BLOCK ? n - base : ORC_FP8_BLOCK;
        float amax = 0.0f;
        for (int i = 0; i < len; i++) {
            float g = gate[base + i], u = up[base + i];
            if (u > limit) u = (float)limit;
            else if (u < -limit) u = (float)(-limit);
            if (g > limit) g = (float)limit;
            float silu = g / (1.0f + expf(-g));
            float t = silu * u;
            y[base + i] = orc_bf16_round(t * route_weight);
            if (fabsf(y[base + i]) > amax) amax = fabsf(y[base + i]);
        }
        float scale = orc_act_scale(amax);
        qys[base / ORC_FP8_BLOCK] = scale;
        float inv = 1.0f / scale;
        for (int i = 0; i < len; i++) {
            float q = y[base + i] * inv;
            if (q > 448.0f) q = 448.0f;
            else if (q < -448.0f) q = -448.0f;
            qy[base + i] = orc_round_e4m3(q);
        }
    }
}

/* expert_forward_l1/l2 (src/dsv4/dsv4_model.c:6289-6345): slot offsets
 * w1 @0, w2 @inter*hidden/2, w3 after w2; scales likewise per 32 columns. */
void orc_expert_forward(float *out, const float *qx, const float *qsc,
                        const uint8_t *scales, const uint8_t *weights,
                        int hidden, int inter, int limit, float route_weight)
{
    const size_t w1_bytes = (size_t)inter * ((hidden + 1) / 2);
    const size_t w2_bytes = (size_t)hidden * ((inter + 1) / 2);
    const size_t s1_bytes = (size_t)inter * ((hidden + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP);
    const size_t s2_bytes = (size_t)hidden * ((inter + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP);
    float *work = (float *)orc_alloc((size_t)(4 * inter + (inter + 127) / 128) * sizeof(float));
    float *gate = work, *up = work + inter, *y = work + 2 * inter;
    float *qy = work + 3 * inter, *qys = work + 4 * inter;
    orc_gemv_fp4_pair_q(gate, up, qx, qsc, weights, scales,
                        weights + w1_bytes + w2_bytes, scales + s1_bytes + s2_bytes,
                        hidden, inter);
    orc_swiglu_quant(y, qy, qys, gate, up, inter, limit, route_weight);
    orc_gemv_fp4_q(out, qy, qys, weights + w1_bytes, scales + s1_bytes, inter,
                   hidden);
    free(work);
}

/* shared_expert_forward (src/dsv4/dsv4_model.c:6399-6433): FP8 pair GEMV,
 * SwiGLU with weight 1, BF16 round, FP8 requant, FP8 down with BF16 out. */
void orc_shared_expert_forward(float *out, const float *qx, const float *qsc,
                               const uint8_t *sh1, const uint8_t *sh1_s,
                               const uint8_t *sh3, const uint8_t *sh3_s,
                               const uint8_t *sh2, const uint8_t *sh2_s,
                               int hidden, int inter, int limit)
{
    float *work = (float *)orc_alloc((size_t)(4 * inter + (inter + 127) / 128) * sizeof(float));
    float *gate = work, *up = work + inter, *y = work + 2 * inter;
    float *qy = work + 3 * inter, *qys = work + 4 * inter;
    orc_gemv_fp8_pair_q(gate, up, qx, qsc, sh1, sh1_s, sh3, sh3_s, hidden, inter);
    orc_swiglu_quant(y, qy, qys, gate, up, inter, limit, 1.0f);
    orc_gemv_fp8_q(out, qy, qys, sh2, sh2_s, inter, hidden, 1);
    free(work);
}

/* ----------------------------------------------------------- MoE layer ---- */

static void orc_layer_expert(const OrcLayer *L, int e, const uint8_t **scales,
                             const uint8_t **weights)
{
    *scales = L->experts + (size_t)e * L->expert_stride;
    *weights = *scales + L->scale_run;
}

/* moe_forward (src/dsv4/dsv4_model.c:6599-6807): BF16 gate GEMV, routing,
 * activation quant, routed experts in ascending id + shared expert, then
 * acc = ((0 + r0) + ... + r_{k-1}) + shared, BF16-rounded. */
void orc_moe_forward(const OrcLayer *L, const float *x, int token_id,
                     float *out, int *idx_out, float *wt_out)
{
    const int H = L->hidden, K = L->topk;
    const int limit = (int)L->swiglu_limit;
    float *z = (float *)orc_alloc((size_t)L->n_experts * sizeof(float));
    float *qx = (float *)orc_alloc((size_t)H * sizeof(float));
    float *qsc = (float *)orc_alloc((size_t)((H + 127) / 128) * sizeof(float));
    float *routed = (float *)orc_alloc((size_t)(K + 1) * H * sizeof(float));
    int idx[64];
    float wt[64];
    orc_gemv_bf16(z, x, L->gate_w, H, L->n_experts, 0);
    orc_route(idx, wt, z, L->bias,
              L->is_hash ? L->tid2eid + (size_t)token_id * K : NULL,
              L->n_experts, K, L->route_scale);
    orc_quant_fp8_act(qx, qsc, x, H);
    for (int k = 0; k < K; k++) {
        const uint8_t *s, *w;
        orc_layer_expert(L, idx[k], &s, &w);
        orc_expert_forward(routed + (size_t)k * H, qx, qsc, s, w, H, L->inter,
                           limit, wt[k]);
    }
    float *shared = routed + (size_t)K * H;
    orc_shared_expert_forward(shared, qx, qsc, L->sh1, L->sh1_s, L->sh3,
                              L->sh3_s, L->sh2, L->sh2_s, H, L->inter, limit);
    for (int i = 0; i < H; i++) {
        float acc = 0.0f;
        for (int k = 0; k < K; k++) acc += routed[(size_t)k * H + i];
        acc += shared[i];
        out[i] = orc_bf16_round(acc);
    }
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int));
    if (wt_out) memcpy(wt_out, wt, (size_t)K * sizeof(float));
    free(z);
    free(qx);
    free(qsc);
    free(routed);
}

/* The router of moe_forward / moe_forward_batch for n tokens at once
 * (src/dsv4/dsv4_model.c:6615-6676, 6865-6906): per token the BF16 gate GEMV
 * and orc_route, tokens spread over OpenMP threads. idx, wt: [n][topk]. */
void orc_route_tokens(const OrcLayer *L, const float *x, const int *token_ids,
                      int n_tokens, int *idx, float *wt)
{
    const int H = L->hidden, E = L->n_experts, K = L->topk;
    #pragma omp parallel
    {
        float *z = (float *)orc_alloc((size_t)E * sizeof(float));
        #pragma omp for schedule(dynamic, 4)
        for (int t = 0; t < n_tokens; t++) {
            const float *xt = x + (size_t)t * H;
            for (int e = 0; e < E; e++)
                z[e] = orc_bf16_row(L->gate_w + (size_t)e * H, xt, H);
            orc_route(idx + (size_t)t * K, wt + (size_t)t * K, z, L->bias,
                      L->is_hash ? L->tid2eid + (size_t)token_ids[t] * K : NULL,
                      E, K, L->route_scale);
        }
        free(z);
    }
}

/* The per-route expert outputs of moe_forward before their BF16 rounding:
 * routes[k] = the down GEMV accumulators of route k (ascending expert id, as
 * moe_forward visits them), routes[K] those of the shared expert. The
 * reference rounds each to BF16 (dsv4_gemv_fp4_q, src/dsv4/dsv4_model.c:1073;
 * dsv4_gemv_fp8_q with round_out = 1, :6433), and bf16(routes) are the
 * outputs orc_moe_forward sums. idx, wt: the routing (optional). */
void orc_moe_route_outputs(const OrcLayer *L, const float *x, int token_id,
                           float *routes, int *idx_out, float *wt_out)
{
    const int H = L->hidden, I = L->inter, K = L->topk;
    const int limit = (int)L->swiglu_limit;
    const int qn = (H + 127) / 128;
    float *z = (float *)orc_alloc((size_t)L->n_experts * sizeof(float));
    float *qx = (float *)orc_alloc((size_t)H * sizeof(float));
    float *qsc = (float *)orc_alloc((size_t)qn * sizeof(float));
    float *work = (float *)orc_alloc((size_t)(4 * I + (I + 127) / 128) * sizeof(float));
    float *gate = work, *up = work + I, *y = work + 2 * I, *qy = work + 3 * I;
    float *qys = work + 4 * I;
    int idx[64];
    float wt[64];
    orc_gemv_bf16(z, x, L->gate_w, H, L->n_experts, 0);
    orc_route(idx, wt, z, L->bias,
              L->is_hash ? L->tid2eid + (size_t)token_id * K : NULL,
              L->n_experts, K, L->route_scale);
    orc_quant_fp8_act(qx, qsc, x, H);
    const size_t w1 = (size_t)I * ((H + 1) / 2), w2 = (size_t)H * ((I + 1) / 2);
    const size_t s1 = (size_t)I * ((H + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP);
    const size_t s2 = (size_t)H * ((I + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP);
    const size_t dpc = (size_t)(I + 1) / 2, dgc = (size_t)(I + ORC_FP4_GROUP - 1) / ORC_FP4_GROUP;
    for (int k = 0; k < K; k++) {
        float *r = routes + (size_t)k * H;
        if (idx[k] < 0 || idx[k] >= L->n_experts) {
            for (int i = 0; i < H; i++) r[i] = 0.0f;
            continue;
        }
        const uint8_t *s, *w;
        orc_layer_expert(L, idx[k], &s, &w);
        orc_gemv_fp4_pair_q(gate, up, qx, qsc, w, s, w + w1 + w2, s + s1 + s2, H, I);
        orc_swiglu_quant(y, qy, qys, gate, up, I, limit, wt[k]);
        #pragma omp parallel for schedule(static)
        for (int row = 0; row < H; row++)
            r[row] = orc_fp4_row(w + w1 + row * dpc, s + s1 + row * dgc, qy, qys, I);
    }
    orc_gemv_fp8_pair_q(gate, up, qx, qsc, L->sh1, L->sh1_s, L->sh3, L->sh3_s, H, I);
    orc_swiglu_quant(y, qy, qys, gate, up, I, limit, 1.0f);
    orc_gemv_fp8_q(routes + (size_t)K * H, qy, qys, L->sh2, L->sh2_s, I, H, 0);
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int));
    if (wt_out) memcpy(wt_out, wt, (size_t)K * sizeof(float));
    free(z);
    free(qx);
    free(qsc);
    free(work);
}

/* moe_forward_batch (src/dsv4/dsv4_model.c:6812-7117): route every token,
 * visit the distinct experts in ascending id, run each on its tokens in
 * chunks of topk+1 (expert_forward_batch_routes, :6486-6524) and add every
 * route output into its token's accumulator as the expert is visited, so each
 * token still sums its routes in ascending id; then + shared and BF16. */
void orc_moe_forward_batch(const OrcLayer *L, const float *x,
                           const int *token_ids, int n_tokens, float *out,
                           int *idx_out, float *wt_out)
{
    const int H = L->hidden, I = L->inter, K = L->topk, E = L->n_experts;
    const int qn = (H + 127) / 128, qin = (I + 127) / 128;
    const int limit = (int)L->swiglu_limit;
    const int chunk_cap = K + 1;
    float *z = (float *)orc_alloc((size_t)E * sizeof(float));
    float *qx = (float *)orc_alloc((size_t)n_tokens * H * sizeof(float));
    float *qsc = (float *)orc_alloc((size_t)n_tokens * qn * sizeof(float));
    int *idx = (int *)orc_alloc((size_t)n_tokens * K * sizeof(int));
    float *wt = (float *)orc_alloc((size_t)n_tokens * K * sizeof(float));
    float *acc = (float *)calloc((size_t)n_tokens * H, sizeof(float));
    float *shared = (float *)orc_alloc((size_t)n_tokens * H * sizeof(float));
    unsigned char *used = (unsigned char *)calloc((size_t)E, 1);
    /* chunk buffers */
    float *cqx = (float *)orc_alloc((size_t)chunk_cap * H * sizeof(float));
    float *cqs = (float *)orc_alloc((size_t)chunk_cap * qn * sizeof(float));
    float *gate = (float *)orc_alloc((size_t)chunk_cap * I * sizeof(float));
    float *up = (float *)orc_alloc((size_t)chunk_cap * I * sizeof(float));
    float *y = (float *)orc_alloc((size_t)I * sizeof(float));
    float *qy = (float *)orc_alloc((size_t)chunk_cap * I * sizeof(float));
    float *qys = (float *)orc_alloc((size_t)chunk_cap * qin * sizeof(float));
    float *cout = (float *)orc_alloc((size_t)chunk_cap * H * sizeof(float));
    if (!acc || !used) {
        fprintf(stderr, "oracle: out of memory\n");
        exit(1);
    }

    for (int t = 0; t < n_tokens; t++) {
        const float *xt = x + (size_t)t * H;
        orc_gemv_bf16(z, xt, L->gate_w, H, E, 0);
        orc_route(idx + (size_t)t * K, wt + (size_t)t * K, z, L->bias,
                  L->is_hash ? L->tid2eid + (size_t)token_ids[t] * K : NULL,
                  E, K, L->route_scale);
        for (int k = 0; k < K; k++) used[idx[(size_t)t * K + k]] = 1;
        orc_quant_fp8_act(qx + (size_t)t * H, qsc + (size_t)t * qn, xt, H);
    }

    /* shared expert over all tokens in chunks of topk+1
     * (shared_expert_forward_many, src/dsv4/dsv4_model.c:6435-6484) */
    for (int first = 0; first < n_tokens; first += chunk_cap) {
        int n = n_tokens - first < chunk_cap ? n_tokens - first : chunk_cap;
        orc_gemv_fp8_batch_q(gate, qx + (size_t)first * H, qsc + (size_t)first * qn,
                             n, L->sh1, L->sh1_s, H, I, 1);
        orc_gemv_fp8_batch_q(up, qx + (size_t)first * H, qsc + (size_t)first * qn,
                             n, L->sh3, L->sh3_s, H, I, 1);
        for (int t = 0; t < n; t++)
            orc_swiglu_quant(y, qy + (size_t)t * I, qys + (size_t)t * qin,
                             gate + (size_t)t * I, up + (size_t)t * I, I, limit,
                             1.0f);
        orc_gemv_fp8_batch_q(shared + (size_t)first * H, qy, qys, n, L->sh2,
                             L->sh2_s, I, H, 1);
    }

    const size_t w1_bytes = (size_t)I * ((H + 1) / 2);
    const size_t w2_bytes = (size_t)H * ((I + 1) / 2);
    const size_t s1_bytes = (size_t)I * ((H + 31) / 32);
    const size_t s2_bytes = (size_t)H * ((I + 31) / 32);
    for (int e = 0; e < E; e++) {
        if (!used[e]) continue;
        const uint8_t *s, *w;
        orc_layer_expert(L, e, &s, &w);
        int next = 0;
        while (next < n_tokens) {
            int tok[64], n = 0;
            float rw[64];
            while (next < n_tokens && n < chunk_cap) {
                int t = next++;
                for (int k = 0; k < K; k++)
                    if (idx[(size_t)t * K + k] == e) {
                        tok[n] = t;
                        rw[n] = wt[(size_t)t * K + k];
                        memcpy(cqx + (size_t)n * H, qx + (size_t)t * H, (size_t)H * sizeof(float));
                        memcpy(cqs + (size_t)n * qn, qsc + (size_t)t * qn, (size_t)qn * sizeof(float));
                        n++;
                        break;
                    }
            }
            if (n == 0) continue;
            /* expert_forward_many (src/dsv4/dsv4_model.c:6347-6396) */
            orc_gemv_fp4_batch_q(gate, cqx, cqs, n, w, s, H, I);
            orc_gemv_fp4_batch_q(up, cqx, cqs, n, w + w1_bytes + w2_bytes,
                                 s + s1_bytes + s2_bytes, H, I);
            for (int r = 0; r < n; r++)
                orc_swiglu_quant(y, qy + (size_t)r * I, qys + (size_t)r * qin,
                                 gate + (size_t)r * I, up + (size_t)r * I, I,
                                 limit, rw[r]);
            orc_gemv_fp4_batch_q(cout, qy, qys, n, w + w1_bytes, s + s1_bytes, I, H);
            for (int r = 0; r < n; r++) {
                float *ta = acc + (size_t)tok[r] * H;
                const float *eo = cout + (size_t)r * H;
                for (int i = 0; i < H; i++) ta[i] += eo[i];
            }
        }
    }
    for (int t = 0; t < n_tokens; t++) {
        float *ta = acc + (size_t)t * H;
        const float *ts = shared + (size_t)t * H;
        for (int i = 0; i < H; i++) out[(size_t)t * H + i] = orc_bf16_round(ta[i] + ts[i]);
    }
    if (idx_out) memcpy(idx_out, idx, (size_t)n_tokens * K * sizeof(int));
    if (wt_out) memcpy(wt_out, wt, (size_t)n_tokens * K * sizeof(float));
    free(z); free(qx); free(qsc); free(idx); free(wt); free(acc); free(shared);
    free(used); free(cqx); free(cqs); free(gate); free(up); free(y); free(qy);
    free(qys); free(cout);
}

/* ------------------------------------------ synthetic-weight quantizers ---- */
/* The reference ships no weight quantizer in C. These build synthetic
 * checkpoints in its formats: FP4 E2M1 with per-row per-32 E8M0 scales
 * 2^ceil(log2(amax/6)) and nearest-value rounding with ties to the even code
 * (the rule of src/dsv4/dsv4_model.c:1420-1447); FP8 E4M3 with per-128x128
 * E8M0 scales 2^ceil(log2(amax/448)) or fp32 absmax/448 scales. */

static int orc_pow2_ceil_exp(float r)
{
    int e;
    float m = frexpf(r, &e);
    if (m == 0.5f) e--;
    return e;
}

static uint8_t orc_fp4_code(float q)
{
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float a = fabsf(q);
    int best = 0;
    float bd = a;
    for (int k = 0; k < 8; k++) {
        float d = fabsf(a - mag[k]);
        if (d < bd) {
            bd = d;
            best = k;
        } else if (d == bd && (k & 1) == 0) {
            best = k;
        }
    }
    return (uint8_t)(best | (q < 0 ? 8 : 0));
}

void orc_quant_fp4_rows(uint8_t *packed, uint8_t *scale_codes, const float *w,
                        int rows, int cols)
{
    const int pcols = (cols + 1) / 2, gcols = (cols + 31) / 32;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *wr = w + (size_t)r * cols;
        uint8_t *pr = packed + (size_t)r * pcols;
        memset(pr, 0, (size_t)pcols);
        for (int g = 0; g < gcols; g++) {
            int c0 = g * 32, c1 = c0 + 32 < cols ? c0 + 32 : cols;
            float amax = 0.0f;
            for (int c = c0; c < c1; c++)
                if (fabsf(wr[c]) > amax) amax = fabsf(wr[c]);
            const float floor_amax = 6.0f * ldexpf(1.0f, -126);
            if (amax < floor_amax) amax = floor_amax;
            int e = orc_pow2_ceil_exp(amax * (1.0f / 6.0f));
            scale_codes[(size_t)r * gcols + g] = (uint8_t)(e + 127);
            float inv = 1.0f / ldexpf(1.0f, e);
            for (int c = c0; c < c1; c++) {
                float q = wr[c] * inv;
                if (q > 6.0f) q = 6.0f;
                else if (q < -6.0f) q = -6.0f;
                uint8_t nib = orc_fp4_code(q);
                pr[c >> 1] |= (uint8_t)((c & 1) ? nib << 4 : nib);
            }
        }
    }
}

/* Code of an E4M3 grid value as produced by orc_round_e4m3. */
uint8_t orc_e4m3_code(float v)
{
    uint8_t sign = (v < 0 || (v == 0.0f && signbit(v))) ? 0x80 : 0;
    float a = fabsf(v);
    if (a == 0.0f) return sign;
    if (a < ldexpf(1.0f, -6)) return (uint8_t)(sign | (int)(a * 512.0f));
    int e;
    float m = frexpf(a, &e);              /* a = m * 2^e, m in [0.5, 1) */
    int man = (int)(m * 16.0f) - 8;       /* 3 mantissa bits            */
    int ef = e - 1 + 7;                   /* biased exponent field      */
    return (uint8_t)(sign | (ef << 3) | man);
}

void orc_quant_fp8_blocks_e8m0(uint8_t *codes, uint8_t *scale_codes,
                               const float *w, int rows, int cols)
{
    const int rb = (rows + 127) / 128, cb = (cols + 127) / 128;
    #pragma omp parallel for schedule(static)
    for (int b = 0; b < rb * cb; b++) {
        int r0 = (b / cb) * 128, c0 = (b % cb) * 128;
        int r1 = r0 + 128 < rows ? r0 + 128 : rows;
        int c1 = c0 + 128 < cols ? c0 + 128 : cols;
        float amax = 0.0f;
        for (int r = r0; r < r1; r++)
            for (int c = c0; c < c1; c++)
                if (fabsf(w[(size_t)r * cols + c]) > amax) amax = fabsf(w[(size_t)r * cols + c]);
        if (amax < 1e-4f) amax = 1e-4f;
        int e = orc_pow2_ceil_exp(amax * (1.0f / 448.0f));
        scale_codes[b] = (uint8_t)(e + 127);
        float inv = 1.0f / ldexpf(1.0f, e);
        for (int r = r0; r < r1; r++)
            for (int c = c0; c < c1; c++) {
                float q = w[(size_t)r * cols + c] * inv;
                if (q > 448.0f) q = 448.0f;
                else if (q < -448.0f) q = -448.0f;
                codes[(size_t)r * cols + c] = orc_e4m3_code(orc_round_e4m3(q));
            }
    }
}

void orc_quant_fp8_blocks_absmax(uint8_t *codes, float *scales, const float *w,
                                 int rows, int cols)
{
    const int rb = (rows + 127) / 128, cb = (cols + 127) / 128;
    #pragma omp parallel for schedule(static)
    for (int b = 0; b < rb * cb; b++) {
        int r0 = (b / cb) * 128, c0 = (b % cb) * 128;
        int r1 = r0 + 128 < rows ? r0 + 128 : rows;
        int c1 = c0 + 128 < cols ? c0 + 128 : cols;
        float amax = 0.0f;
        for (int r = r0; r < r1; r++)
            for (int c = c0; c < c1; c++)
                if (fabsf(w[(size_t)r * cols + c]) > amax) amax = fabsf(w[(size_t)r * cols + c]);
        float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        scales[b] = s;
        for (int r = r0; r < r1; r++)
            for (int c = c0; c < c1; c++) {
                float q = w[(size_t)r * cols + c] / s;
                if (q > 448.0f) q = 448.0f;
                else if (q < -448.0f) q = -448.0f;
                codes[(size_t)r * cols + c] = orc_e4m3_code(orc_round_e4m3(q));
            }
    }
}

/* ------------------------------------------------ bench-protocol helpers ---- */

/* xorshift64 of benchmarks/bench_dsv4_kernels.c:25-32. */
uint64_t orc_xorshift_next(uint64_t *state)
{
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* sqrt(sum y^2) in double (benchmarks/bench_dsv4_kernels.c:41-47); the caller
 * narrows to float as the bench does. */
double orc_checksum(const float *v, int n)
{
    double s = 0.0;
    for (int i = 0; i < n; i++) s += (double)v[i] * v[i];
    return sqrt(s);
}

/* ------------------------------------------- caller step around the MoE ---- */

/* rmsnorm_bf16 (src/dsv4/dsv4_model.c:4934-4951): sum of squares in double,
 * in index order, each square formed from the widened floats; the scale
 * 1/sqrtf((float)(ss/n) + eps); y = x * r (* gain) evaluated left to right,
 * then BF16 when round_out. y may alias x. */
void orc_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps,
                      int round_out)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) {
        const double d = (double)x[i];
        ss += d * d;
    }
    const float r = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) {
        float v = x[i] * r;
        if (w) v = v * orc_bf16_to_f32(w[i]);
        y[i] = round_out ? orc_bf16_round(v) : v;
    }
}

/* the logistic function in its two overflow-free forms (src/dsv4/dsv4_ops.c:401-409) */
static float orc_sigmoid(float x)
{
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}

/* dsv4_hc_split (src/dsv4/dsv4_ops.c:415-466): mixes = [pre | post | comb]
 * sections of mult, mult, mult*mult; pre = sigmoid(m*s0 + b) + eps,
 * post = 2 sigmoid(m*s1 + b), comb = row softmax + eps, one column pass,
 * then iters-1 (row, column) passes; each pass divides by (sum + eps). */
void orc_hc_split(float *pre, float *post, float *comb, const float *mixes,
                  const float *scale3, const float *base, int mult, int iters, float eps)
{
    const int m = mult;
    for (int i = 0; i < m; i++) {
        pre[i] = orc_sigmoid(mixes[i] * scale3[0] + base[i]) + eps;
        post[i] = 2.0f * orc_sigmoid(mixes[m + i] * scale3[1] + base[m + i]);
    }
    float *c = comb;
    for (int k = 0; k < m * m; k++) c[k] = mixes[2 * m + k] * scale3[2] + base[2 * m + k];
    for (int i = 0; i < m; i++) {
        float *row = c + i * m;
        float mx = row[0];
        for (int j = 1; j < m; j++) mx = row[j] > mx ? row[j] : mx;
        float s = 0.0f;
        for (int j = 0; j < m; j++) s += expf(row[j] - mx);
        for (int j = 0; j < m; j++) row[j] = expf(row[j] - mx) / s + eps;
    }
    for (int pass = 0; pass < 2 * iters - 1; pass++) {
        const int by_col = (pass % 2) == 0; /* column, then (row, column) pairs */
        for (int a = 0; a < m; a++) {
            float s = 0.0f;
            for (int b = 0; b < m; b++) s += by_col ? c[b * m + a] : c[a * m + b];
            for (int b = 0; b < m; b++) {
                float *v = by_col ? &c[b * m + a] : &c[a * m + b];
                *v /= (s + eps);
            }
        }
    }
}

/* hc_pre (src/dsv4/dsv4_model.c:7123-7156) on the flattened state [mult][hid]:
 * rsqrt from the double sum of squares over all mult*hid values; mixes[j] =
 * (fmaf chain of fn row j with the state, index order) * rsqrt; the split;
 * bin[c] = bf16(fmaf chain over the mult streams of pre[i] * state[i][c]). */
void orc_hc_pre(float *bin, float *post, float *comb, const float *state, const float *fn,
                const float *scale3, const float *base, int mult, int hid, int iters,
                float rms_eps, float hc_eps)
{
    const int K = mult * hid, mix_n = (2 + mult) * mult;
    double ss = 0.0;
    for (int i = 0; i < K; i++) {
        const double d = (double)state[i];
        ss += d * d;
    }
    const float rs = 1.0f / sqrtf((float)(ss / K) + rms_eps);
    float *mixes = (float *)orc_alloc((size_t)mix_n * sizeof(float));
    for (int j = 0; j < mix_n; j++) {
        const float *row = fn + (size_t)j * K;
        float acc = 0.0f;
        for (int i = 0; i < K; i++) acc = fmaf(row[i], state[i], acc);
        mixes[j] = acc * rs;
    }
    float pre[8];
    orc_hc_split(pre, post, comb, mixes, scale3, base, mult, iters, hc_eps);
    free(mixes);
    for (int c = 0; c < hid; c++) {
        float acc = 0.0f;
        for (int i = 0; i < mult; i++) acc = fmaf(pre[i], state[(size_t)i * hid + c], acc);
        bin[c] = orc_bf16_round(acc);
    }
}

/* hc_post (src/dsv4/dsv4_model.c:7165-7177): new[i][c] = post[i] * branch[c],
 * then fmaf of comb[i][k] * state[k][c] for k in order; state = bf16(new). */
void orc_hc_post(float *state, const float *branch, const float *post, const float *comb,
                 int mult, int hid)
{
    float *nw = (float *)orc_alloc((size_t)mult * hid * sizeof(float));
    for (int i = 0; i < mult; i++)
        for (int c = 0; c < hid; c++) {
            float y = post[i] * branch[c];
            for (int k = 0; k < mult; k++)
                y = fmaf(comb[i * mult + k], state[(size_t)k * hid + c], y);
            nw[(size_t)i * hid + c] = y;
        }
    for (int i = 0; i < mult * hid; i++) state[i] = orc_bf16_round(nw[i]);
    free(nw);
}
