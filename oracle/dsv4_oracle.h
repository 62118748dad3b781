/* dsv4_oracle.h - CPU oracle for the quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a scalar C restatement of the reference
 * engine's CPU kernels (src/dsv4/dsv4_ops.c, src/dsv4/dsv4_model.c), used as
 * the checker for the HIP path. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never does.
 *
 * Every entry point follows the reference's scalar loop order (the contract the
 * reference pins with its SIMD == scalar tests, tests/unit/test_dsv4_ops.c:197-235)
 * and is built with -ffp-contract=off so that each fmaf() below is the only
 * fused operation, exactly as in the reference build (GNUmakefile:48).
 *
 * Batched entry points take contiguous [batch][n] arrays instead of the
 * reference's arrays of pointers; the per-token arithmetic is unchanged.
 */
#ifndef DSV4_ORACLE_H
#define DSV4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar decode primitives (a1-a6) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
float orc_bf16_round(float f);
float orc_fp8_e4m3(uint8_t code);
float orc_e8m0(uint8_t code);
float orc_fp4_e2m1(uint8_t nibble);
float orc_round_e4m3(float v);
void orc_quant_fp8_act(float *qx, float *qscale, const float *x, int n);

/* ---- GEMVs (a7-a15) ---- */
void orc_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                   int round_out);
void orc_gemv_bf16_batch(float *y, const float *x, int batch, const uint16_t *W,
                         int in, int out, int round_out);
void orc_gemv_fp8_q(float *y, const float *qx, const float *qscale,
                    const uint8_t *W, const uint8_t *S, int in, int out,
                    int round_out);
void orc_gemv_fp8_batch_q(float *y, const float *qx, const float *qscale,
                          int batch, const uint8_t *W, const uint8_t *S,
                          int in, int out, int round_out);
void orc_gemv_fp8_pair_q(float *y0, float *y1, const float *qx,
                         const float *qscale, const uint8_t *W0,
                         const uint8_t *S0, const uint8_t *W1,
                         const uint8_t *S1, int in, int out);
void orc_gemv_fp4_q(float *y, const float *qx, const float *qscale,
                    const uint8_t *W, const uint8_t *S, int in, int rows);
void orc_gemv_fp4_batch_q(float *y, const float *qx, const float *qscale,
                          int batch, const uint8_t *W, const uint8_t *S,
                          int in, int rows);
void orc_gemv_fp4_pair_q(float *y0, float *y1, const float *qx,
                         const float *qscale, const uint8_t *W0,
                         const uint8_t *S0, const uint8_t *W1,
                         const uint8_t *S1, int in, int rows);
void orc_gemv_fp8_legacy(float *y, const float *x, const uint8_t *W,
                         const float *wscale, int in, int rows, int block);
void orc_gemv_fp8_tbl(float *y, const float *x, const uint8_t *W,
                      const float *wscale, int in, int rows, int block);
void orc_gemv_fp4_legacy(float *y, const float *qx, const float *qscale,
                         const uint8_t *W, const float *wscale, int in,
                         int rows, int group);

/* ---- router (a16, a17) ---- */
float orc_sqrt_softplus(float z);
/* moe_forward's routing from precomputed logits z[n_experts]. tid2eid_row is
 * the token's row of tid2eid (topk entries) for hash layers, else NULL. */
void orc_route(int *idx, float *wt, const float *z, const float *bias,
               const int64_t *tid2eid_row, int n_experts, int topk,
               float route_scale);
/* public dsv4_router(): the BF16 gate is passed as uint16_t here. */
void orc_router_public(int *idx, float *wt, const float *x,
                       const uint16_t *gate, const float *bias,
                       const int64_t *tid2eid, int token_id, int hidden,
                       int n_experts, int topk, int hash_layer,
                       float route_scale);

/* ---- expert block (a18-a21) ---- */
void orc_swiglu_quant(float *y, float *qy, float *qys, const float *gate,
                      const float *up, int n, int limit, float route_weight);
/* One routed FP4 expert. scales / weights point at the expert's scale run
 * [w1|w2|w3] and weight run [w1|w2|w3]. out[hidden] holds BF16 values. */
void orc_expert_forward(float *out, const float *qx, const float *qsc,
                        const uint8_t *scales, const uint8_t *weights,
                        int hidden, int inter, int limit, float route_weight);
void orc_shared_expert_forward(float *out, const float *qx, const float *qsc,
                               const uint8_t *sh1, const uint8_t *sh1_s,
                               const uint8_t *sh3, const uint8_t *sh3_s,
                               const uint8_t *sh2, const uint8_t *sh2_s,
                               int hidden, int inter, int limit);

/* ---- MoE layer (a22, a23) ---- */
typedef struct {
    int hidden, inter, n_experts, topk;
    float route_scale, swiglu_limit;
    const uint16_t *gate_w;      /* BF16 [n_experts][hidden]                  */
    const float *bias;           /* F32 [n_experts] or NULL                   */
    const int64_t *tid2eid;      /* I64 [vocab][topk] (hash layers) or NULL   */
    int is_hash;
    const uint8_t *experts;      /* expert e at experts + e*expert_stride:    */
    size_t expert_stride;        /*   scale run, then weight run at +scale_run */
    size_t scale_run;
    const uint8_t *sh1, *sh1_s, *sh3, *sh3_s, *sh2, *sh2_s;
} OrcLayer;

void orc_moe_forward(const OrcLayer *L, const float *x, int token_id,
                     float *out, int *idx_out, float *wt_out);
void orc_route_tokens(const OrcLayer *L, const float *x, const int *token_ids,
                      int n_tokens, int *idx, float *wt);
void orc_moe_route_outputs(const OrcLayer *L, const float *x, int token_id,
                           float *routes, int *idx_out, float *wt_out);
void orc_moe_forward_batch(const OrcLayer *L, const float *x,
                           const int *token_ids, int n_tokens, float *out,
                           int *idx_out, float *wt_out);

/* ---- synthetic-weight quantizers (not in the reference; harness only) ---- */
void orc_quant_fp4_rows(uint8_t *packed, uint8_t *scale_codes, const float *w,
                        int rows, int cols);
void orc_quant_fp8_blocks_e8m0(uint8_t *codes, uint8_t *scale_codes,
                               const float *w, int rows, int cols);
void orc_quant_fp8_blocks_absmax(uint8_t *codes, float *scales, const float *w,
                                 int rows, int cols);
uint8_t orc_e4m3_code(float grid_value);

/* ---- bench-protocol helpers (benchmarks/bench_dsv4_kernels.c) ---- */
/* ---- caller step around the MoE: RMSNorm and Hyper-Connections ---- */
void orc_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps,
                      int round_out);
void orc_hc_split(float *pre, float *post, float *comb, const float *mixes,
                  const float *scale3, const float *base, int mult, int iters, float eps);
void orc_hc_pre(float *bin, float *post, float *comb, const float *state, const float *fn,
                const float *scale3, const float *base, int mult, int hid, int iters,
                float rms_eps, float hc_eps);
void orc_hc_post(float *state, const float *branch, const float *post, const float *comb,
                 int mult, int hid);

uint64_t orc_xorshift_next(uint64_t *state);
double orc_checksum(const float *v, int n);

#ifdef __cplusplus
}
#endif

#endif
