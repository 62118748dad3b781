/* dsv4_gpu.h - C ABI of the gfx950 (MI355X) quantized MoE expert path.
 *
 * Two layers, both plain C (extern "C", pointers and sizes only):
 *
 * 1. Drop-in entry points with the reference engine's exact names and
 *    signatures (host pointers, void return, abort with a message on a GPU
 *    error, as the reference exits on fatal conditions). They live in
 *    libdsv4_gpu.so next to layer 2 and replace:
 *      include/dsv4/dsv4.h:185-211, 251-254  (public kernels, router)
 *      src/dsv4/dsv4_internal.h:256-286, 326-331 (internal GEMVs, quant)
 *    Weights stay resident in HBM for host ranges registered with
 *    dsv4_gpu_register_weights() (re-registering a range uploads its current
 *    contents; dsv4_gpu_forget_weights*() drop it); weights from an
 *    unregistered range are uploaded for that call only, so a refilled host
 *    buffer can never be served stale. Activations are copied per call.
 *
 * 2. Device-pointer API (dsv4g_*): every pointer is device memory, every call
 *    is asynchronous on the given HIP stream (NULL = default stream) and
 *    returns 0 or a DSV4G_E* code; dsv4g_last_error() gives the message.
 *    This is the layer a device-resident engine calls (the fused MoE entries
 *    replace the static moe_forward / moe_forward_batch of
 *    src/dsv4/dsv4_model.c:6599, 6812, which have no exported symbol).
 *
 * Numerics: the decode-path GEMVs, the public float-scale and BF16 GEMVs,
 * activation quantisation, SwiGLU requant, router (indices and weights) and
 * combine are bit-identical to the reference's scalar loop order. The
 * grouped-GEMM batch path has bit-identical routing and agrees to fp32
 * rounding otherwise (documented tolerance), not bit for bit.
 */
#ifndef DSV4_GPU_H
#define DSV4_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSV4G_VERSION "0.1.0"

#define DSV4G_OK 0
#define DSV4G_EINVAL 1 /* bad argument or unsupported shape */
#define DSV4G_EHIP 2   /* HIP runtime error */

/* One MoE layer resident in HBM (device pointers). Routed expert e occupies
 * expert_stride bytes at experts + e*expert_stride: the E8M0 scale run
 * [w1 | w2 | w3] (per row, per 32 columns) followed at +scale_run by the
 * packed E2M1 weight run [w1 | w2 | w3] (two nibbles per byte, low nibble =
 * even column); w1 = gate [inter][hidden], w2 = down [hidden][inter],
 * w3 = up [inter][hidden]. This is the checkpoint's contiguous per-expert
 * layout (src/dsv4/dsv4_internal.h:8-17, 33-37;
 * src/dsv4/dsv4_model.c:6298-6305). The shared expert is FP8 E4M3 with
 * per-128x128 E8M0 block scales (src/dsv4/dsv4_model.c:2029-2053). */
typedef struct {
    int hidden;            /* 4096 */
    int inter;             /* moe_inter, 2048 */
    int n_experts;         /* 256 */
    int topk;              /* 6 */
    float route_scale;     /* 1.5 */
    float swiglu_limit;    /* 10.0 (used as (int)swiglu_limit, as the reference) */
    const uint16_t *gate_w;   /* BF16 [n_experts][hidden] */
    const float *bias;        /* F32 [n_experts] or NULL */
    const int64_t *tid2eid;   /* I64 [vocab][topk] for hash layers, else NULL */
    const uint8_t *experts;   /* routed experts, see above */
    size_t expert_stride;     /* >= scale_run + weight run (13,369,344 at full size) */
    size_t scale_run;         /* 786,432 at full size */
    const uint8_t *sh1, *sh1_s;  /* shared gate FP8 [inter][hidden] + scales */
    const uint8_t *sh3, *sh3_s;  /* shared up   FP8 [inter][hidden] + scales */
    const uint8_t *sh2, *sh2_s;  /* shared down FP8 [hidden][inter] + scales */
} DSV4GLayer;

/* ------------------------------------------------------ runtime helpers */
const char *dsv4g_last_error(void);
const char *dsv4g_version(void);
int dsv4g_device_count(int *count);
int dsv4g_malloc(void **ptr, size_t bytes);
int dsv4g_free(void *ptr);
int dsv4g_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int dsv4g_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream); /* syncs */
/* Page-locked host memory (the drop-in layer stages activations and outputs
 * through it, so that its copies are asynchronous), and a device-to-host copy
 * that does not synchronise (dst page-locked for it to be asynchronous). */
int dsv4g_host_malloc(void **ptr, size_t bytes);
int dsv4g_host_free(void *ptr);
int dsv4g_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream);
int dsv4g_stream_sync(void *stream);

/* ----------------------------------------------- device-pointer kernels */
/* dsv4_quant_fp8_codes / dsv4_quant_fp8_act over nvec rows of n
 * (src/dsv4/dsv4_model.c:5580-5606, src/dsv4/dsv4_ops.c:122-146). */
int dsv4g_quant_fp8_act(float *qx, float *qscale, const float *x, int n, int nvec,
                        void *stream);
/* Dequantised weights (value * scale), bit-exact with the reference decode. */
int dsv4g_dequant_fp4(float *out, const uint8_t *W, const uint8_t *S, int rows, int cols,
                      void *stream);
int dsv4g_dequant_fp8(float *out, const uint8_t *W, const uint8_t *S, int rows, int cols,
                      void *stream);

/* dsv4_gemv_fp4_q / _pair_q / _batch_q (src/dsv4/dsv4_internal.h:274-286).
 * Batched arrays are contiguous: y [batch][rows], qx [batch][in],
 * qscale [batch][in/128]. in: multiple of 32, at most 8192. */
int dsv4g_gemv_fp4_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *S, int in, int rows, void *stream);
int dsv4g_gemv_fp4_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int rows, void *stream);
int dsv4g_gemv_fp4_batch_q(float *y, const float *qx, const float *qscale, int batch,
                           const uint8_t *W, const uint8_t *S, int in, int rows,
                           void *stream);
/* dsv4_gemv_fp8_q / _pair_q / _batch_q (src/dsv4/dsv4_internal.h:261-272).
 * in: multiple of 16, at most 8192. */
int dsv4g_gemv_fp8_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *S, int in, int out, int round_out, void *stream);
int dsv4g_gemv_fp8_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int out, void *stream);
int dsv4g_gemv_fp8_batch_q(float *y, const float *qx, const float *qscale, int batch,
                           const uint8_t *W, const uint8_t *S, int in, int out,
                           int round_out, void *stream);
/* dsv4_gemv_bf16 / _batch (src/dsv4/dsv4_internal.h:256-259); x [batch][in]
 * (16-byte aligned for the streaming kernels), any batch: in runs of 64, 32,
 * 16, 8 or 4 tokens and a remainder of 1-3 when in is a multiple of 64, each
 * run one launch that reads W once. The vocabulary head
 * (head_logits / head_logits_batch, src/dsv4/dsv4_model.c:7314-7445: the same
 * per-row fmaf chain, logits unrounded) is this call with in = hidden,
 * out = vocab, round_out = 0. */
int dsv4g_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                    int round_out, int batch, void *stream);
/* The greedy token of each of n rows of logits (row r at logits + r * stride):
 * the CLI's first-largest rule (src/cli/dsv4_run.c:357-359), NaN never taken,
 * 0 when logits[0] is NaN. idx [n], device. */
int dsv4g_argmax(int *idx, const float *logits, int vocab, int n, size_t stride,
                 void *stream);
/* dsv4_gemv_fp8 (mode 0) / dsv4_gemv_fp8_tbl (mode 1) (include/dsv4/dsv4.h:200-206)
 * and dsv4_gemv_fp4 (include/dsv4/dsv4.h:208-211), float block scales. */
int dsv4g_gemv_fp8_float(float *y, const float *x, const uint8_t *W, const float *wscale,
                         int in, int rows, int block, int mode, void *stream);
int dsv4g_gemv_fp4_float(float *y, const float *qx, const float *qscale, const uint8_t *W,
                         const float *wscale, int in, int rows, int group, void *stream);

/* Router of moe_forward (src/dsv4/dsv4_model.c:6615-6676) for n_tokens
 * rows of x: idx [n][topk] ascending, wt [n][topk]. z_ws, zabs_ws: device
 * scratch of n_tokens*n_experts floats each. */
int dsv4g_router(int *idx, float *wt, const float *x, const DSV4GLayer *L,
                 const int *token_ids, int n_tokens, float *z_ws, float *zabs_ws,
                 void *stream);
/* Public dsv4_router semantics (src/dsv4/dsv4_ops.c:473-545) for one token:
 * unfused logits, weights (score * (1/sum)) * route_scale. For a hash layer
 * tid2eid points at the token's row and token_id at a device 0. */
int dsv4g_router_public(int *idx, float *wt, const float *x, const uint16_t *gate,
                        const float *bias, const int64_t *tid2eid, const int *token_id,
                        int hidden, int n_experts, int topk, int hash_layer,
                        float route_scale, float *z_ws, float *zabs_ws, void *stream);
/* expert_forward (src/dsv4/dsv4_model.c:6289-6345) for one token: out [hidden]
 * = the BF16-rounded FP4 down GEMV of routed_swiglu_quant(gate, up) of the
 * paired FP4 gate/up GEMV of qx / qscale (from dsv4g_quant_fp8_act). slot: one
 * expert in the checkpoint layout (scales [s1|s2|s3], then scale_run bytes on
 * the weights [w1|w2|w3]); weight: device pointer to the route weight, NULL
 * for 1. workspace: dsv4g_expert_workspace_bytes(inter) bytes, 256-aligned.
 * Two launches on the stream up to inter 4096 and hidden 8192 (the paired
 * GEMV with the SwiGLU epilogue, then the down GEMV with the requant folded
 * in), three beyond. */
size_t dsv4g_expert_workspace_bytes(int inter);
int dsv4g_expert_forward(float *out, const float *qx, const float *qscale, const uint8_t *slot,
                         size_t scale_run, int hidden, int inter, float swiglu_limit,
                         const float *weight, void *workspace, size_t workspace_bytes,
                         void *stream);
/* routed_swiglu_quant (src/dsv4/dsv4_model.c:6239-6287) over n_slots slots;
 * slot s reads gate at gate_up + 2*s*inter and up right after it. Weights:
 * K > 0: slots are [token][K+1], slot (t,k<K) uses wt[t*K+k], slot K uses 1;
 * K == 0: slot s uses wt[s]; wt == NULL: weight 1. */
int dsv4g_swiglu_quant(float *qy, float *qys, const float *gate_up, const float *wt, int K,
                       int n_slots, int inter, float limit, void *stream);

/* Decode MoE layer: moe_forward for each of n_tokens (at most 1020) rows of
 * x (BF16 values in fp32), bit-exact. out [n][hidden]. idx_out/wt_out
 * (optional, device) receive the routing. workspace: 256-byte aligned device
 * memory of at least dsv4g_moe_workspace_bytes(L, n_tokens), zeroed once
 * before its first use (dsv4g_moe_workspace_init, or any zero fill); every
 * call leaves it ready for the next, for any token count it holds. A
 * workspace serves layers of one shape (hidden, inter, n_experts, topk);
 * zero it again before a call with another shape. Calls sharing one
 * workspace must not overlap. */
size_t dsv4g_moe_workspace_bytes(const DSV4GLayer *L, int n_tokens);
int dsv4g_moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream);
int dsv4g_moe_forward(float *out, const float *x, const DSV4GLayer *L, const int *token_ids,
                      int n_tokens, void *workspace, size_t workspace_bytes, int *idx_out,
                      float *wt_out, void *stream);
/* The same layer with a tolerance (expert outputs within 1e-3 relative) instead
 * of bit-exactness: top-k indices identical to the reference's always; when a
 * token's candidate experts are exactly its top-k (the rigorous bound of the
 * parallel router logits separates the k-th from the (k+1)-th), the route
 * weights come from the parallel logits (within a few fp32 ulps of the
 * reference's) and the exact sequential chains are skipped; otherwise the
 * token is routed exactly as by dsv4g_moe_forward. Expert outputs agree to
 * fp32 rounding, so a BF16 output element may differ by one BF16 ulp. No
 * counterpart in the reference: for decode loops that accept that tolerance. */
int dsv4g_moe_forward_fast(float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, int *idx_out, float *wt_out, void *stream);
/* dsv4g_moe_forward with no workspace argument and no allocation of any kind:
 * the workspace is the library's own 16 MiB device array (one per GPU, held
 * until the process ends), so the call fits code under HIP graph capture and
 * loops that may not allocate. No counterpart in the reference: for callers
 * that cannot allocate. Same results as dsv4g_moe_forward; EINVAL when
 * dsv4g_moe_workspace_bytes(L, n_tokens) exceeds 16 MiB (about 2.1 MiB per
 * token at the model's shape: up to 7 tokens per call). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race and must not be issued. A call with a layer of another shape
 * than the previous call's on that GPU first clears the array (a fill
 * kernel). That decision is taken on the host when the call is enqueued: a
 * captured call replays without it, so a graph holding noalloc calls must
 * not be replayed after a noalloc call of another layer shape on that GPU
 * (all MoE layers of the model share one shape). */
int dsv4g_moe_forward_noalloc(float *out, const float *x, const DSV4GLayer *L,
                              const int *token_ids, int n_tokens, int *idx_out, float *wt_out,
                              void *stream);
/* The status word of the current GPU's no-allocation array, read into
 * *status (host) with a synchronisation of the stream: 0 when every
 * cross-workgroup wait of the noalloc calls since the last read completed,
 * nonzero when one ran out (their outputs are not valid). A nonzero status
 * also clears the whole array (a fill kernel on the stream), so the next
 * call starts from zeroed records and flags. No counterpart in the
 * reference: the status query of dsv4g_moe_forward_noalloc. */
int dsv4g_moe_noalloc_status(unsigned *status, void *stream);
/* The same layer as DSV4G_DECODE_PHASES ordered launches, for callers that
 * interleave or time them: 0 the activation's E4M3 codes, the approximate
 * router logits, the candidate experts and the shared expert's gate/up; 1
 * the exact router chains and top-k, the candidates' gate/up GEMVs and the
 * shared expert's down GEMV; 2 the routes' SwiGLU requant, the routed down
 * GEMVs and the ordered combine. Phases 0 .. DSV4G_DECODE_PHASES - 1 in
 * order equal one fused call (the workspace is left as the fused call
 * leaves it only after the last). phase | DSV4G_DECODE_FAST runs those of
 * dsv4g_moe_forward_fast. dsv4g_moe_decode_routing copies the routing of the
 * last call. x and out: 16-byte aligned. */
#define DSV4G_DECODE_PHASES 3
#define DSV4G_DECODE_FAST 256
int dsv4g_moe_decode_phase(int phase, float *out, const float *x, const DSV4GLayer *L,
                           const int *token_ids, int n_tokens, void *workspace,
                           size_t workspace_bytes, void *stream);
int dsv4g_moe_decode_routing(int *idx_out, float *wt_out, const DSV4GLayer *L, int n_tokens,
                             void *workspace, void *stream);
/* The decode workspace's sticky status word, read into *status (host) with a
 * synchronisation of the stream, then cleared: 0 when every cross-workgroup
 * wait of the calls since the last read completed; nonzero when one ran out
 * (the outputs of those calls are not valid; re-initialise the workspace with
 * dsv4g_moe_workspace_init). No counterpart in the reference. */
int dsv4g_moe_decode_status(unsigned *status, void *workspace, void *stream);
/* dsv4g_moe_forward (fast = 0) or dsv4g_moe_forward_fast (fast = 1), also
 * writing each route's expert output before its BF16 rounding to route_out
 * [n_tokens][topk + 1][hidden] (routes in ascending expert id, slot topk the
 * shared expert). No counterpart in the reference, which rounds each expert
 * output to BF16 (src/dsv4/dsv4_model.c:1073): for validating the
 * accumulation. */
int dsv4g_moe_forward_routes(float *out, const float *x, const DSV4GLayer *L,
                             const int *token_ids, int n_tokens, void *workspace,
                             size_t workspace_bytes, int *idx_out, float *wt_out,
                             float *route_out, int fast, void *stream);

/* Batched MoE layer: moe_forward_batch (src/dsv4/dsv4_model.c:6812-7117) for
 * n_tokens rows of x (speculative verify, prefill) as grouped GEMMs on the
 * BF16 MFMA (v_mfma_f32_16x16x32_bf16) with exactly scaled operands: FP4/FP8
 * weights times their E8M0 scale and the E4M3-quantised activations are
 * exact in BF16, so every product is exact and only the fp32 summation order
 * differs from the reference. Routing (idx, wt) is bit-exact; expert outputs
 * agree to fp32 rounding of the accumulation. x must hold BF16 values for the
 * tightest router bound (other inputs are handled with a wider margin).
 * A route without a selectable expert adds nothing to its token's output.
 * workspace: at least dsv4g_moe_batch_workspace_bytes(L, n_tokens). */
size_t dsv4g_moe_batch_workspace_bytes(const DSV4GLayer *L, int n_tokens);
int dsv4g_moe_forward_batch(float *out, const float *x, const DSV4GLayer *L,
                            const int *token_ids, int n_tokens, void *workspace,
                            size_t workspace_bytes, int *idx_out, float *wt_out,
                            void *stream);
/* The same, also writing each route's expert output before its BF16 rounding
 * to route_out [n_tokens][topk + 1][hidden] (fp32; routes in ascending expert
 * id, slot topk the shared expert; slots of routes without an expert are not
 * written). No counterpart in the reference, which rounds each expert output
 * to BF16 (src/dsv4/dsv4_model.c:1073): for validating the accumulation. */
int dsv4g_moe_forward_batch_routes(float *out, const float *x, const DSV4GLayer *L,
                                   const int *token_ids, int n_tokens, void *workspace,
                                   size_t workspace_bytes, int *idx_out, float *wt_out,
                                   float *route_out, void *stream);

/* Synthetic-checkpoint quantisers (the reference ships none in C):
 * FP4 rows with per-32 E8M0 scales; FP8 128x128 blocks with E8M0 codes
 * (mode 0, scales = uint8) or fp32 absmax/448 (mode 1, scales = float). */
int dsv4g_quant_fp4_rows(uint8_t *packed, uint8_t *scales, const float *w, int rows,
                         int cols, void *stream);
int dsv4g_quant_fp8_blocks(uint8_t *codes, void *scales, const float *w, int rows, int cols,
                           int mode, void *stream);

/* ---------------------------------------- caller step around the MoE ----
 * The FFN half of forward_loaded_layer (src/dsv4/dsv4_model.c:7549-7559) on
 * device, bit-exact: Hyper-Connection pre-mix with its Sinkhorn split, the
 * RMSNorm with BF16 gain, the MoE layer, the post-mix into the residual
 * state. state: [n_tokens][mult][hidden] fp32 (BF16 values), updated in place
 * by hc_post; hc_fn [(2+mult)*mult][mult*hidden], hc_scale [3],
 * hc_base [(2+mult)*mult] (the layer's hc_ffn_fn / _scale / _base, F32);
 * mult at most 7; hidden a multiple of 4; state and hc_fn 16-byte aligned.
 * status (optional, device): bit 2 is set if a wait inside hc_pre ran out
 * (never expected; the outputs are then not valid). */
/* rmsnorm_bf16 (src/dsv4/dsv4_model.c:4934-4951) over rows of n: y may be x;
 * w: BF16 gain [n] or NULL. */
int dsv4g_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps,
                       int round_out, int rows, void *stream);
/* dsv4_hc_split (include/dsv4/dsv4.h:236-244) for n rows of mixes
 * [(2+mult)*mult]: pre, post [n][mult], comb [n][mult*mult]. */
int dsv4g_hc_split(float *pre, float *post, float *comb, const float *mixes,
                   const float *scale3, const float *base, int mult, int iters, float eps,
                   int n, void *stream);
/* hc_pre (src/dsv4/dsv4_model.c:7123-7156) for n_tokens: bin [n][hidden],
 * post [n][mult], comb [n][mult*mult]; with norm_w, bin is then
 * rmsnorm_bf16(bin, bin, norm_w, hidden, rms_eps, 1) as the caller applies
 * it (src/dsv4/dsv4_model.c:7524, 7553). */
int dsv4g_hc_pre(float *bin, float *post, float *comb, const float *state, const float *fn,
                 const float *scale3, const float *base, const uint16_t *norm_w, int mult,
                 int hidden, int iters, float rms_eps, float hc_eps, int n_tokens,
                 unsigned *status, void *stream);
/* hc_post (src/dsv4/dsv4_model.c:7165-7177): state [n][mult][hidden] updated
 * in place from branch [n][hidden], post, comb. */
int dsv4g_hc_post(float *state, const float *branch, const float *post, const float *comb,
                  int mult, int hidden, int n_tokens, void *stream);
/* hc_pre + rmsnorm_bf16(ffn_norm) -> dsv4g_moe_forward -> hc_post for
 * n_tokens states (token_ids for hash layers). workspace: 256-byte aligned,
 * at least dsv4g_ffn_step_workspace_bytes(L, mult, n_tokens), zeroed once
 * before first use (it begins with the decode MoE workspace, whose status
 * word dsv4g_moe_decode_status reads; the same shape rules apply; the step's
 * own buffers sit at its end, so a workspace sized for N tokens serves every
 * call with at most N). idx_out / wt_out: optional routing. Asynchronous:
 * the caller reads dsv4g_moe_decode_status at its next synchronisation
 * (the sticky word covers hc_pre's and the MoE layer's waits of every step
 * since the last read) and treats a nonzero status as fatal. */
size_t dsv4g_ffn_step_workspace_bytes(const DSV4GLayer *L, int mult, int n_tokens);
int dsv4g_ffn_step(float *state, const float *hc_fn, const float *hc_scale,
                   const float *hc_base, const uint16_t *ffn_norm, const DSV4GLayer *L,
                   const int *token_ids, int n_tokens, int mult, int iters, float rms_eps,
                   float hc_eps, void *workspace, size_t workspace_bytes, int *idx_out,
                   float *wt_out, void *stream);

/* ------------------------------------------ checkpoint index + HBM loader
 * The safetensors index replaces the reference reader K3St
 * (src/io/k3_st.h:34-103): k3_st_open / close / find / read / read_f32 /
 * numel / elemsize become dsv4g_st_*, with the same dtype numbering, tensor
 * record (absolute file offset, byte span) and validation (byte span equal to
 * numel * elemsize, inside the file; names unique across shards; shards are
 * the directory's *.safetensors sorted by name). k3_st_read_aligned
 * (O_DIRECT widening for the expert cache) becomes dsv4g_st_read_range: with
 * every expert resident in HBM there is no per-token streaming. Index calls
 * touch no GPU. Errors: DSV4G_EIO with the message in dsv4g_last_error(). */
#define DSV4G_EIO 3 /* checkpoint file missing, malformed or short */

enum { DSV4G_DT_UNKNOWN = 0, DSV4G_DT_U8, DSV4G_DT_BF16, DSV4G_DT_F16, DSV4G_DT_F32,
       DSV4G_DT_I8, DSV4G_DT_I64, DSV4G_DT_F8_E4M3, DSV4G_DT_F8_E8M0 };

typedef struct {
    const char *name;
    int shard;        /* index into the sorted shard list */
    int dtype;        /* DSV4G_DT_* */
    int ndim;         /* 0 (scalar) .. 4 */
    int64_t shape[4];
    int64_t off;      /* absolute byte offset in its shard file */
    int64_t nbytes;
} DSV4GTensor;

typedef struct DSV4GSt DSV4GSt;

int dsv4g_st_open(DSV4GSt **st, const char *dir);                 /* k3_st.h:67 */
void dsv4g_st_close(DSV4GSt *st);                                 /* k3_st.h:68 */
const DSV4GTensor *dsv4g_st_find(const DSV4GSt *st, const char *name); /* k3_st.h:72 */
int64_t dsv4g_st_read(const DSV4GSt *st, const DSV4GTensor *t, void *buf); /* k3_st.h:75 */
int64_t dsv4g_st_read_f32(const DSV4GSt *st, const DSV4GTensor *t, float *out); /* k3_st.h:99 */
int64_t dsv4g_st_numel(const DSV4GTensor *t);                     /* k3_st.h:102 */
int dsv4g_st_elemsize(int dtype);                                 /* k3_st.h:103 */
/* [off, off + nbytes) of a shard into buf; returns the bytes read
 * (k3_st.h:92-93 without the O_DIRECT widening: the payload is at buf[0]). */
int64_t dsv4g_st_read_range(const DSV4GSt *st, int shard, int64_t off, int64_t nbytes,
                            void *buf);
/* Iteration in discovery order (shard, then header order): K3St.t / .nt. */
int dsv4g_st_count(const DSV4GSt *st);
const DSV4GTensor *dsv4g_st_tensor(const DSV4GSt *st, int i);
int dsv4g_st_nshard(const DSV4GSt *st);
const char *dsv4g_st_shard_path(const DSV4GSt *st, int shard);
const char *dsv4g_st_dtype_name(int dtype);
/* One tensor's bytes into device memory dst (pinned staging; returns when
 * the copy has completed). */
int dsv4g_st_upload(const DSV4GSt *st, const DSV4GTensor *t, void *dst, void *stream);

/* One layer's MoE weights, read from the checkpoint into one device arena in
 * the DSV4GLayer layout: the named tensors "<scope>.<layer>.ffn.gate.weight",
 * ".ffn.gate.bias" (or ".ffn.gate.tid2eid" when is_hash), the shared expert
 * ".ffn.shared_experts.w{1,3,2}.{weight,scale}" and every routed expert's
 * ".ffn.experts.<e>.w{1,2,3}.{scale,weight}", bound with the reference's
 * checks (src/dsv4/dsv4_model.c:1587-1611, 2014-2053, 3063-3136; scope
 * "layers" or "mtp"). On entry L holds the layer's configuration (hidden,
 * inter, n_experts, topk, route_scale, swiglu_limit); on success its pointers
 * point into arena. arena: device memory of at least
 * dsv4g_moe_layer_bytes(L, is_hash, vocab) bytes (vocab: rows of tid2eid).
 * Returns when every byte is in place. Routed expert slots are 256-byte
 * aligned; a checkpoint with each expert's runs stored w1, w2, w3 is read in
 * long sequential spans. */
size_t dsv4g_moe_layer_bytes(const DSV4GLayer *shape, int is_hash, int vocab);
int dsv4g_load_moe_layer(DSV4GLayer *L, void *arena, size_t arena_bytes, const DSV4GSt *st,
                         const char *scope, int layer, int is_hash, int vocab, void *stream);

/* -------------------------------------------- drop-in (host pointers) ----
 * Same names, argument meaning and error behaviour as the reference. */
uint16_t dsv4_f32_to_bf16(float f);                                 /* dsv4.h:183 */
float dsv4_fp8_e4m3(uint8_t code);                                  /* dsv4.h:186 */
float dsv4_e8m0(uint8_t code);                                      /* dsv4.h:188 */
float dsv4_round_e4m3(float v);                                     /* dsv4_internal.h:331 */
void dsv4_quant_fp8_act(float *out, float *scales, const float *x, int n); /* dsv4.h:193 */
void dsv4_quant_fp8_codes(float *qx, float *qscale, const float *x, int n); /* dsv4_internal.h:327 */
void dsv4_gemv_fp8(float *y, const float *x, const uint8_t *W, const float *wscale,
                   int in, int rows, int block);                    /* dsv4.h:200 */
void dsv4_gemv_fp8_tbl(float *y, const float *x, const uint8_t *W, const float *wscale,
                       int in, int rows, int block);                /* dsv4.h:203 */
void dsv4_gemv_fp4(float *y, const float *qx, const float *qscale, const uint8_t *W,
                   const float *wscale, int in, int rows, int group); /* dsv4.h:209 */
void dsv4_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                    int round_out);                                 /* dsv4_internal.h:256 */
void dsv4_gemv_bf16_batch(float *const *y, const float *const *x, int batch,
                          const uint16_t *W, int in, int out, int round_out);
void dsv4_gemv_fp8_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *wscale_code, int in, int out, int round_out);
void dsv4_gemv_fp8_batch_q(float *const *y, const float *const *qx,
                           const float *const *qscale, int batch, const uint8_t *W,
                           const uint8_t *wscale_code, int in, int out, int round_out);
void dsv4_gemv_fp8_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int out);
void dsv4_gemv_fp4_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *wscale_code, int in, int rows);
void dsv4_gemv_fp4_batch_q(float *const *y, const float *const *qx,
                           const float *const *qscale, int batch, const uint8_t *W,
                           const uint8_t *wscale_code, int in, int rows);
void dsv4_gemv_fp4_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int rows);
void dsv4_router(int *idx, float *wt, const float *x, const float *gate, const float *bias,
                 const int64_t *tid2eid, int token_id, int hidden, int n_experts,
                 int topk, int hash_layer, float route_scale, float rms_eps); /* dsv4.h:251 */

/* Weight residency for the drop-in entry points (no counterpart in the
 * reference, whose weights are host memory). register: keep [host, host +
 * bytes) resident, uploading its current contents (again, if it overlaps a
 * registered range: that range is dropped first); the caller keeps the
 * contents unchanged until it forgets or re-registers the range. forget:
 * drop every registered range containing host; forget_range: every range
 * overlapping [host, host + bytes). Unregistered weights are uploaded per
 * call. */
int dsv4_gpu_register_weights(const void *host, size_t bytes);
void dsv4_gpu_forget_weights(const void *host);
void dsv4_gpu_forget_weights_range(const void *host, size_t bytes);
void dsv4_gpu_forget_all_weights(void);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_GPU_H */
