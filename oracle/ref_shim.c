/* ref_shim.c - exposes the reference engine's static MoE routines to the
 * checker. TEST INFRASTRUCTURE ONLY.
 *
 * This translation unit compiles the reference's src/dsv4/dsv4_model.c where
 * it lies (the include path is set by oracle/Makefile) and adds thin exported
 * wrappers around its static functions:
 *   routed_swiglu_quant      src/dsv4/dsv4_model.c:6239
 *   expert_forward           src/dsv4/dsv4_model.c:6337
 *   shared_expert_forward    src/dsv4/dsv4_model.c:6399
 *   moe_forward              src/dsv4/dsv4_model.c:6599
 *   moe_forward_batch        src/dsv4/dsv4_model.c:6812
 *   sqrt_softplus            src/dsv4/dsv4_model.c:5827
 *   head_logits              src/dsv4/dsv4_model.c:7313
 *   head_logits_batch        src/dsv4/dsv4_model.c:7373
 * The MoE entries run on a hand-built DSV4Model whose expert cache holds every
 * expert of layer 0, so every expert lookup is a hit and no I/O path runs
 * (expert_get_many, src/dsv4/dsv4_model.c:3642-3663).
 * Output goes to oracle/_ref/ only: git-ignored, so it never enters the
 * repository's history, but it travels with the working tree to the GPU
 * host as a built file, where the benchmark's CPU-baseline leg times it.
 * It is the checker and the CPU baseline, never part of the product.
 */
#include "dsv4_model.c"

#include "dsv4_oracle.h"

float ref_shim_sqrt_softplus(float z) { return sqrt_softplus(z); }

void ref_shim_routed_swiglu_quant(float *y, float *qy, float *qscale,
                                  const float *gate, const float *up, int n,
                                  int limit, float route_weight)
{
    routed_swiglu_quant(y, qy, qscale, gate, up, n, limit, route_weight);
}

typedef struct {
    DSV4Model *m;
    DSV4LayerW w;
} RefShimModel;

static void ref_shim_build(RefShimModel *s, const OrcLayer *L)
{
    const int H = L->hidden, I = L->inter, E = L->n_experts, K = L->topk;
    DSV4Model *m = (DSV4Model *)calloc(1, sizeof(DSV4Model));
    if (!m) { fprintf(stderr, "ref_shim: OOM\n"); exit(1); }
    m->cfg.hidden = H;
    m->cfg.moe_inter = I;
    m->cfg.n_experts = E;
    m->cfg.topk = K;
    m->cfg.n_layers = 1;
    m->cfg.route_scale = L->route_scale;
    m->cfg.swiglu_limit = L->swiglu_limit;
    /* bind_moe_scratch layout, src/dsv4/dsv4_model.c:5895-5908 */
    size_t scratch = (size_t)H + (H + 127) / 128 + 2 * (size_t)E + K + H +
                     (size_t)K * H + H;
    m->scratch = (float *)calloc(scratch, sizeof(float));
    m->route_scratch = (int *)calloc((size_t)2 * E + K, sizeof(int));
    /* bind_expert_work stride, src/dsv4/dsv4_model.c:5882-5893 */
    size_t stride = (size_t)4 * I + (I + 127) / 128;
    m->expert_work = (float *)calloc(stride * (DSV4_MAX_TOPK + 2), sizeof(float));
    m->cache = (DSV4ExpertSlot *)calloc((size_t)(E > 0 ? E : 1), sizeof(DSV4ExpertSlot));
    if (!m->scratch || !m->route_scratch || !m->expert_work || !m->cache) {
        fprintf(stderr, "ref_shim: OOM\n");
        exit(1);
    }
    for (int e = 0; e < E; e++) {
        uint8_t *base = (uint8_t *)(L->experts + (size_t)e * L->expert_stride);
        m->cache[e].scales = base;
        m->cache[e].weights = base + L->scale_run;
        m->cache[e].layer = 0;
        m->cache[e].expert = e;
        m->cache[e].segment = 1;
    }
    m->cache_slots = E;
    m->main_cache_slots = E;
    m->cur_layer = 0;
    memset(&s->w, 0, sizeof(s->w));
    s->w.gate_w = L->gate_w;
    s->w.bias = L->bias;
    s->w.tid2eid = L->tid2eid;
    s->w.is_hash = L->is_hash;
    s->w.sh1 = L->sh1;
    s->w.sh1_s = L->sh1_s;
    s->w.sh3 = L->sh3;
    s->w.sh3_s = L->sh3_s;
    s->w.sh2 = L->sh2;
    s->w.sh2_s = L->sh2_s;
    s->m = m;
}

static void ref_shim_free(RefShimModel *s)
{
    free(s->m->scratch);
    free(s->m->route_scratch);
    free(s->m->expert_work);
    free(s->m->cache);
    free(s->m);
}

void ref_shim_expert_forward(float *out, const float *qx, const float *qsc,
                             const uint8_t *scales, const uint8_t *weights,
                             int hidden, int inter, int limit,
                             float route_weight)
{
    OrcLayer L;
    memset(&L, 0, sizeof(L));
    L.hidden = hidden;
    L.inter = inter;
    L.n_experts = 0;
    L.topk = 1;
    L.swiglu_limit = (float)limit;
    RefShimModel s;
    ref_shim_build(&s, &L);
    DSV4ExpertSlot slot;
    memset(&slot, 0, sizeof(slot));
    slot.scales = (uint8_t *)scales;
    slot.weights = (uint8_t *)weights;
    DSV4ExpertWork work;
    bind_expert_work(s.m, &work, 0);
    expert_forward(s.m, &slot, qx, qsc, &work, route_weight, 0, 0, out);
    ref_shim_free(&s);
}

void ref_shim_shared_expert_forward(float *out, const float *qx,
                                    const float *qsc, const uint8_t *sh1,
                                    const uint8_t *sh1_s, const uint8_t *sh3,
                                    const uint8_t *sh3_s, const uint8_t *sh2,
                                    const uint8_t *sh2_s, int hidden,
                                    int inter, int limit)
{
    OrcLayer L;
    memset(&L, 0, sizeof(L));
    L.hidden = hidden;
    L.inter = inter;
    L.topk = 1;
    L.swiglu_limit = (float)limit;
    L.sh1 = sh1; L.sh1_s = sh1_s;
    L.sh3 = sh3; L.sh3_s = sh3_s;
    L.sh2 = sh2; L.sh2_s = sh2_s;
    RefShimModel s;
    ref_shim_build(&s, &L);
    DSV4ExpertWork work;
    bind_expert_work(s.m, &work, 0);
    shared_expert_forward(s.m, &s.w, qx, qsc, &work, 0, out);
    ref_shim_free(&s);
}

/* moe_forward on one token; idx/wt are read back from the routing scratch
 * that bind_moe_scratch assigns (src/dsv4/dsv4_model.c:5895-5908). */
void ref_shim_moe_forward(const OrcLayer *L, const float *x, int token_id,
                          float *out, int *idx_out, float *wt_out)
{
    RefShimModel s;
    ref_shim_build(&s, L);
    moe_forward(s.m, &s.w, x, token_id, 0, NULL, out);
    DSV4MoEScratch scratch;
    bind_moe_scratch(s.m, &scratch);
    if (idx_out) memcpy(idx_out, scratch.idx, (size_t)L->topk * sizeof(int));
    if (wt_out) memcpy(wt_out, scratch.wt, (size_t)L->topk * sizeof(float));
    ref_shim_free(&s);
}

void ref_shim_moe_forward_batch(const OrcLayer *L, const float *x,
                                const int *token_ids, int n_tokens, float *out)
{
    RefShimModel s;
    ref_shim_build(&s, L);
    moe_forward_batch(s.m, &s.w, x, token_ids, 0, n_tokens, NULL, NULL, 0,
                      NULL, out);
    ref_shim_free(&s);
}

/* The reference safetensors reader (src/io/k3_st.c:371-602) behind a heap
 * handle, so the checker can compare the checkpoint index and its reads
 * with it. NULL when k3_st_open fails. */
K3St *ref_shim_st_open(const char *dir)
{
    K3St *s = (K3St *)calloc(1, sizeof *s);
    if (!s) return NULL;
    if (k3_st_open(s, dir) != 0) { free(s); return NULL; }
    return s;
}

void ref_shim_st_close(K3St *s)
{
    if (s) { k3_st_close(s); free(s); }
}

int ref_shim_st_count(const K3St *s) { return s->nt; }
int ref_shim_st_nshard(const K3St *s) { return s->nshard; }
const K3Tensor *ref_shim_st_tensor(const K3St *s, int i) { return &s->t[i]; }

/* The caller step around the MoE: the reference's static rmsnorm_bf16
 * (src/dsv4/dsv4_model.c:4934), hc_pre_scratch (:7123) and hc_post_scratch
 * (:7165); hc_pre reads its sizes and epsilons from a bare model config. */
void ref_shim_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps,
                           int round_out)
{
    rmsnorm_bf16(y, x, w, n, eps, round_out);
}

void ref_shim_hc_pre(float *bin, float *post, float *comb, const float *state,
                     const float *fn, const float *scale3, const float *base, int mult,
                     int hid, int iters, float rms_eps, float hc_eps)
{
    DSV4Model *m = (DSV4Model *)calloc(1, sizeof(DSV4Model));
    float *mixes = (float *)calloc((size_t)(2 + mult) * mult, sizeof(float));
    if (!m || !mixes) { fprintf(stderr, "ref_shim: OOM\n"); exit(1); }
    m->cfg.hc_mult = mult;
    m->cfg.hidden = hid;
    m->cfg.hc_iters = iters;
    m->cfg.rms_eps = rms_eps;
    m->cfg.hc_eps = hc_eps;
    hc_pre_scratch(m, NULL, state, fn, scale3, base, bin, post, comb, mixes);
    free(mixes);
    free(m);
}

void ref_shim_hc_post(float *state, const float *branch, const float *post,
                      const float *comb, int mult, int hid)
{
    float *nw = (float *)calloc((size_t)mult * hid, sizeof(float));
    if (!nw) { fprintf(stderr, "ref_shim: OOM\n"); exit(1); }
    hc_post_scratch(state, branch, post, comb, mult, hid, nw);
    free(nw);
}

/* The vocabulary head on a DSV4Model whose head tensor is the given BF16 rows
 * [vocab][hid] in memory, as for a mapped checkpoint (head_map_rows), on
 * `threads` OpenMP threads: one token through head_logits, more through
 * head_logits_batch. */
void ref_shim_head_logits(float *logits, const float *h, const uint16_t *rows, int hid,
                          int vocab, int n_tokens, int threads)
{
    DSV4Model *m = (DSV4Model *)calloc(1, sizeof(DSV4Model));
    if (!m) { fprintf(stderr, "ref_shim: OOM\n"); exit(1); }
    m->cfg.hidden = hid;
    m->cfg.vocab = vocab;
    m->threads = threads > 0 ? threads : 1;
    m->head_map_rows = rows;
    if (n_tokens == 1)
        head_logits(m, h, logits);
    else
        head_logits_batch(m, h, n_tokens, logits);
    free(m);
}
