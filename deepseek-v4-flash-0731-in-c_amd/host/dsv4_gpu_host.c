/* dsv4_gpu_host.c - the drop-in host layer: the reference engine's kernel
 * entry points, with its exact names and signatures, running on the gfx950
 * kernels through the dsv4g_* C ABI.
 *
 * Contract kept from the reference:
 *  - callers own every buffer; y is fully overwritten; weights are const;
 *  - kernels return void; fatal conditions print "dsv4: ..." to stderr and
 *    exit(1) (src/dsv4/dsv4_model.c:689-693, 1094-1098);
 *  - batched calls accept at most 33 token vectors (DSV4_MAX_TOPK + 1);
 *  - calls may come from several threads (src/dsv4/dsv4_model.c:6703-6726):
 *    one process-wide mutex serialises GPU use.
 * Weights (host pointers) stay resident in HBM when their range is
 * registered and are uploaded per call otherwise (the weight cache below);
 * activations and outputs are copied per call on the default stream.
 */
#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dsv4_gpu.h"

#define DSV4_HOST_MAX_BATCH 33

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

static void fatal(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "dsv4: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
    exit(1);
}

static void check(int rc, const char *what)
{
    if (rc) fatal("%s: %s", what, dsv4g_last_error());
}

/* ------------------------------------------------------ weight cache ---- */
/* Weights stay resident in HBM only for host ranges the caller registered
 * (dsv4_gpu_register_weights): registration is the caller's promise that the
 * range's contents stay as they are until it forgets or re-registers the
 * range. Registering a range again uploads its current contents afresh, so a
 * caller that refills a buffer with other weights (the reference's expert
 * cache refills its slot buffers on a miss, src/dsv4/dsv4_model.c:3430-3458)
 * re-registers it, or forgets it. Weights passed from an unregistered range
 * are uploaded for that call only, so they can never be stale. */
typedef struct WeightEntry {
    const unsigned char *host;
    size_t bytes;
    void *dev;
    struct WeightEntry *next;
} WeightEntry;

static WeightEntry *g_weights;

static void *weights_find(const void *host, size_t bytes)
{
    const unsigned char *p = (const unsigned char *)host;
    for (WeightEntry *w = g_weights; w; w = w->next)
        if (p >= w->host && p + bytes <= w->host + w->bytes)
            return (unsigned char *)w->dev + (p - w->host);
    return NULL;
}

/* caller holds g_lock: drop every entry that overlaps [host, host + bytes)
 * (bytes = 0: every entry containing host) */
static void weights_drop(const void *host, size_t bytes)
{
    const unsigned char *lo = (const unsigned char *)host;
    const unsigned char *hi = lo + (bytes ? bytes : 1);
    WeightEntry **pp = &g_weights;
    while (*pp) {
        WeightEntry *w = *pp;
        if (w->host < hi && lo < w->host + w->bytes) {
            *pp = w->next;
            dsv4g_free(w->dev);
            free(w);
        } else {
            pp = &w->next;
        }
    }
}

/* Per-call staging of unregistered weights: one grow-only device buffer per
 * weight operand of a call (a call passes at most four). */
#define DSV4_HOST_WSLOTS 4
static void *g_wstage[DSV4_HOST_WSLOTS];
static size_t g_wstage_bytes[DSV4_HOST_WSLOTS];

/* caller holds g_lock; slot: the operand's index within the call */
static void *weights_get(const void *host, size_t bytes, int slot)
{
    if (!host) return NULL;
    void *d = weights_find(host, bytes);
    if (d) return d;
    if (bytes > g_wstage_bytes[slot]) {
        if (g_wstage[slot]) dsv4g_free(g_wstage[slot]);
        g_wstage[slot] = NULL;
        g_wstage_bytes[slot] = 0;
        check(dsv4g_malloc(&g_wstage[slot], bytes), "weight staging");
        g_wstage_bytes[slot] = bytes;
    }
    check(dsv4g_memcpy_h2d(g_wstage[slot], host, bytes, NULL), "weight staging");
    return g_wstage[slot];
}

int dsv4_gpu_register_weights(const void *host, size_t bytes)
{
    if (!host || !bytes) return -1;
    pthread_mutex_lock(&g_lock);
    weights_drop(host, bytes);
    WeightEntry *w = (WeightEntry *)calloc(1, sizeof(*w));
    if (!w) fatal("out of memory in the weight cache");
    check(dsv4g_malloc(&w->dev, bytes), "weight upload");
    check(dsv4g_memcpy_h2d(w->dev, host, bytes, NULL), "weight upload");
    check(dsv4g_stream_sync(NULL), "weight upload");
    w->host = (const unsigned char *)host;
    w->bytes = bytes;
    w->next = g_weights;
    g_weights = w;
    pthread_mutex_unlock(&g_lock);
    return 0;
}

void dsv4_gpu_forget_weights(const void *host)
{
    pthread_mutex_lock(&g_lock);
    weights_drop(host, 0);
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gpu_forget_weights_range(const void *host, size_t bytes)
{
    pthread_mutex_lock(&g_lock);
    weights_drop(host, bytes);
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gpu_forget_all_weights(void)
{
    pthread_mutex_lock(&g_lock);
    while (g_weights) {
        WeightEntry *w = g_weights;
        g_weights = w->next;
        dsv4g_free(w->dev);
        free(w);
    }
    pthread_mutex_unlock(&g_lock);
}

/* ---------------------------------------------------- per-call staging ---- */
/* One grow-only device arena for activations and outputs (caller holds the
 * lock, so a single arena suffices), mirrored by a page-locked host arena of
 * the same size: up() copies the caller's input into the mirror and queues
 * an asynchronous upload from it; down() queues an asynchronous download into
 * the mirror and records where the caller wants it; finish() waits once for
 * the stream and copies every recorded output out. So a call costs one
 * synchronisation, not one per output, and no copy goes through pageable
 * memory. */
static void *g_arena;
static unsigned char *g_pin;
static size_t g_arena_bytes;

#define DSV4_HOST_MAXDOWN 80
typedef struct { void *host; size_t off, bytes; } PendingDown;
static PendingDown g_down[DSV4_HOST_MAXDOWN];
static int g_ndown;

static void *arena(size_t bytes)
{
    if (bytes > g_arena_bytes) {
        if (g_arena) dsv4g_free(g_arena);
        if (g_pin) dsv4g_host_free(g_pin);
        g_arena = NULL;
        g_pin = NULL;
        g_arena_bytes = 0;
        size_t want = bytes + bytes / 2 + 4096;
        check(dsv4g_malloc(&g_arena, want), "staging allocation");
        check(dsv4g_host_malloc((void **)&g_pin, want), "staging allocation");
        g_arena_bytes = want;
    }
    return g_arena;
}

/* carve 256-byte aligned pieces out of the arena */
typedef struct { unsigned char *base; size_t off; } Carver;

static void *carve(Carver *c, size_t bytes)
{
    void *p = c->base + c->off;
    c->off += (bytes + 255) & ~(size_t)255;
    return p;
}

static size_t arena_off(const void *dev)
{
    return (size_t)((const unsigned char *)dev - (const unsigned char *)g_arena);
}

static void up(void *dev, const void *host, size_t bytes)
{
    unsigned char *m = g_pin + arena_off(dev);
    memcpy(m, host, bytes);
    check(dsv4g_memcpy_h2d(dev, m, bytes, NULL), "copy to device");
}

static void finish(void);

static void down(void *host, const void *dev, size_t bytes)
{
    if (g_ndown == DSV4_HOST_MAXDOWN) finish(); /* a list full of outputs: deliver them */
    const size_t off = arena_off(dev);
    check(dsv4g_memcpy_d2h_async(g_pin + off, dev, bytes, NULL), "copy to host");
    g_down[g_ndown].host = host;
    g_down[g_ndown].off = off;
    g_down[g_ndown].bytes = bytes;
    g_ndown++;
}

static void finish(void)
{
    check(dsv4g_stream_sync(NULL), "copy to host");
    for (int i = 0; i < g_ndown; i++)
        memcpy(g_down[i].host, g_pin + g_down[i].off, g_down[i].bytes);
    g_ndown = 0;
}

/* ------------------------------------------------------- scalar decode ---- */
/* Scalar helpers of the public API; pure functions of their argument with
 * the reference's bit-level rules (include/dsv4/dsv4.h:183-190). */
uint16_t dsv4_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float from_bits(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float dsv4_fp8_e4m3(uint8_t code)
{
    uint32_t e = (code >> 3) & 15u, m = code & 7u;
    float mag;
    if (e == 0)
        mag = (float)m * (1.0f / 512.0f);
    else if (e == 15 && m == 7)
        mag = from_bits(0x7fc00000u);
    else
        mag = from_bits(((e + 120u) << 23) | (m << 20));
    return (code & 0x80) ? -mag : mag;
}

float dsv4_e8m0(uint8_t code)
{
    if (code == 255) return from_bits(0x7fc00000u);
    return code == 0 ? from_bits(0x00400000u) : from_bits((uint32_t)code << 23);
}

/* Nearest E4M3 grid value, ties to even, overflow to +-448
 * (src/dsv4/dsv4_ops.c:93-109): frexp split, 3-bit mantissa for exponents
 * >= -5, subnormal step 2^-9 otherwise. rintf (default rounding) is the
 * round-half-even the reference builds from floorf/fmodf. */
float dsv4_round_e4m3(float v)
{
    if (v == 0.0f) return 0.0f;
    const float s = v < 0 ? -1.0f : 1.0f;
    const float a = fabsf(v);
    int e;
    float m = frexpf(a, &e);
    if (e >= -5) {
        float mr = rintf(m * 16.0f) / 16.0f;
        if (mr >= 1.0f) {
            mr = 0.5f;
            e++;
        }
        if (e - 1 > 8) return s * 448.0f;
        return s * mr * ldexpf(1.0f, e);
    }
    return s * (rintf(a * 512.0f) / 512.0f);
}

/* --------------------------------------------------------- activation ---- */
static void quant_act(float *qx, float *qscale, const float *x, int n)
{
    if (n <= 0) return;
    pthread_mutex_lock(&g_lock);
    const size_t nb = (size_t)(n + 127) / 128;
    Carver c = {arena((size_t)n * 8 + nb * 4 + 1024), 0};
    float *dx = carve(&c, (size_t)n * 4), *dq = carve(&c, (size_t)n * 4);
    float *ds = carve(&c, nb * 4);
    up(dx, x, (size_t)n * 4);
    check(dsv4g_quant_fp8_act(dq, ds, dx, n, 1, NULL), "quant_fp8");
    down(qx, dq, (size_t)n * 4);
    down(qscale, ds, nb * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_quant_fp8_act(float *out, float *scales, const float *x, int n)
{
    quant_act(out, scales, x, n);
}

void dsv4_quant_fp8_codes(float *qx, float *qscale, const float *x, int n)
{
    quant_act(qx, qscale, x, n);
}

/* --------------------------------------------------------------- GEMVs ---- */
static size_t fp4_w_bytes(int in, int rows) { return (size_t)rows * ((in + 1) / 2); }
static size_t fp4_s_bytes(int in, int rows) { return (size_t)rows * ((in + 31) / 32); }
static size_t fp8_w_bytes(int in, int rows) { return (size_t)rows * in; }
static size_t fp8_s_bytes(int in, int rows)
{
    return (size_t)((rows + 127) / 128) * ((in + 127) / 128);
}

/* Gather batched host vectors into one contiguous device block. */
static void up_rows(float *dev, const float *const *rows, int batch, size_t n)
{
    for (int t = 0; t < batch; t++) up(dev + (size_t)t * n, rows[t], n * 4);
}

static void down_rows(float *const *rows, const float *dev, int batch, size_t n)
{
    for (int t = 0; t < batch; t++) down(rows[t], dev + (size_t)t * n, n * 4);
}

static void batch_guard(int batch, const char *kind)
{
    if (batch > DSV4_HOST_MAX_BATCH)
        fatal("%s batch %d exceeds %d", kind, batch, DSV4_HOST_MAX_BATCH);
}

void dsv4_gemv_fp4_batch_q(float *const *y, const float *const *qx,
                           const float *const *qscale, int batch, const uint8_t *W,
                           const uint8_t *wscale_code, int in, int rows)
{
    if (batch <= 0 || rows <= 0) return;
    batch_guard(batch, "FP4");
    pthread_mutex_lock(&g_lock);
    const size_t qn = (size_t)(in + 127) / 128;
    const uint8_t *dW = weights_get(W, fp4_w_bytes(in, rows), 0);
    const uint8_t *dS = weights_get(wscale_code, fp4_s_bytes(in, rows), 1);
    Carver c = {arena((size_t)batch * (in + qn + rows) * 4 + 3 * 256), 0};
    float *dq = carve(&c, (size_t)batch * in * 4), *ds = carve(&c, (size_t)batch * qn * 4);
    float *dy = carve(&c, (size_t)batch * rows * 4);
    up_rows(dq, qx, batch, (size_t)in);
    up_rows(ds, qscale, batch, qn);
    check(dsv4g_gemv_fp4_batch_q(dy, dq, ds, batch, dW, dS, in, rows, NULL), "gemv_fp4");
    down_rows(y, dy, batch, (size_t)rows);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_fp4_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *wscale_code, int in, int rows)
{
    dsv4_gemv_fp4_batch_q(&y, &qx, &qscale, 1, W, wscale_code, in, rows);
}

void dsv4_gemv_fp4_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int rows)
{
    if (rows <= 0) return;
    pthread_mutex_lock(&g_lock);
    const size_t qn = (size_t)(in + 127) / 128;
    const uint8_t *dW0 = weights_get(W0, fp4_w_bytes(in, rows), 0);
    const uint8_t *dS0 = weights_get(S0, fp4_s_bytes(in, rows), 1);
    const uint8_t *dW1 = weights_get(W1, fp4_w_bytes(in, rows), 2);
    const uint8_t *dS1 = weights_get(S1, fp4_s_bytes(in, rows), 3);
    Carver c = {arena(((size_t)in + qn + 2 * (size_t)rows) * 4 + 4 * 256), 0};
    float *dq = carve(&c, (size_t)in * 4), *ds = carve(&c, qn * 4);
    float *d0 = carve(&c, (size_t)rows * 4), *d1 = carve(&c, (size_t)rows * 4);
    up(dq, qx, (size_t)in * 4);
    up(ds, qscale, qn * 4);
    check(dsv4g_gemv_fp4_pair_q(d0, d1, dq, ds, dW0, dS0, dW1, dS1, in, rows, NULL),
          "gemv_fp4_pair");
    down(y0, d0, (size_t)rows * 4);
    down(y1, d1, (size_t)rows * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_fp8_batch_q(float *const *y, const float *const *qx,
                           const float *const *qscale, int batch, const uint8_t *W,
                           const uint8_t *wscale_code, int in, int out, int round_out)
{
    if (batch <= 0 || out <= 0) return;
    batch_guard(batch, "FP8");
    pthread_mutex_lock(&g_lock);
    const size_t qn = (size_t)(in + 127) / 128;
    const uint8_t *dW = weights_get(W, fp8_w_bytes(in, out), 0);
    const uint8_t *dS = weights_get(wscale_code, fp8_s_bytes(in, out), 1);
    Carver c = {arena((size_t)batch * (in + qn + out) * 4 + 3 * 256), 0};
    float *dq = carve(&c, (size_t)batch * in * 4), *ds = carve(&c, (size_t)batch * qn * 4);
    float *dy = carve(&c, (size_t)batch * out * 4);
    up_rows(dq, qx, batch, (size_t)in);
    up_rows(ds, qscale, batch, qn);
    check(dsv4g_gemv_fp8_batch_q(dy, dq, ds, batch, dW, dS, in, out, round_out, NULL),
          "gemv_fp8");
    down_rows(y, dy, batch, (size_t)out);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_fp8_q(float *y, const float *qx, const float *qscale, const uint8_t *W,
                     const uint8_t *wscale_code, int in, int out, int round_out)
{
    dsv4_gemv_fp8_batch_q(&y, &qx, &qscale, 1, W, wscale_code, in, out, round_out);
}

void dsv4_gemv_fp8_pair_q(float *y0, float *y1, const float *qx, const float *qscale,
                          const uint8_t *W0, const uint8_t *S0, const uint8_t *W1,
                          const uint8_t *S1, int in, int out)
{
    if (out <= 0) return;
    pthread_mutex_lock(&g_lock);
    const size_t qn = (size_t)(in + 127) / 128;
    const uint8_t *dW0 = weights_get(W0, fp8_w_bytes(in, out), 0);
    const uint8_t *dS0 = weights_get(S0, fp8_s_bytes(in, out), 1);
    const uint8_t *dW1 = weights_get(W1, fp8_w_bytes(in, out), 2);
    const uint8_t *dS1 = weights_get(S1, fp8_s_bytes(in, out), 3);
    Carver c = {arena(((size_t)in + qn + 2 * (size_t)out) * 4 + 4 * 256), 0};
    float *dq = carve(&c, (size_t)in * 4), *ds = carve(&c, qn * 4);
    float *d0 = carve(&c, (size_t)out * 4), *d1 = carve(&c, (size_t)out * 4);
    up(dq, qx, (size_t)in * 4);
    up(ds, qscale, qn * 4);
    check(dsv4g_gemv_fp8_pair_q(d0, d1, dq, ds, dW0, dS0, dW1, dS1, in, out, NULL),
          "gemv_fp8_pair");
    down(y0, d0, (size_t)out * 4);
    down(y1, d1, (size_t)out * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_bf16_batch(float *const *y, const float *const *x, int batch,
                          const uint16_t *W, int in, int out, int round_out)
{
    if (batch <= 0 || out <= 0) return;
    batch_guard(batch, "BF16");
    pthread_mutex_lock(&g_lock);
    const uint16_t *dW = weights_get(W, (size_t)in * out * 2, 0);
    Carver c = {arena((size_t)batch * (in + out) * 4 + 2 * 256), 0};
    float *dx = carve(&c, (size_t)batch * in * 4), *dy = carve(&c, (size_t)batch * out * 4);
    up_rows(dx, x, batch, (size_t)in);
    check(dsv4g_gemv_bf16(dy, dx, dW, in, out, round_out, batch, NULL), "gemv_bf16");
    down_rows(y, dy, batch, (size_t)out);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_bf16(float *y, const float *x, const uint16_t *W, int in, int out,
                    int round_out)
{
    dsv4_gemv_bf16_batch(&y, &x, 1, W, in, out, round_out);
}

static void gemv_fp8_float(float *y, const float *x, const uint8_t *W, const float *wscale,
                           int in, int rows, int block, int mode)
{
    if (rows <= 0) return;
    pthread_mutex_lock(&g_lock);
    const size_t nsc = (size_t)((rows + block - 1) / block) * ((in + block - 1) / block);
    const uint8_t *dW = weights_get(W, (size_t)rows * in, 0);
    const float *dS = weights_get(wscale, nsc * 4, 1);
    Carver c = {arena(((size_t)in + rows) * 4 + 512), 0};
    float *dx = carve(&c, (size_t)in * 4), *dy = carve(&c, (size_t)rows * 4);
    up(dx, x, (size_t)in * 4);
    check(dsv4g_gemv_fp8_float(dy, dx, dW, dS, in, rows, block, mode, NULL), "gemv_fp8");
    down(y, dy, (size_t)rows * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}

void dsv4_gemv_fp8(float *y, const float *x, const uint8_t *W, const float *wscale, int in,
                   int rows, int block)
{
    gemv_fp8_float(y, x, W, wscale, in, rows, block, 0);
}

void dsv4_gemv_fp8_tbl(float *y, const float *x, const uint8_t *W, const float *wscale,
                       int in, int rows, int block)
{
    gemv_fp8_float(y, x, W, wscale, in, rows, block, 1);
}

void dsv4_gemv_fp4(float *y, const float *qx, const float *qscale, const uint8_t *W,
                   const float *wscale, int in, int rows, int group)
{
    if (rows <= 0) return;
    pthread_mutex_lock(&g_lock);
    const size_t qn = (size_t)(in + 127) / 128;
    const size_t gcols = (size_t)(in + group - 1) / group;
    const uint8_t *dW = weights_get(W, fp4_w_bytes(in, rows), 0);
    const float *dS = weights_get(wscale, (size_t)rows * gcols * 4, 1);
    Carver c = {arena(((size_t)in + qn + rows) * 4 + 768), 0};
    float *dq = carve(&c, (size_t)in * 4), *ds = carve(&c, qn * 4);
    float *dy = carve(&c, (size_t)rows * 4);
    up(dq, qx, (size_t)in * 4);
    up(ds, qscale, qn * 4);
    check(dsv4g_gemv_fp4_float(dy, dq, ds, dW, dS, in, rows, group, NULL), "gemv_fp4");
    down(y, dy, (size_t)rows * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}

/* -------------------------------------------------------------- router ---- */
void dsv4_router(int *idx, float *wt, const float *x, const float *gate, const float *bias,
                 const int64_t *tid2eid, int token_id, int hidden, int n_experts, int topk,
                 int hash_layer, float route_scale, float rms_eps)
{
    (void)rms_eps; /* unused by the reference as well */
    if (topk <= 0) return;
    pthread_mutex_lock(&g_lock);
    /* gate is a BF16 matrix passed as const float * (src/dsv4/dsv4_ops.c:494) */
    const uint16_t *dG = weights_get(gate, (size_t)n_experts * hidden * 2, 0);
    const float *dB = bias ? weights_get(bias, (size_t)n_experts * 4, 1) : NULL;
    const int64_t *dT = NULL; /* hash layers: the token's tid2eid row only */
    Carver c = {arena(((size_t)hidden + 2 * (size_t)n_experts + 2 * (size_t)topk) * 4 +
                      (size_t)topk * 8 + 8 * 256), 0};
    float *dx = carve(&c, (size_t)hidden * 4);
    float *dz = carve(&c, (size_t)n_experts * 4), *da = carve(&c, (size_t)n_experts * 4);
    int *didx = carve(&c, (size_t)topk * 4);
    float *dwt = carve(&c, (size_t)topk * 4);
    int *dtok = carve(&c, 4);
    int64_t *drow = carve(&c, (size_t)topk * 8);
    up(dx, x, (size_t)hidden * 4);
    if (hash_layer) {
        int zero = 0;
        up(drow, tid2eid + (size_t)token_id * topk, (size_t)topk * 8);
        up(dtok, &zero, 4);
        dT = drow;
    }
    check(dsv4g_router_public(didx, dwt, dx, dG, dB, dT, dtok, hidden, n_experts, topk,
                              hash_layer, route_scale, dz, da, NULL),
          "router");
    down(idx, didx, (size_t)topk * 4);
    down(wt, dwt, (size_t)topk * 4);
    finish();
    pthread_mutex_unlock(&g_lock);
}
