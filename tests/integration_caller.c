/* integration_caller.c - the decode caller of INTEGRATION.md section 1
 * (GpuMoE, gpu_moe_forward) compiled as it stands, on a small synthetic
 * layer in the library's formats. Used by tests/test_gpu_status.py:
 *
 *   integration_caller            one token through gpu_moe_forward; prints
 *                                 "ok" and exits 0
 *   integration_caller preset     the same after the host has set the
 *                                 workspace's sticky status word (its first
 *                                 32-bit word): every cross-workgroup wait
 *                                 gives up at its first status check, every
 *                                 kernel ends normally, and the caller must
 *                                 take the fatal path (exit 1 with a message)
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dsv4_gpu.h"

typedef struct {
    DSV4GLayer L;          /* device pointers, see dsv4_gpu.h */
    void *ws;              /* decode workspace */
    size_t ws_bytes;
    void *bws;             /* batch workspace */
    size_t bws_bytes;
    float *x_dev, *out_dev;
    int *tok_dev;
} GpuMoE;

/* moe_forward(m, w, x, out, ...) for one token */
static void gpu_moe_forward(GpuMoE *g, const float *x, int token_id, float *out) {
    unsigned st = 0;
    if (dsv4g_memcpy_h2d(g->x_dev, x, g->L.hidden * sizeof(float), NULL) ||
        dsv4g_memcpy_h2d(g->tok_dev, &token_id, sizeof(int), NULL) ||
        dsv4g_moe_forward(g->out_dev, g->x_dev, &g->L, g->tok_dev, 1,
                          g->ws, g->ws_bytes, NULL, NULL, NULL) ||
        dsv4g_memcpy_d2h(out, g->out_dev, g->L.hidden * sizeof(float), NULL) ||  /* syncs */
        dsv4g_moe_decode_status(&st, g->ws, NULL)) {
        fprintf(stderr, "dsv4: %s\n", dsv4g_last_error());
        exit(1);                                   /* the reference's fatal path */
    }
    if (st) {  /* a cross-workgroup wait of the layer ran out: out is not valid */
        fprintf(stderr, "dsv4: MoE decode failed on the GPU (status %#x)\n", st);
        exit(1);
    }
}

static void die(const char *what) {
    fprintf(stderr, "integration_caller: %s: %s\n", what, dsv4g_last_error());
    exit(2);
}

static unsigned rng_state = 12345u;
static unsigned rnd(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 17;
    rng_state ^= rng_state << 5;
    return rng_state;
}

/* device buffer of n bytes filled by fill(i) */
static void *dev_bytes(size_t n, int kind) {
    unsigned char *h = malloc(n);
    void *d = NULL;
    if (!h) exit(2);
    for (size_t i = 0; i < n; i++) {
        if (kind == 0) h[i] = (unsigned char)rnd();           /* packed FP4 / FP8 codes */
        else h[i] = (unsigned char)(120 + rnd() % 8);         /* E8M0 scales near 1 */
    }
    if (dsv4g_malloc(&d, n) || dsv4g_memcpy_h2d(d, h, n, NULL)) die("upload");
    free(h);
    return d;
}

int main(int argc, char **argv) {
    const int H = 256, I = 128, E = 16, K = 6;
    GpuMoE g;
    memset(&g, 0, sizeof g);
    g.L.hidden = H;  g.L.inter = I;  g.L.n_experts = E;  g.L.topk = K;
    g.L.route_scale = 1.5f;  g.L.swiglu_limit = 10.0f;
    /* gate: BF16 values of small magnitude */
    {
        unsigned short *h = malloc((size_t)E * H * 2);
        for (int i = 0; i < E * H; i++) {
            float v = ((int)(rnd() % 2001) - 1000) * 2e-5f;
            unsigned u;
            memcpy(&u, &v, 4);
            h[i] = (unsigned short)(u >> 16);
        }
        void *d = NULL;
        if (dsv4g_malloc(&d, (size_t)E * H * 2) || dsv4g_memcpy_h2d(d, h, (size_t)E * H * 2, NULL))
            die("gate");
        g.L.gate_w = d;
        free(h);
    }
    const size_t s1 = (size_t)I * (H / 32), s2 = (size_t)H * (I / 32);
    const size_t w1 = (size_t)I * (H / 2), w2 = (size_t)H * (I / 2);
    g.L.scale_run = 2 * s1 + s2;
    g.L.expert_stride = g.L.scale_run + 2 * w1 + w2;
    {
        unsigned char *h = malloc(E * g.L.expert_stride);
        for (int e = 0; e < E; e++)
            for (size_t i = 0; i < g.L.expert_stride; i++)
                h[e * g.L.expert_stride + i] =
                    i < g.L.scale_run ? (unsigned char)(120 + rnd() % 8) : (unsigned char)rnd();
        void *d = NULL;
        if (dsv4g_malloc(&d, E * g.L.expert_stride) ||
            dsv4g_memcpy_h2d(d, h, E * g.L.expert_stride, NULL))
            die("experts");
        g.L.experts = d;
        free(h);
    }
    g.L.sh1 = dev_bytes((size_t)I * H, 0);  g.L.sh1_s = dev_bytes(((I + 127) / 128) * ((H + 127) / 128), 1);
    g.L.sh3 = dev_bytes((size_t)I * H, 0);  g.L.sh3_s = dev_bytes(((I + 127) / 128) * ((H + 127) / 128), 1);
    g.L.sh2 = dev_bytes((size_t)H * I, 0);  g.L.sh2_s = dev_bytes(((H + 127) / 128) * ((I + 127) / 128), 1);
    g.ws_bytes = dsv4g_moe_workspace_bytes(&g.L, 1);
    if (dsv4g_malloc(&g.ws, g.ws_bytes)) die("workspace");
    if (dsv4g_moe_workspace_init(g.ws, g.ws_bytes, NULL)) die("workspace_init");
    if (dsv4g_malloc((void **)&g.x_dev, H * sizeof(float)) ||
        dsv4g_malloc((void **)&g.out_dev, H * sizeof(float)) ||
        dsv4g_malloc((void **)&g.tok_dev, sizeof(int)))
        die("buffers");
    float x[256], out[256];
    for (int i = 0; i < H; i++) {
        float v = ((int)(rnd() % 2001) - 1000) * 1e-3f;
        unsigned u;
        memcpy(&u, &v, 4);
        u &= 0xFFFF0000u; /* BF16-valued, as the caller's RMSNorm output */
        memcpy(&x[i], &u, 4);
    }
    if (argc > 1 && strcmp(argv[1], "preset") == 0) {
        const unsigned one = 1u;
        if (dsv4g_memcpy_h2d(g.ws, &one, sizeof one, NULL)) die("preset");
    }
    fprintf(stderr, "integration_caller: calling gpu_moe_forward (%s)\n",
            argc > 1 ? argv[1] : "plain");
    gpu_moe_forward(&g, x, 0, out);
    printf("ok %g\n", out[0]);
    return 0;
}
