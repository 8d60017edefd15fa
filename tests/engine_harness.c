/* engine_harness.c -- an engine-shaped C caller of libzzmoe.so.
 *
 * TEST INFRASTRUCTURE. It plays the part of a zunzuncito engine's MoE block: the
 * layer is registered once at load (zz_moe_layer_create + one expert upload per
 * record, as the engine's slot fill would do), then each forward goes through
 * moe_start / moe_finish written the way an engine's would be patched
 * (gemma4.c:750 / 792, lfm25.c:837 / 891): moe_start tries zz_moe_forward_begin and
 * otherwise runs the CPU path; moe_finish collects with zz_moe_forward_end and, on a
 * late decline, runs the CPU path too. The CPU path here is the repository's CPU
 * restatement of the reference's moe_start + moe_finish (oracle/), standing in for
 * the engine's own code. Built by tests/Makefile with gcc against the headers in include/
 * and linked with -lzzmoe.
 *
 *   engine_harness <case.bin> <result.bin>
 *
 * case.bin: an int32 header (D MI E K gating act fmt_gate fmt_up fmt_down norm_topk
 * use_bias n_group topk_group S has_scale has_pes has_bias has_norms), three f32
 * (eps routed_scaling clamp), the int64 record size, then the f32 router [E*D],
 * router_scale [D], pes [E], bias [E], pre_ln [D], post_ln [D] (each only when
 * present), the expert records [E*esz] and the input [S*D].
 * result.bin: out [S*D] f32, eidx [S*K] i32, ewt [S*K] f32.
 * stdout: "path gpu" or "path cpu", then the decline checks' verdict.
 */
#include "zz_moe.h"
#include "zz_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    zz_moe_desc d;
    orc_cfg c;
    orc_weights w;
    int zz;                 /* the GPU layer id, -1 when not registered */
} Layer;

typedef struct {            /* the engine's per-call buffers (Buf in gemma4.c) */
    int live;               /* a GPU forward is pending */
    const float *res;       /* moe_start's input, kept for a late decline */
    int *eidx;
    float *ewt;
} Buf;

static void cpu_moe(Layer *L, const float *in, float *out, int S, Buf *b) {
    int uniq[512], nu = 0;
    if (orc_moe_layer(&L->c, &L->w, in, S, out, b->eidx, b->ewt, uniq, &nu, NULL) != 0) {
        fprintf(stderr, "cpu path: bad layer config\n");
        exit(2);
    }
}

static const char *g_path = "none";

/* gemma4.c:750 moe_start: the GPU first, the reference body as the fallback */
static void moe_start(Layer *L, const float *residual, float *out, int S, Buf *b) {
    b->res = residual;
    b->live = L->zz >= 0 && zz_moe_forward_begin(L->zz, residual, S);
    if (b->live) return;                       /* the dense branch would run meanwhile */
    g_path = "cpu";
    cpu_moe(L, residual, out, S, b);
}

/* gemma4.c:792 moe_finish */
static void moe_finish(Layer *L, float *out, int S, Buf *b) {
    if (!b->live) return;
    b->live = 0;
    if (zz_moe_forward_end(L->zz, out, b->eidx, b->ewt)) {
        g_path = "gpu";
        return;
    }
    g_path = "cpu";                            /* late decline: the CPU path */
    cpu_moe(L, b->res, out, S, b);
}

static void *slurp(FILE *f, size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p || fread(p, 1, n, f) != n) {
        fprintf(stderr, "short read (%zu bytes)\n", n);
        exit(2);
    }
    return p;
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s case.bin result.bin\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) { perror(argv[1]); return 2; }
    int h[18];
    float hf[3];
    int64_t esz;
    if (fread(h, sizeof h, 1, f) != 1 || fread(hf, sizeof hf, 1, f) != 1 || fread(&esz, 8, 1, f) != 1) {
        fprintf(stderr, "bad header\n");
        return 2;
    }
    Layer L;
    memset(&L, 0, sizeof L);
    zz_moe_desc *d = &L.d;
    d->D = h[0]; d->MI = h[1]; d->E = h[2]; d->K = h[3]; d->gating = h[4]; d->act = h[5];
    d->fmt_gate = h[6]; d->fmt_up = h[7]; d->fmt_down = h[8]; d->norm_topk = h[9];
    d->use_bias = h[10]; d->n_group = h[11]; d->topk_group = h[12];
    d->eps = hf[0]; d->routed_scaling = hf[1]; d->clamp = hf[2];
    const int S = h[13], D = d->D, E = d->E, K = d->K;
    float *router = slurp(f, sizeof(float) * (size_t)E * D);
    float *rscale = h[14] ? slurp(f, sizeof(float) * D) : NULL;
    float *pes = h[15] ? slurp(f, sizeof(float) * E) : NULL;
    float *bias = h[16] ? slurp(f, sizeof(float) * E) : NULL;
    float *pre = h[17] ? slurp(f, sizeof(float) * D) : NULL;
    float *post = h[17] ? slurp(f, sizeof(float) * D) : NULL;
    uint8_t *experts = slurp(f, (size_t)E * esz);
    float *x = slurp(f, sizeof(float) * (size_t)S * D);
    fclose(f);

    orc_cfg *c = &L.c;
    c->D = D; c->MI = d->MI; c->E = E; c->K = K; c->gating = d->gating; c->act = d->act;
    c->fmt_gate = d->fmt_gate; c->fmt_up = d->fmt_up; c->fmt_down = d->fmt_down;
    c->norm_topk = d->norm_topk; c->use_bias = d->use_bias; c->eps = d->eps;
    c->routed_scaling = d->routed_scaling; c->clamp = d->clamp;
    c->n_group = d->n_group; c->topk_group = d->topk_group;
    L.w.router = router; L.w.router_scale = rscale; L.w.pes = pes; L.w.bias = bias;
    L.w.pre_ln = pre; L.w.post_ln = post; L.w.experts = experts; L.w.esz = esz;

    /* load time: register the layer and fill its slot table (gemma4.c:2046-2058 fills
     * slots lazily from experts.bin; with every expert resident it is done once) */
    L.zz = -1;
    if (gpu_init()) {
        zz_moe_weights w = {router, rscale, pes, bias, pre, post};
        L.zz = zz_moe_layer_create(d, &w);
        if (L.zz >= 0 && zz_moe_record_bytes(d) != esz) {
            fprintf(stderr, "record size mismatch\n");
            return 2;
        }
        for (int e = 0; L.zz >= 0 && e < E; e++)
            if (!zz_moe_expert_upload(L.zz, e, experts + (size_t)e * esz, (size_t)esz)) {
                fprintf(stderr, "upload declined (%s): CPU path\n", zz_last_error());
                zz_moe_layer_destroy(L.zz);
                L.zz = -1;
            }
    }

    float *out = malloc(sizeof(float) * (size_t)S * D);
    Buf b;
    memset(&b, 0, sizeof b);
    b.eidx = malloc(sizeof(int) * (size_t)S * K);
    b.ewt = malloc(sizeof(float) * (size_t)S * K);
    moe_start(&L, x, out, S, &b);
    /* ... the engine's dense MLP runs here (gemma4.c:1012-1020) ... */
    moe_finish(&L, out, S, &b);
    printf("path %s\n", g_path);

    /* the decline contract: a refused call leaves its outputs untouched */
    int ok = 1;
    if (gpu_ready()) {
        float *sent = malloc(sizeof(float) * (size_t)S * D);
        for (size_t i = 0; i < (size_t)S * D; i++) sent[i] = 7.0f;
        ok &= zz_moe_forward(L.zz >= 0 ? L.zz + 1000 : 1000, x, sent, S, NULL, NULL) == 0;  /* no such layer */
        ok &= zz_moe_forward(L.zz, x, sent, 0, NULL, NULL) == 0;                               /* S = 0 */
        ok &= zz_moe_forward_end(L.zz, sent, NULL, NULL) == 0;                                  /* nothing pending */
        for (size_t i = 0; i < (size_t)S * D; i++) ok &= sent[i] == 7.0f;
        free(sent);
    }
    printf("declines %s\n", ok ? "ok" : "BROKEN");

    FILE *g = fopen(argv[2], "wb");
    if (!g || fwrite(out, sizeof(float), (size_t)S * D, g) != (size_t)S * D ||
        fwrite(b.eidx, sizeof(int), (size_t)S * K, g) != (size_t)S * K ||
        fwrite(b.ewt, sizeof(float), (size_t)S * K, g) != (size_t)S * K) {
        fprintf(stderr, "cannot write %s\n", argv[2]);
        return 2;
    }
    fclose(g);
    if (L.zz >= 0) zz_moe_layer_destroy(L.zz);
    gpu_shutdown();
    return ok ? 0 : 1;
}
