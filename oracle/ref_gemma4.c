/* ref_gemma4.c -- drives the reference gemma4.c MoE block, unmodified.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile against the sources in
 * /root/reference (never copied here) into oracle/_ref/libref_gemma4.so. The
 * engine translation unit is included whole, so its static route_row /
 * moe_start / moe_finish (gemma4.c:581-809) run exactly as the engine runs them.
 * The model struct is filled by hand for one layer with every expert resident
 * and pinned: slot_for (gemma4.c:520-540) always hits, no I/O thread is started,
 * and g_use_gpu stays 0, so the default int8 CPU path runs.
 */
#define main zz_gemma4_engine_main
#include "gemma4.c"
#undef main

static void *zz_calloc(size_t n) { return calloc(n ? n : 1, 1); }

static M *g4_model(int D, int MI, int E, int K, float eps, const float *router,
                   const float *rscale, const float *pes, const float *pre_ln,
                   const float *post_ln, const uint8_t *experts, int64_t esz) {
    M *m = zz_calloc(sizeof(M));
    Cfg *c = &m->c;
    c->hidden = D; c->n_layers = 1; c->n_experts = E; c->topk = K; c->moe_inter = MI;
    c->eps = eps; c->slots_per_layer = E;
    Layer *L = &m->L[0];
    L->router_proj.O = E; L->router_proj.I = D; L->router_proj.f = router;
    L->router_scale.f = rscale; L->router_pes.f = pes;
    L->pre_ffn_ln2.f = pre_ln; L->post_ffn_ln2.f = post_ln;
    m->gate_b = q40_tensor_bytes(MI, D);
    m->down_b = q40_tensor_bytes(D, MI);
    m->esz = esz;
    m->slots = zz_calloc(sizeof(Slot) * (size_t)E);
    for (int e = 0; e < E; e++) {
        m->slots[e].eid = e;
        m->slots[e].buf = (uint8_t *)experts + (size_t)e * (size_t)esz;
        m->slots[e].pinned = 1;
    }
    m->npin = E;
    m->ucount = zz_calloc(sizeof(int64_t) * (size_t)E);
    pthread_mutex_init(&m->mu, NULL);
    pthread_cond_init(&m->cv, NULL);
    pthread_cond_init(&m->done, NULL);
    m->qcap = E + 1;
    m->q = zz_calloc(sizeof(*m->q) * (size_t)m->qcap);
    return m;
}

static void g4_free_model(M *m) {
    free(m->slots); free(m->ucount); free(m->q);
    pthread_mutex_destroy(&m->mu);
    pthread_cond_destroy(&m->cv);
    pthread_cond_destroy(&m->done);
    free(m);
}

static void g4_buf(Buf *b, int D, int MI, int E, int K, int S) {
    memset(b, 0, sizeof *b);
    b->S = S;
    b->xn = zz_calloc(sizeof(float) * (size_t)D);
    b->gate = zz_calloc(sizeof(float) * ((size_t)MI + (size_t)S * K + 64));
    b->eout = zz_calloc(sizeof(float) * (size_t)2 * S * D);
    b->egate = zz_calloc(sizeof(float) * (size_t)S * (MI + 64));
    b->esx = zz_calloc(sizeof(float) * (size_t)S * (D / Q40_BLK + 8));
    b->ehs = zz_calloc(sizeof(float) * (size_t)S * (MI / Q40_BLK + 8));
    b->exq = zz_calloc((size_t)S * (D + 64));
    b->ehq = zz_calloc((size_t)S * (MI + 64));
    b->xq = zz_calloc((size_t)D + 64);
    b->hq = zz_calloc((size_t)MI + 64);
    b->sx = zz_calloc(sizeof(float) * (size_t)(D / Q40_BLK + 8));
    b->hs = zz_calloc(sizeof(float) * (size_t)(MI / Q40_BLK + 8));
    b->eidx = zz_calloc(sizeof(int) * (size_t)S * K);
    b->ewt = zz_calloc(sizeof(float) * (size_t)S * K);
    b->rows = zz_calloc(sizeof(int) * (size_t)S + 4);
    b->uniq = zz_calloc(sizeof(int) * (size_t)E);
}

static void g4_free_buf(Buf *b) {
    free(b->xn); free(b->gate); free(b->eout); free(b->egate); free(b->esx); free(b->ehs);
    free(b->exq); free(b->ehq); free(b->xq); free(b->hq); free(b->sx); free(b->hs);
    free(b->eidx); free(b->ewt); free(b->rows); free(b->uniq);
}

/* One MoE layer call: moe_start + moe_finish (gemma4.c:750-809). */
int ref_g4_moe(int D, int MI, int E, int K, float eps, const float *router,
               const float *rscale, const float *pes, const float *pre_ln,
               const float *post_ln, const uint8_t *experts, int64_t esz,
               const float *residual, int S, float *out, int *eidx, float *ewt,
               int *uniq, int *nu, float *xin) {
    if (K > MAXTOPK || K > E || E > 128) return -1;    /* moe_slots[128] in Buf */
    M *m = g4_model(D, MI, E, K, eps, router, rscale, pes, pre_ln, post_ln, experts, esz);
    Buf b;
    g4_buf(&b, D, MI, E, K, S);
    moe_start(m, 0, residual, out, S, &b);
    moe_finish(m, 0, out, S, &b);
    memcpy(eidx, b.eidx, sizeof(int) * (size_t)S * K);
    memcpy(ewt, b.ewt, sizeof(float) * (size_t)S * K);
    memcpy(uniq, b.uniq, sizeof(int) * (size_t)b.moe_nu);
    *nu = b.moe_nu;
    if (xin) memcpy(xin, b.eout + (size_t)S * D, sizeof(float) * (size_t)S * D);
    g4_free_buf(&b);
    g4_free_model(m);
    return 0;
}

/* The same call on a layer set up once (the engine's steady state: model and Buf
 * live across calls, as in gemma4.c's decode loop), for timing. Buf is sized for
 * Smax tokens. */
typedef struct { M *m; Buf b; int Smax; } G4Layer;

void *ref_g4_layer_new(int D, int MI, int E, int K, float eps, const float *router,
                       const float *rscale, const float *pes, const float *pre_ln,
                       const float *post_ln, const uint8_t *experts, int64_t esz, int Smax) {
    if (K > MAXTOPK || K > E || E > 128 || Smax < 1) return NULL;
    G4Layer *h = zz_calloc(sizeof *h);
    h->m = g4_model(D, MI, E, K, eps, router, rscale, pes, pre_ln, post_ln, experts, esz);
    g4_buf(&h->b, D, MI, E, K, Smax);
    h->Smax = Smax;
    return h;
}

int ref_g4_layer_call(void *hp, const float *residual, int S, float *out, int *nu) {
    G4Layer *h = hp;
    if (!h || S < 1 || S > h->Smax) return -1;
    moe_start(h->m, 0, residual, out, S, &h->b);
    moe_finish(h->m, 0, out, S, &h->b);
    if (nu) *nu = h->b.moe_nu;
    return 0;
}

void ref_g4_layer_free(void *hp) {
    G4Layer *h = hp;
    if (!h) return;
    g4_free_buf(&h->b);
    g4_free_model(h->m);
    free(h);
}

/* route_row alone (gemma4.c:581-613), one token. */
int ref_g4_route(int D, int E, int K, float eps, const float *router, const float *rscale,
                 const float *pes, const float *residual, int *idx, float *wts) {
    if (K > MAXTOPK || K > E) return -1;
    M *m = g4_model(D, 64, E, K, eps, router, rscale, pes, NULL, NULL, NULL, 0);
    Buf b;
    memset(&b, 0, sizeof b);
    b.xn = zz_calloc(sizeof(float) * (size_t)D);
    route_row(m, 0, residual, idx, wts, &b);
    free(b.xn);
    g4_free_model(m);
    return 0;
}

/* expert_apply_batch_cpu for one expert and `n` rows of X (gemma4.c:618-654),
 * dumping the int8 activations and the int8 hidden it quantised. */
int ref_g4_expert(int D, int MI, const uint8_t *blob, const float *X, const int *rows,
                  int n, const float *w, float *OUT, int8_t *xq, float *sx, int8_t *hq,
                  float *hs) {
    M *m = g4_model(D, MI, 1, 1, 1e-6f, NULL, NULL, NULL, NULL, NULL, blob, 0);
    int S = 0;
    for (int r = 0; r < n; r++) if (rows[r] + 1 > S) S = rows[r] + 1;
    Buf b;
    g4_buf(&b, D, MI, 1, 1, n > S ? n : S);
    expert_apply_batch_cpu(m, blob, blob + m->gate_b, blob + 2 * m->gate_b,
                           q40_row_bytes(D), q40_row_bytes(MI), X, OUT, rows, n, w, &b);
    for (int r = 0; r < n; r++) {
        if (xq) memcpy(xq + (size_t)r * D, b.exq + (size_t)r * (D + 64), (size_t)D);
        if (sx) memcpy(sx + (size_t)r * (D / 32), b.esx + (size_t)r * (D / Q40_BLK + 8), sizeof(float) * (D / 32));
        if (hq) memcpy(hq + (size_t)r * MI, b.ehq + (size_t)r * (MI + 64), (size_t)MI);
        if (hs) memcpy(hs + (size_t)r * (MI / 32), b.ehs + (size_t)r * (MI / Q40_BLK + 8), sizeof(float) * (MI / 32));
    }
    g4_free_buf(&b);
    g4_free_model(m);
    return 0;
}

/* The feed-forward half of layer_fwd (gemma4.c:1003-1030) with attention as the
 * identity: the engine's own moe_start / moe_finish, rmsnorm, matvec and gelu_tanh,
 * called in the order of those lines on its Buf (res = b->eout as there). The dense
 * MLP record is mlp_gate [DI, D] | mlp_up [DI, D] | mlp_down [D, DI] in q4_0. */
int ref_g4_ffn_block(int D, int MI, int E, int K, int DI, float eps, const float *router,
                     const float *rscale, const float *pes, const float *pre_ln2,
                     const float *post_ln2, const uint8_t *experts, int64_t esz,
                     const uint8_t *mlp, const float *pre_ffn_ln, const float *post_ffn_ln1,
                     const float *post_ffn_ln, float layer_scalar, float *H, int S,
                     int *eidx, float *ewt) {
    if (K > MAXTOPK || K > E || E > 128) return -1;
    M *m = g4_model(D, MI, E, K, eps, router, rscale, pes, pre_ln2, post_ln2, experts, esz);
    Buf b;
    g4_buf(&b, D, MI, E, K, S);
    const int IM = D > DI ? D : DI;
    float *gate = zz_calloc(sizeof(float) * (size_t)DI), *up = zz_calloc(sizeof(float) * (size_t)DI);
    float *act = zz_calloc(sizeof(float) * (size_t)DI), *tmp = zz_calloc(sizeof(float) * (size_t)D);
    float *h2 = zz_calloc(sizeof(float) * (size_t)S * D);
    int8_t *xq = zz_calloc((size_t)IM + 64);
    float *sx = zz_calloc(sizeof(float) * (size_t)(IM / Q40_BLK + 8));
    size_t gb = q40_tensor_bytes(DI, D);
    W wg = {0, DI, D, mlp, NULL}, wu = {0, DI, D, mlp + gb, NULL}, wd = {0, D, DI, mlp + 2 * gb, NULL};
    float *res = b.eout;
    memcpy(res, H, sizeof(float) * (size_t)S * D);
    moe_start(m, 0, res, h2, S, &b);
    for (int s = 0; s < S; s++) {
        rmsnorm(b.xn, res + (size_t)s * D, pre_ffn_ln, D, eps);
        matvec(gate, &wg, b.xn, xq, sx);
        matvec(up, &wu, b.xn, xq, sx);
        for (int i = 0; i < DI; i++) act[i] = gelu_tanh(gate[i]) * up[i];
        float *h1 = H + (size_t)s * D;
        matvec(h1, &wd, act, xq, sx);
        rmsnorm(h1, h1, post_ffn_ln1, D, eps);
    }
    moe_finish(m, 0, h2, S, &b);
    for (int s = 0; s < S; s++) {
        const float *r = res + (size_t)s * D;
        float *h1 = H + (size_t)s * D, *hb = h2 + (size_t)s * D;
        for (int i = 0; i < D; i++) tmp[i] = h1[i] + hb[i];
        rmsnorm(tmp, tmp, post_ffn_ln, D, eps);
        for (int i = 0; i < D; i++) h1[i] = (r[i] + tmp[i]) * layer_scalar;
    }
    if (eidx) memcpy(eidx, b.eidx, sizeof(int) * (size_t)S * K);
    if (ewt) memcpy(ewt, b.ewt, sizeof(float) * (size_t)S * K);
    free(gate); free(up); free(act); free(tmp); free(h2); free(xq); free(sx);
    g4_free_buf(&b);
    g4_free_model(m);
    return 0;
}

/* embed_row (gemma4.c:1131-1145) from a q4_0 [V, D] table. */
int ref_g4_embed(const uint8_t *table, int V, int D, float embed_scale, int tok, float *h) {
    M *m = g4_model(D, 64, 1, 1, 1e-6f, NULL, NULL, NULL, NULL, NULL, NULL, 0);
    m->c.embed_scale = embed_scale;
    m->c.vocab = V;
    m->L[MAXL - 1].q_proj.q = table;
    m->L[MAXL - 1].q_proj.O = V;
    m->L[MAXL - 1].q_proj.I = D;
    embed_row(m, tok, h);
    g4_free_model(m);
    return 0;
}

/* The head of forward() for one row (gemma4.c:1264-1275: final rmsnorm, tied lm_head
 * matvec, softcap) and the greedy token of sample() at temp 0 (gemma4.c:2149-2152). */
int ref_g4_head(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
                const float *h, float *logits) {
    float *xn = zz_calloc(sizeof(float) * (size_t)D);
    int8_t *xq = zz_calloc((size_t)D + 64);
    float *sx = zz_calloc(sizeof(float) * (size_t)(D / Q40_BLK + 8));
    W we = {0, V, D, table, NULL};
    rmsnorm(xn, h, fnorm, D, eps);
    matvec(logits, &we, xn, xq, sx);
    if (softcap > 0)
        for (int i = 0; i < V; i++) logits[i] = tanhf(logits[i] / softcap) * softcap;
    uint64_t rng = 1;
    int tok = sample(logits, V, 0.0f, 1.0f, 0, NULL, &rng);
    free(xn); free(xq); free(sx);
    return tok;
}

/* The engine's FlashHead, flash_logits (gemma4.c:1055-1110), on one row: the model
 * holds only the tied table and the four flash tensors, the buffers only what
 * flash_logits touches. rmsnorm with the final norm first, as forward() does
 * (gemma4.c:1239-1242); then the greedy token by sample at temp 0. */
int ref_g4_flash(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
                 const uint8_t *cent, int NC, const int32_t *tmap, int CS, int NP,
                 const float *cscale, int scaled, const int32_t *force, int nforce,
                 const float *h, float *logits) {
    M *m = zz_calloc(sizeof(M));
    Cfg *c = &m->c;
    c->hidden = D; c->vocab = V; c->eps = eps; c->final_logit_softcap = softcap;
    c->flash_n_clusters = NC; c->flash_cluster_size = CS; c->flash_n_probes = NP;
    c->flash_scaled_centroids = scaled; c->flash_n_force = nforce;
    m->L[MAXL - 1].q_proj = (W){0, V, D, table, NULL};
    m->flash_centroids = (W){0, NC, D, cent, NULL};
    m->flash_token_map = (W){5, NC, CS, (const uint8_t *)tmap, NULL};
    m->flash_cluster_scale = (W){0, 1, NC, NULL, cscale};
    m->flash_force = (W){5, 1, nforce, (const uint8_t *)force, NULL};
    m->use_flash = 1;
    Buf b;
    memset(&b, 0, sizeof b);
    b.xn = zz_calloc(sizeof(float) * (size_t)D);
    b.xq = zz_calloc((size_t)D + 64);
    b.sx = zz_calloc(sizeof(float) * (size_t)(D / Q40_BLK + 8));
    b.fsim = zz_calloc(sizeof(float) * ((size_t)NC + 64));
    b.fsel = zz_calloc(sizeof(int) * ((size_t)NC + 64));
    b.fids = zz_calloc(sizeof(int) * ((size_t)NP * CS + nforce + 64));
    rmsnorm(b.xn, h, fnorm, D, eps);
    flash_logits(m, b.xn, logits, &b);
    uint64_t rng = 1;
    int tok = sample(logits, V, 0.0f, 1.0f, 0, NULL, &rng);
    free(b.xn); free(b.xq); free(b.sx); free(b.fsim); free(b.fsel); free(b.fids);
    free(m);
    return tok;
}

/* The engine's own container reader, manifest() (gemma4.c:260-403), on a directory:
 * the record size, every expert offset (n_layers * n_experts), layer 0's router,
 * each layer's layer_scalar, the final norm, embed_tokens row 0, and the bytes of
 * expert (li, e) read at the engine's offset. Returns n_layers, or -1. */
int ref_g4_manifest_probe(const char *dir, int64_t *esz3, int64_t *eoff, float *router0,
                          float *scalars, float *fnorm, uint8_t *embed_row0, int li, int e,
                          uint8_t *rec) {
    M *m = zz_calloc(sizeof(M));
    manifest(m, dir);
    Cfg *c = &m->c;
    esz3[0] = m->esz; esz3[1] = m->gate_b; esz3[2] = m->down_b;
    memcpy(eoff, m->eoff, sizeof(int64_t) * (size_t)c->n_layers * c->n_experts);
    memcpy(router0, m->L[0].router_proj.f, sizeof(float) * (size_t)c->n_experts * c->hidden);
    for (int l = 0; l < c->n_layers; l++) scalars[l] = m->L[l].layer_scalar.f[0];
    memcpy(fnorm, m->L[MAXL - 1].o_proj.f, sizeof(float) * (size_t)c->hidden);
    memcpy(embed_row0, m->L[MAXL - 1].q_proj.q, q40_row_bytes(c->hidden));
    int64_t off = m->eoff[(int64_t)li * c->n_experts + e], esz = m->esz;
    ssize_t r = pread(m->efd, rec, (size_t)esz, off);
    int nl = c->n_layers;
    close(m->efd);
    free(m->eoff); free(m->dense); free(m);
    return r == (ssize_t)esz ? nl : -1;
}

void ref_g4_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
