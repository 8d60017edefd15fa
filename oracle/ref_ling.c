/* ref_ling.c -- drives the reference ling.c MoE block, unmodified.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile against /root/reference
 * into oracle/_ref/libref_ling.so. One layer, every expert resident and pinned,
 * g_use_gpu = 0: the grouped route_row, moe_start, moe_finish and expert_apply
 * (ling.c:705-1043) run as in the engine's default int8 build. The shared expert
 * (shared_fwd) sits outside the MoE block and is not called. One expert format per
 * layer (q4_0 or q8_0).
 */
#define main zz_ling_engine_main
#include "ling.c"
#undef main

static void *zz_calloc(size_t n) { return calloc(n ? n : 1, 1); }

int ref_ling_moe(int D, int MI, int E, int K, int fmt, int n_group, int topk_group,
                 int norm_topk, float routed_scale, const float *router, const float *bias,
                 const uint8_t *experts, int64_t esz, const float *X, int S,
                 float *out, int *eidx, float *ewt, int *uniq, int *nu) {
    if (K > MAXTOPK || K > E || E > MAXEXPERTS || n_group > MAXGROUP) return -1;
    if (fmt != FMT_Q40 && fmt != FMT_Q80) return -1;
    M *m = zz_calloc(sizeof(M));
    Cfg *c = &m->c;
    c->hidden = D; c->n_layers = 1; c->n_experts = E; c->topk = K; c->moe_inter = MI;
    c->n_group = n_group; c->topk_group = topk_group; c->norm_topk_prob = norm_topk;
    c->routed_scale = routed_scale; c->slots_per_layer = E; c->eps = 1e-6f;
    m->L[0].router.O = E; m->L[0].router.I = D; m->L[0].router.f = router;
    m->L[0].expert_bias.f = bias;
    m->expert_fmt[0] = fmt;
    m->gate_b[0] = fmt_row_bytes(fmt, D) * MI;
    m->down_b[0] = fmt_row_bytes(fmt, MI) * D;
    m->esz[0] = esz;
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

    Buf b;
    memset(&b, 0, sizeof b);
    b.eidx = zz_calloc(sizeof(int) * (size_t)S * K);
    b.ewt = zz_calloc(sizeof(float) * (size_t)S * K);
    b.rwt = zz_calloc(sizeof(float) * (size_t)E);
    b.rsel = zz_calloc(sizeof(float) * (size_t)E);
    b.rows = zz_calloc(sizeof(int) * (size_t)S + 4);
    b.roww = zz_calloc(sizeof(float) * (size_t)S + 4);
    b.uniq = zz_calloc(sizeof(int) * (size_t)E);
    b.exq = zz_calloc((size_t)S * (D + 64));
    b.esx = zz_calloc(sizeof(float) * (size_t)S * (D / Q40_BLK + 8));
    b.egate = zz_calloc(sizeof(float) * (size_t)S * (MI + 64));
    b.ehq = zz_calloc((size_t)S * (MI + 64));
    b.ehs = zz_calloc(sizeof(float) * (size_t)S * (MI / Q40_BLK + 8));
    b.xq = zz_calloc((size_t)D + 64);
    b.sx = zz_calloc(sizeof(float) * (size_t)(D / Q40_BLK + 8));
    b.gate = zz_calloc(sizeof(float) * (size_t)(MI + 64));
    b.hq = zz_calloc((size_t)MI + 64);
    b.hs = zz_calloc(sizeof(float) * (size_t)(MI / Q40_BLK + 8));

    moe_start(m, 0, X, out, S, 0, &b);
    moe_finish(m, 0, X, out, S, &b);
    memcpy(eidx, b.eidx, sizeof(int) * (size_t)S * K);
    memcpy(ewt, b.ewt, sizeof(float) * (size_t)S * K);
    memcpy(uniq, b.uniq, sizeof(int) * (size_t)b.moe_nu);
    *nu = b.moe_nu;

    free(b.eidx); free(b.ewt); free(b.rwt); free(b.rsel); free(b.rows); free(b.roww);
    free(b.uniq); free(b.exq); free(b.esx); free(b.egate); free(b.ehq); free(b.ehs);
    free(b.xq); free(b.sx); free(b.gate); free(b.hq); free(b.hs);
    free(m->slots); free(m->ucount); free(m->q);
    pthread_mutex_destroy(&m->mu);
    pthread_cond_destroy(&m->cv);
    pthread_cond_destroy(&m->done);
    free(m);
    return 0;
}
