/* ref_maple.c -- drives the reference maple.c MoE block, unmodified.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile against /root/reference
 * into oracle/_ref/libref_maple.so. One layer, every tq2 expert resident and
 * pinned, g_use_gpu = 0: the batched f32 router matmul, route_row, moe_start,
 * moe_finish and expert_apply (maple.c:582-805) run as in the default int8 build.
 */
#define main zz_maple_engine_main
#include "maple.c"
#undef main

static void *zz_calloc(size_t n) { return calloc(n ? n : 1, 1); }

int ref_maple_moe(int D, int MI, int E, int K, int norm_topk, float clamp,
                  const float *router, const uint8_t *experts, int64_t esz,
                  const float *X, int S, float *out, int *eidx, float *ewt, int *uniq,
                  int *nu) {
    if (K > MAXTOPK || K > E || E > MAXEXPERTS) return -1;
    M *m = zz_calloc(sizeof(M));
    Cfg *c = &m->c;
    c->hidden = D; c->n_layers = 1; c->n_experts = E; c->topk = K; c->moe_inter = MI;
    c->norm_topk_prob = norm_topk; c->mlp_clamp = clamp; c->slots_per_layer = E;
    c->eps = 1e-5f;
    m->L[0].router.fmt = FMT_F32; m->L[0].router.O = E; m->L[0].router.I = D;
    m->L[0].router.f = router;
    m->gate_b = tq2_tensor_bytes(MI, D);
    m->down_b = tq2_tensor_bytes(D, MI);
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

    Buf b;
    memset(&b, 0, sizeof b);
    b.S = S;
    b.act.q = zz_calloc((size_t)S * D); b.act.s = zz_calloc(sizeof(float) * (size_t)S * (D / 32));
    b.act.tot = zz_calloc(sizeof(float) * (size_t)S);
    b.eact.q = zz_calloc((size_t)S * D); b.eact.s = zz_calloc(sizeof(float) * (size_t)S * (D / 32));
    b.eact.tot = zz_calloc(sizeof(float) * (size_t)S);
    b.hact.q = zz_calloc((size_t)S * MI); b.hact.s = zz_calloc(sizeof(float) * (size_t)S * (MI / 32));
    b.hact.tot = zz_calloc(sizeof(float) * (size_t)S);
    b.egate = zz_calloc(sizeof(float) * (size_t)S * MI);
    b.eidx = zz_calloc(sizeof(int) * (size_t)S * K);
    b.ewt = zz_calloc(sizeof(float) * (size_t)S * K);
    b.rlog = zz_calloc(sizeof(float) * (size_t)S * E);
    b.rows = zz_calloc(sizeof(int) * (size_t)S + 4);
    b.roww = zz_calloc(sizeof(float) * (size_t)S + 4);
    b.uniq = zz_calloc(sizeof(int) * (size_t)E);

    moe_start(m, 0, X, out, S, &b);
    moe_finish(m, 0, X, out, S, &b);
    memcpy(eidx, b.eidx, sizeof(int) * (size_t)S * K);
    memcpy(ewt, b.ewt, sizeof(float) * (size_t)S * K);
    memcpy(uniq, b.uniq, sizeof(int) * (size_t)b.moe_nu);
    *nu = b.moe_nu;

    free(b.act.q); free(b.act.s); free(b.act.tot);
    free(b.eact.q); free(b.eact.s); free(b.eact.tot);
    free(b.hact.q); free(b.hact.s); free(b.hact.tot);
    free(b.egate); free(b.eidx); free(b.ewt); free(b.rlog); free(b.rows); free(b.roww);
    free(b.uniq);
    free(m->slots); free(m->ucount); free(m->q);
    pthread_mutex_destroy(&m->mu);
    pthread_cond_destroy(&m->cv);
    pthread_cond_destroy(&m->done);
    free(m);
    return 0;
}
