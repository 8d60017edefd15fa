/* zz_oracle.h -- CPU restatement of the zunzuncito MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The HIP
 * library under zunzuncito_amd/ never links or calls it.
 *
 * Every function restates one reference routine (file:line into mseri/zunzuncito)
 * and is pinned by the tests listed in its comment:
 *   - the reference's own known-answer tests (tests/test_q40.c, tests/test_tq2.c),
 *   - bit-exact comparison against oracle/_ref (the reference sources compiled
 *     by oracle/Makefile, x86-64-v3 AVX2 path),
 *   - golden vectors in tests/golden/ written from oracle/_ref,
 *   - closed forms (numpy float16 for the fp16 codec, brute-force integer dots).
 * Floats follow the reference AVX2 build's operation order (lane partials, four
 * accumulators, FMA where gcc -O3 -march=x86-64-v3 contracts), so results are
 * bit-identical to the compiled reference, not merely close.
 */
#ifndef ZZ_ORACLE_H
#define ZZ_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight formats: same codes as gpu.h:49-52 */
#define ORC_FMT_Q40 1
#define ORC_FMT_Q80 2
#define ORC_FMT_TQ2 3
#define ORC_FMT_Q4A 4   /* f32-activation matmul only (tq2.h:269-292) */

/* gating kinds */
#define ORC_GATE_GEMMA 0    /* gemma4.c:581-613  rmsnorm->scale->f32 logits->topk->softmax(K)*pes */
#define ORC_GATE_LFM   1    /* lfm25.c:636-668   double logits->sigmoid->(+bias) topk->norm*scale  */
#define ORC_GATE_MAPLE 2    /* maple.c:582-601   double logits->topk->softmax(K)                    */
#define ORC_GATE_LING  4    /* ling.c:705-789    8-acc double logits->sigmoid(+bias)->groups->topk  */

/* activation kinds */
#define ORC_ACT_GEGLU_TANH 0   /* gemma4.c:432-434 */
#define ORC_ACT_SWIGLU     1   /* lfm25.c:456-458  */
#define ORC_ACT_SWIGLU_CL  2   /* maple.c:607-611 silu(min(g,c))*clip(u,-c,c) */

typedef struct {
    int D, MI, E, K;
    int gating, act;
    int fmt_gate, fmt_up, fmt_down;
    int norm_topk;          /* lfm/maple: renormalise the K weights          */
    int use_bias;           /* lfm: expert_bias on the selection score;
                               gemma: harness Zipf logit offset (0 = reference) */
    float eps;              /* gemma rmsnorm epsilon                          */
    float routed_scaling;   /* lfm                                            */
    float clamp;            /* maple mlp_clamp                                */
    int n_group, topk_group;/* ling: expert groups, groups kept               */
} orc_cfg;

typedef struct {
    const float *router;        /* [E, D] f32                                  */
    const float *router_scale;  /* [D]  gemma                                  */
    const float *pes;           /* [E]  gemma per-expert scale                 */
    const float *bias;          /* [E]  lfm expert_bias / gemma Zipf offset    */
    const float *pre_ln;        /* [D]  gemma pre_ffn_ln2                      */
    const float *post_ln;       /* [D]  gemma post_ffn_ln2                     */
    const uint8_t *experts;     /* E records of esz bytes: [gate | up | down]  */
    int64_t esz;                /* record stride in bytes                      */
} orc_weights;

/* Optional per-call dumps (any pointer may be NULL). */
typedef struct {
    float  *xin;     /* [S, D]   expert input after the gemma pre-norm (or X)   */
    int8_t *xq;      /* [S, D]   int8 activations                               */
    float  *xs;      /* [S, D/32] activation block scales                        */
    float  *xtot;    /* [S]      tq2 Sx of the expert input                      */
    int8_t *hq;      /* [S*K, MI] int8 hidden, by (token, slot)                  */
    float  *hs;      /* [S*K, MI/32]                                             */
    float  *htot;    /* [S*K]    tq2 Sx of the hidden                            */
    float  *logits;  /* [S, E]   router logits (gemma: after the optional bias)  */
} orc_dump;

/* ---- A1: fp16 codec (q40.h:46-80) ---- */
float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);

/* ---- A3/A7: weight quantisers (q40.h:83-121, 332-356) ---- */
void orc_q40_quant_row(const float *w, uint8_t *dst, int I);
void orc_q80_quant_row(const float *w, uint8_t *dst, int I);
void orc_q40_dequant_row(const uint8_t *src, float *w, int I);
void orc_q80_dequant_row(const uint8_t *src, float *w, int I);
/* tq2 tensor = alpha[O] f32 then codes[O][I/4] (tq2.h:17-28, 81-91);
 * codes[] are values in {0,1,2} in natural order, packed per tq2.h:46-51. */
void orc_tq2_pack_row(const int8_t *code, uint8_t *dst, int I);
void orc_tq2_dequant_row(const uint8_t *codes, float alpha, float *w, int I);

/* ---- A4/A8: activation quantisers (q40.h:124-138, tq2.h:98-108) ---- */
void  orc_quant_act(const float *x, int8_t *xq, float *sx, int I);
float orc_tq2_quant_act(const float *x, int8_t *xq, float *sx, int I);

/* ---- A5/A7/A8: int8-activation dots, AVX2 operation order ---- */
float orc_q40_dot(const uint8_t *w, const int8_t *xq, const float *sx, int I);
float orc_q80_dot(const uint8_t *w, const int8_t *xq, const float *sx, int I);
float orc_tq2_dot(const uint8_t *codes, float alpha, const int8_t *xq,
                  const float *sx, float sxtot, int I);
/* per-block exact int32 dots: q4_0 sum (q-8)*x, q8_0 sum q*x, tq2 sum (c-1)*x */
void orc_blockdots(int fmt, const uint8_t *row, const int8_t *xq, int I, int32_t *out);

/* ---- A6/A9: f32-activation dots, double accumulation (q40.h:290-305,
 *      443-455, tq2.h:235-252, 405-427) -- the gpu.h matmul contract ---- */
float orc_q40_dot_f32(const uint8_t *w, const float *x, int I);
float orc_q80_dot_f32(const uint8_t *w, const float *x, int I);
float orc_tq2_dot_f32(const uint8_t *codes, float alpha, const float *x, int I);
float orc_q4a_dot_f32(const uint8_t *w, const float *x, int I);
/* y[S,O] = W[O,I] x[S,I] for any format (gpu.h:71-84 semantics) */
void  orc_matmul_f32(int fmt, float *y, const uint8_t *W, const float *x, int O, int I, int S);

/* ---- sizes (q40.h:313-314, 461-462; tq2.h:81-86) ---- */
int64_t orc_tensor_bytes(int fmt, int O, int I);

/* ---- A18: norms and activations ---- */
void  orc_rmsnorm(float *o, const float *x, const float *w, int D, float eps);
float orc_act(int act, float g, float u, float clamp);

/* ---- A10-A12: routers, one token ---- */
/* Planted mistakes, for tests that show a pin rejects a plausible slip (0 = the
 * faithful oracle; anything else is never used outside those tests):
 *   1  gemma Zipf offset as the chain's starting value (added first, not last)
 *   2  gemma Zipf offset added before the chain's last product
 *   3  gemma Zipf offset in the softmax only (selection on unbiased logits)
 *   4  gemma Zipf offset in the selection only (softmax on unbiased logits)
 *   5  q8_0 dequantisation with the block scale of the previous block */
void orc_set_plant(int plant);
void orc_route(const orc_cfg *c, const orc_weights *w, const float *x,
               int *idx, float *wts, float *logits_out);

/* ---- A14-A17: whole MoE layer (moe_start + moe_finish) ----
 * in: [S, D] -- the gemma residual, or the lfm/maple normed hidden X.
 * out: [S, D]. eidx/ewt: [S*K]. uniq: [E] first-seen expert order, *nu its size.
 * Returns 0 on success, -1 on a bad config. */
int orc_moe_layer(const orc_cfg *c, const orc_weights *w, const float *in, int S,
                  float *out, int *eidx, float *ewt, int *uniq, int *nu, orc_dump *dump);

/* A15: dispatch lists exactly as moe_apply_chunk builds them (gemma4.c:779-786):
 * for each uniq[u], rows ascending with the slot's weight. offs[nu+1]. */
void orc_dispatch(const int *eidx, const float *ewt, int S, int K, const int *uniq, int nu,
                  int *offs, int *rows, float *wts, int *slots);

/* ---- gemma around the MoE block: the feed-forward half of layer_fwd
 *      (gemma4.c:1003-1030) and the tied q4_0 embedding / lm_head ---- */
typedef struct {
    int DI;                         /* dense_inter                                  */
    const uint8_t *mlp;             /* q4_0 mlp_gate [DI,D] | mlp_up [DI,D] | mlp_down [D,DI] */
    const float *pre_ffn_ln;        /* [D] */
    const float *post_ffn_ln1;      /* [D] */
    const float *post_ffn_ln;       /* [D] */
    float layer_scalar;
} orc_dense;

/* dense branch of S rows (gemma4.c:1012-1020): h1 = rmsnorm(mlp(rmsnorm(r, pre_ffn_ln)),
 * post_ffn_ln1), q8_0 activations (matvec, gemma4.c:445-460) */
void orc_dense_mlp(const orc_dense *dn, int D, float eps, const float *r, int S, float *h1);
/* H [S, D] in place: H = (H + rmsnorm(dense(H) + moe(H), post_ffn_ln)) * layer_scalar.
 * c must be gemma gating. Returns 0, or -1 on a bad config. */
int orc_gemma_ffn_block(const orc_cfg *c, const orc_weights *w, const orc_dense *dn, float *H, int S,
                        int *eidx, float *ewt);
/* embed_row (gemma4.c:1131-1145) of a q4_0 [V, D] table */
void orc_embed_row(const uint8_t *table, int D, float embed_scale, int tok, float *h);
/* lm_head of one row (gemma4.c:1264-1275): logits[V] = softcap(table . q8_0(rmsnorm(h,
 * fnorm))); returns the greedy token (gemma4.c:2149-2152) */
int orc_head(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
             const float *h, float *logits);

/* FlashHead (gemma4.c:1055-1131), the approximate lm_head of one row: centroid scores
 * fsim = q4_0 [NC, D] centroids . q8_0(rmsnorm(h, fnorm)) (times cluster_scale unless
 * the scale is folded into the centroids, `scaled`), the NP best clusters by the
 * reference's quickselect, their token_map rows [NC, CS] (-1 = padding) and the force
 * list as candidates; logits[V] = -inf except the candidates' softcapped q4_0 logits.
 * Returns the greedy token; sel (may be NULL) receives the NP chosen clusters, sorted. */
int orc_flash_head(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
                   const uint8_t *cent, int NC, const int32_t *tmap, int CS, int NP,
                   const float *cscale, int scaled, const int32_t *force, int nforce,
                   const float *h, float *logits, int *sel);

/* threads used by the parallel loops (OpenMP); 0 = runtime default */
void orc_set_threads(int n);

/* the host libm's expf (glibc) on n values */
void orc_expf(const float *x, float *y, long long n);

#ifdef __cplusplus
}
#endif
#endif
