/* zz_moe.h -- MoE-layer C ABI of libzzmoe.so (MI355X, gfx950).
 *
 * The whole MoE block of an engine layer runs on the GPU in one call, with every
 * expert resident in an HBM slot table. It slots under the engines' unchanged
 * entry points:
 *   gemma4.c:750 moe_start(M*, li, residual, out, S, Buf*) + 792 moe_finish(...)
 *   lfm25.c:837/891 and maple.c:738/791 moe_start/moe_finish(M*, li, X, out, S, Buf*)
 * A zz_moe_forward() call computes what that pair computes in the default int8
 * build: route_row for every row, the first-seen batch union, the per-expert
 * dispatch lists, expert_apply's gated FFN on q8_0-quantised activations, the
 * gate-weighted combine, and gemma's pre/post ffn_ln2 norms.
 *
 * Conventions (gpu.h:31-33): calls return 1 when done and 0 to decline, leaving
 * outputs untouched; the engine then runs its CPU path. Single caller; calls are
 * synchronous unless the _dev or begin/end forms are used. Device memory is owned
 * by the library until zz_moe_layer_destroy() or gpu_shutdown().
 * gpu_init() (zz_gpu.h) must have returned 1 first.
 */
#ifndef ZZ_MOE_H
#define ZZ_MOE_H

#include <stdint.h>
#include <stddef.h>
#include "zz_gpu.h"

/* gating: how route_row turns logits into (ids, weights) */
#define ZZ_GATE_SOFTMAX_PES  0  /* gemma4.c:581-613: rmsnorm*scale*D^-1/2, f32 logits,
                                   top-k, softmax over k, x per-expert scale        */
#define ZZ_GATE_SIGMOID_BIAS 1  /* lfm25.c:636-668: double logits, sigmoid, +bias for
                                   selection only, normalise, x routed_scaling      */
#define ZZ_GATE_SOFTMAX_TOPK 2  /* maple.c:582-601: double logits, top-k, softmax    */
#define ZZ_GATE_DENSE        3  /* gemma4.c:1012-1020: the dense MLP branch. No router:
                                   E = K = 1 and every row goes through expert 0 with
                                   weight 1 (its record holds mlp_gate|mlp_up|mlp_down);
                                   pre_ln = pre_ffn_ln, post_ln = post_ffn_ln1, applied
                                   as gemma's two ffn_ln2 norms are                    */
#define ZZ_GATE_GROUPED      4  /* ling.c:705-789: 8-accumulator double logits, sigmoid,
                                   +bias; groups of E/n_group ranked by their top-2 sum,
                                   the best topk_group kept, top-k inside them; weights
                                   the unbiased sigmoid, normalised, x routed_scaling   */

/* activation between gate/up and down */
#define ZZ_ACT_GEGLU_TANH   0   /* gemma4.c:432-434, 644 */
#define ZZ_ACT_SWIGLU       1   /* lfm25.c:456-458, 714  */
#define ZZ_ACT_SWIGLU_CLAMP 2   /* maple.c:607-611, 672-675: silu(min(g,c))*clip(u,+-c) */

typedef struct zz_moe_desc {
    int D, MI, E, K;          /* hidden, expert intermediate, experts, top-k        */
    int gating, act;          /* ZZ_GATE_*, ZZ_ACT_*                                  */
    int fmt_gate, fmt_up, fmt_down;   /* GPU_FMT_Q40 / Q80 / TQ2 per tensor          */
    int norm_topk;            /* lfm/maple norm_topk_prob                            */
    int use_bias;             /* lfm: expert_bias on the selection score.
                                 gemma: a per-expert logit offset added after the
                                 dot (harness extension for skewed routing; 0 is the
                                 reference, gemma4.c:600-601)                         */
    float eps;                /* gemma rmsnorm epsilon                                */
    float routed_scaling;     /* lfm                                                  */
    float clamp;              /* maple mlp_clamp                                      */
    int n_group, topk_group;  /* ZZ_GATE_GROUPED: expert groups, groups kept          */
} zz_moe_desc;

typedef struct zz_moe_weights {   /* host pointers, copied at layer creation        */
    const float *router;          /* [E, D]                                          */
    const float *router_scale;    /* [D] gemma router_scale                          */
    const float *pes;             /* [E] gemma router_pes                            */
    const float *bias;            /* [E] lfm expert_bias / gemma logit offset        */
    const float *pre_ln;          /* [D] gemma pre_ffn_ln2                           */
    const float *post_ln;         /* [D] gemma post_ffn_ln2                          */
} zz_moe_weights;

#ifdef __cplusplus
extern "C" {
#endif

/* Register one MoE layer. Returns a layer id >= 0, or -1 to decline (bad shape:
 * D, MI multiples of 64 and <= 8192, E <= 512, 1 <= K <= 16, K <= E). */
int zz_moe_layer_create(const zz_moe_desc *d, const zz_moe_weights *w);
void zz_moe_layer_destroy(int layer);

/* Bytes of one expert record in the reference layout [gate | up | down]
 * (gemma4.c:660 offsets 0, gate_b, 2*gate_b; per-tensor sizes q40.h:313-314,
 * 461-462, tq2.h:84-86). The record is what experts.bin holds per expert. */
int64_t zz_moe_record_bytes(const zz_moe_desc *d);

/* Fill slot `eid` of the layer's HBM slot table from one host record
 * (replaces slot_for/io_worker, gemma4.c:487-540: every expert stays resident). */
int zz_moe_expert_upload(int layer, int eid, const uint8_t *rec, size_t n);
/* Same from a device buffer (already in HBM). */
int zz_moe_expert_upload_dev(int layer, int eid, const void *d_rec, size_t n);

/* Fill every slot of `layer` from layer `li` of a zunzuncito container directory
 * (convert_*.py output). dir/manifest.txt gives the record size -- gemma/maple
 * `esz esz gate_b down_b` (gemma4.c:310-312), lfm `eszl li esz gate_b down_b fmt`
 * (lfm25.c:328-330) -- and each record's offset, `expert li e off`
 * (gemma4.c:326-329). The 4096-aligned [gate | up | down] records of
 * dir/experts.bin (convert_gemma4.py:361-390) are read once and uploaded; the
 * reference's slot/LRU tier and its I/O threads (gemma4.c:487-540) have no
 * counterpart, every expert stays resident. Declines on a record size that is not
 * the layer's zz_moe_record_bytes, a missing expert line or a short read. */
int zz_moe_load_experts(int layer, const char *dir, int li);

/* moe_start + moe_finish for S rows. in: gemma the residual [S, D], lfm/maple the
 * normed hidden X [S, D]. out [S, D]. eidx/ewt [S*K] (may be NULL) receive the
 * routing in route_row's order. Host pointers; synchronous. */
int zz_moe_forward(int layer, const float *in, float *out, int S, int *eidx, float *ewt);

/* Same on device pointers, enqueued on `stream` (a hipStream_t; NULL = the
 * library's stream) and not waited for. */
int zz_moe_forward_dev(int layer, const float *d_in, float *d_out, int S, int *d_eidx,
                       float *d_ewt, void *stream);

/* zz_moe_forward_dev without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The layer's
 * workspace is replaced by a fixed 64 MiB scratch array that the library's code
 * object brings with it, one per device, held until the process ends. A chunk of
 * min(S, the layer's chunk size) tokens must fit it: Gemma-4's layer (D 2816,
 * E 128, K 8) takes up to 580 tokens per call, LFM2.5's 1239, Maple's 751.
 * Larger S is declined with a message naming the limit, outputs untouched. No
 * per-kernel timing is recorded. Every call on a device shares the one array:
 * calls that overlap on one device (two streams, two threads) race. */
int zz_moe_forward_dev_noalloc(int layer, const float *d_in, float *d_out, int S, int *d_eidx,
                               float *d_ewt, void *stream);

/* Split form for overlap (gemma runs its dense MLP between moe_start and
 * moe_finish, gemma4.c:1012-1021): begin uploads `in` and enqueues the layer;
 * end waits and writes out/eidx/ewt. One begin may be outstanding. */
int zz_moe_forward_begin(int layer, const float *in, int S);
int zz_moe_forward_end(int layer, float *out, int *eidx, float *ewt);

/* Debug dump of the last forward's first chunk (any pointer may be NULL):
 * xq/xs [S, D] / [S, D/32]: the int8 expert input; hq/hs [S*K, MI] / [S*K, MI/32]:
 * the int8 hidden by (token, slot); dispatch: uniq[E] union order (nu is set),
 * and for union entry u the tokens rows[offs[u] .. offs[u+1]) ascending with
 * their top-k slots (offs[nu+1], rows[S*K], slots[S*K]); logits [S, E]: the
 * router logits, the reference's own float values for the lfm, maple and ling
 * routers at every S, and for gemma (after the bias) when S >= 16 and D % 64 == 0;
 * gemma's other batched logits are interval centres, and its decode path (S <= 2
 * with q4_0 / q8_0 experts, S <= 4 with tq2) keeps none. items: the FFN work
 * items of the batched path as 4 ints each (expert, union entry, first pair in
 * the dispatch lists, pairs; 0 pairs: an empty slot), slot i runs on XCD i % 8;
 * at most items_cap are copied and nitems is set to the slot count. */
typedef struct zz_moe_dump {
    int8_t *xq; float *xs;
    int8_t *hq; float *hs;
    int *uniq, *offs, *rows, *slots;
    int nu;
    double *logits;
    int *items;
    int items_cap, nitems;
} zz_moe_dump;
int zz_moe_debug(int layer, zz_moe_dump *dump);

/* Exact per-block int32 dots of rows [row0, row0+nrows) of one resident expert
 * tensor (0 gate, 1 up, 2 down) against int8 activations xq[I]:
 * q4_0 sum (q-8)*x, q8_0 sum q*x, tq2 sum (c-1)*x; out [nrows, I/32]. */
int zz_moe_blockdots(int layer, int eid, int tensor, int row0, int nrows,
                     const int8_t *xq, int32_t *out);

/* Device weight quantiser (the converters' q40_quant_row / q80_quant_row,
 * q40.h:83-110, 332-348, bit-exact for finite input): n f32 values at d_w (n % 32
 * == 0, rows laid end to end) -> n/32 blocks at d_out in the reference layout.
 * Device pointers, enqueued on `stream` (NULL = the library's stream). */
int zz_quantize(int fmt, const float *d_w, uint8_t *d_out, int64_t n, void *stream);

/* Counters since gpu_init: [0] rmsnorm serial replays, [1] lfm/maple/ling logit
 * serial replays, [2] gemma tokens that needed the exact router replay, [3] tokens
 * whose selection met an exact tie (equal scores at or above the k-th, or ling
 * groups tied at the kept/dropped boundary), decided by the lower index as the
 * reference's strict '>' insertion does (gemma4.c:604-607, lfm25.c:656-660). */
int zz_moe_stats(unsigned *counters4);

/* Diagnostic: the expf that the sigmoid routers evaluate on the device, which is
 * glibc's bit for bit (the reference's libm: lfm25.c:654, ling.c:731), on n floats
 * of device memory d_x -> d_y, enqueued on `stream` (NULL = the library's stream).
 * For checking the device's bits against the host's expf. */
int zz_router_expf(const float *d_x, float *d_y, int64_t n, void *stream);

/* Per-kernel timing with HIP events recorded on the stream each kernel is
 * launched on. zz_moe_profile(1) clears and starts recording, (0) stops.
 * zz_moe_profile_read fills, for kernel k in the order ZZ_K_*, the summed
 * duration in ms and the launch count; returns the number of kernels. */
#define ZZ_K_PREP 0
#define ZZ_K_LOGITS 1
#define ZZ_K_TOPK 2
#define ZZ_K_DISPATCH 3
#define ZZ_K_FFN_UP 4
#define ZZ_K_FFN_DOWN 5
#define ZZ_K_COMBINE 6
#define ZZ_K_DEC_ROUTE 7      /* decode batches: input quantisation + router logits */
#define ZZ_K_DEC_DOWN 8       /* decode batches: down projection + combine (+ post-norm) */
#define ZZ_K_COUNT 9
int zz_moe_profile(int on);
int zz_moe_profile_read(double *ms, int *launches, int n);

/* Diagnostic, for the integer tier: one forward of S host rows (synchronous, S within
 * one chunk, at most 64 Mi dots in all) on diagnostics builds of the FFN kernels that
 * store every per-block int32 dot before its fp32 scaling -- the integer dots of
 * q40.h:179-186 (q4_0), q40.h:374-414 (q8_0) and tq2.h:134-155 (tq2), as the kernels
 * that run the layer form them. By flat pair p = token*K + slot:
 *   up[p][0 = gate, 1 = up][MI][D/32], down[p][D][MI/32].
 * Values are the kernels' raw integers: q4_0 enters as 16*(q - 8), so its dots are 16
 * times the reference's; tq2 on the matrix cores is sum (c - 1)*x, on the decode path
 * (S <= 4) sum c*x with c in {0, 1, 2}. The timed kernels are separate builds without
 * these stores. */
int zz_moe_dots(int layer, const float *in, int S, int32_t *up, int32_t *down);

/* Diagnostic: how many times gpu_matmul (zz_gpu.h) found a mapped tensor rewritten
 * on the host since its last upload (its sampled fingerprint changed) and uploaded
 * it again before computing. The engines pread other experts into mapped slots
 * (gemma4.c:484-491); this counts those refreshes. */
long long zz_gpu_map_refreshes(void);

/* Text of the last failure (a declined call), or "". */
const char *zz_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* ZZ_MOE_H */
