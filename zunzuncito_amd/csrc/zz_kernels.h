// zz_kernels.h -- kernel argument blocks and launchers shared by the HIP sources
// and the C-ABI host layer. Plain structs passed by value to each kernel.
#pragma once
#include "zz_common.h"

struct ZzPrepArgs {
    int D, gemma;
    float eps;
    const float *in;            // [S, D]
    const float *router_scale;  // [D]   gemma
    const float *pre_ln;        // [D]   gemma
    float *xn;                  // [S, D] gemma router input
    int8_t *xq;                 // [S, D]
    float *xs;                  // [S, D/32]
    int *xsum;                  // [S, D/32]
    float *xt;                  // [S] tq2 Sx, or null
    unsigned *diag;             // diagnostics counters
    int *route_eidx;            // dense branch: [S] set to expert 0, or null
    float *route_ewt;           // dense branch: [S] set to weight 1
};

struct ZzLogitArgs {
    int D, E, gating, S;
    int exact_min_s;            // batches of at least this many tokens take the exact chains
    const float *router;        // [E, D]
    const float *xn;            // [S, D] gemma
    const float *x;             // [S, D] lfm / maple
    const float *bias;          // [E] gemma Zipf offset, or null
    double *cen, *bnd;          // [S, E]
    unsigned *diag;
};

struct ZzTopkArgs {
    int D, E, K, gating, norm_topk;
    int n_group, topk_group;    // grouped router
    float routed_scaling;
    const double *cen, *bnd;    // [S, E]
    const float *router, *xn;   // gemma refinement
    const float *bias;          // gemma Zipf offset / lfm expert_bias
    const float *pes;           // gemma
    int *eidx;                  // [S, K]
    float *ewt;                 // [S, K]
    float *topv;                // [S, K] selected scores (debug), or null
    unsigned *diag;
};

struct ZzItem {                 // one FFN work unit: <= tch pairs of one expert
    int e, u, p0, n;
};

struct ZzDispatchArgs {
    int P, E, K, tch;
    int xslots;                 // work-item slots per XCD the FFN grids hold
    int wcost;                  // an expert's weight stream, in token columns of FFN work
    const int *eidx;            // [P]
    const float *ewt;           // [P]
    int *ptok, *pslot;          // [P] sorted pair -> token, slot
    float *pwt;                 // [P] sorted pair -> weight
    int *ppos;                  // [P] flat (token*K + slot) -> sorted position
    int *uniq, *uoff, *ucnt;    // [E] union order
    ZzItem *items;              // [8 * xslots]: XCD x's j-th item at j*8 + x; n = 0: none
    int *meta;                  // [0] = nu, [1] = item slots used (a multiple of 8)
};

struct ZzFfnArgs {
    int D, MI, K, act;
    float clamp;
    const uint8_t *experts;     // slot table base of this layer
    int64_t estride;            // bytes per expert
    ZzLayout lay;
    const ZzItem *items;
    const int *meta;
    const int *ptok;            // sorted pair -> token
    const int8_t *xq;           // [S, D]
    const float *xs;            // [S, D/32]
    const int *xsum;            // [S, D/32]
    const float *xt;            // [S]
    int8_t *hq;                 // [P, MI] by sorted pair
    float *hs;                  // [P, MI/32]
    int *hsum;                  // [P, MI/32]
    float *y;                   // [P, D] expert outputs before weighting, row token*K + slot
    const int *pslot;           // sorted pair -> slot
    // diagnostics (zz_moe_dots), null otherwise: the kernels' per-block integer dots
    // before scaling, by flat pair p = token*K + slot
    int32_t *dbg_up;            // [P][gate, up][MI][D/32]
    int32_t *dbg_dn;            // [P][D][MI/32]
};

struct ZzCombineArgs {
    int D, K, gemma;
    float eps;
    const float *y;             // [S*K, D] by flat pair token*K + slot
    const float *ewt;           // [S, K]
    const float *post_ln;       // [D] gemma
    float *out;                 // [S, D]
};

#define ZZ_DEC_MAXS 4   // largest batch of the fused decode path
#define ZZ_DEC_LDS 49152  // LDS for the decode down kernel's quantised hidden rows

// Decode tail of a gemma FFN block with the dense branch fused in: both post-norms
// from their per-tile sums, then Hout = (H + rmsnorm(h1 + h2, post_ffn_ln)) * ls.
struct ZzDecFinalArgs {
    int D, G;                   // G = D/16 tiles
    float eps, ls;
    const float *out;           // [S, D] routed combine (before post_ffn_ln2)
    const double *ss;
    const float *post2;         // post_ffn_ln2
    const float *yd;            // [S, D] dense down (before post_ffn_ln1)
    const double *ssd;
    const float *post1;         // post_ffn_ln1
    const float *post;          // post_ffn_ln
    const float *H;             // [S, D] the block's residual input
    float *Hout;                // [S, D] the result (H itself, or another buffer)
};

// A block's combine deferred into the next block's router holds S*D <= this many
// floats in each router workgroup's LDS
#define ZZ_DEC_FIN_MAXF 12288

// Decode router (two kernels): logits per expert workgroup, then top-k gating and
// the small-batch dispatch in one workgroup.
struct ZzDecRouteArgs {
    ZzPrepArgs prep;            // quantisation of the expert input
    ZzLogitArgs lg;             // logits (cen/bnd) of all tokens
    ZzTopkArgs tk;              // top-k of all tokens
    ZzDispatchArgs dp;          // dispatch lists and work items
    int S;
    int dense;                  // dense branch: norms and quantisation only, no logits
    int dual;                   // also quantise the dense branch's input into prep2
    ZzPrepArgs prep2;           // dual: the dense layer's pre-norm and input buffers
    int fin;                    // first apply the previous block's combine `fa`: every
    ZzDecFinalArgs fa;          // workgroup forms the rows, workgroup 0 stores fa.Hout
};

// Decode gate/up: the routing of each token and the expert GEMVs of its pairs.
struct ZzDecUpArgs {
    ZzFfnArgs f;
    ZzTopkArgs tk;
    int dense;                  // dense branch: expert 0 for every pair, no top-k
    int pk;                     // routed pairs S*K: grid rows >= pk are dense-branch rows
    int nd;                     // dense-branch rows (0, or S with a dense layer fused in)
    ZzFfnArgs fd;               // the dense layer (nd > 0)
};

// Fused decode down projection + gate-weighted combine.
struct ZzDecDownArgs {
    ZzFfnArgs f;
    int S, K, E;
    const int *eidx;            // [S, K]
    const float *ewt;           // [S, K]
    float *out;                 // [S, D]
    double *ss;                 // [S, D/16] per-tile sums of squares of out (gemma), or null
    int nd;                     // dense-branch rows fused in (0 or S)
    ZzFfnArgs fd;               // the dense layer (nd > 0)
    float *yd;                  // [S, D] its down projection
    double *ssd;                // [S, D/16] per-tile sums of squares of yd
};

// FlashHead (zz_flash.hip): the tensors of tools/flashhead.py on the device, and one
// step's working buffers
#define ZZ_FLASH_MAXNC 16384    // clusters held by the select kernel's LDS
struct ZzFlashArgs {
    int V, D, NC, CS, NP, nforce, scaled;
    float cap;                  // final_logit_softcap (0: none)
    const uint8_t *rtab;        // [V, D] q4_0 table, reference layout
    const uint8_t *cent;        // [NC, D] q4_0 centroids, reference layout
    const int *tmap;            // [NC, CS] token ids, -1 = padding
    const float *cscale;        // [NC] (read when !scaled)
    const int *force;           // [nforce]
    const int8_t *xq;           // [S, D] q8_0 of rmsnorm(H, final_norm)
    const float *xs;            // [S, D/32]
    float *fsim;                // [S, NC] centroid scores
    int *sel;                   // [S, NP] chosen clusters
    float *logits;              // [S, V] or null
    unsigned long long *part;   // [S, probe groups] argmax keys
    unsigned *diag;             // [4]: quickselect replays
};
int zz_launch_flash(const ZzFlashArgs &a, int S, hipStream_t st);
int zz_flash_probe_groups(const ZzFlashArgs &a);
int zz_launch_flash_unpack(const uint8_t *src, const ZzTensor &T, uint8_t *dst, hipStream_t st);

// Host-side internals of the library (zz_api.hip), shared by its host files.
struct zz_moe_desc;
hipStream_t zz_lib_stream();
int zz_lib_ready();
unsigned *zz_lib_diag();
const zz_moe_desc *zz_layer_desc(int id);
int zz_lib_prof_set(int on);        // per-kernel event timing on/off; returns the old state
// Generation of the library's device buffers: bumped whenever a buffer that a
// captured HIP graph may hold (a layer, its workspace, a block's rows, a head or its
// FlashHead tensors) is freed or reallocated. A captured graph is valid only while
// the generation it was captured at is current.
unsigned long long zz_lib_mem_gen();
void zz_lib_mem_bump();
// a gemma FFN block's decode rows with the dense branch fused into the routed layer's
// launches: 1 done, 0 failed, -1 not applicable. pend_in: the previous block's
// combine, applied by this block's router (d_H must be pend_in->Hout); pend_out: this
// block's combine is not launched but returned, with Hout left to the caller.
int zz_block_decode(int moe_id, int dense_id, float *d_H, float *d_h1, float *d_h2, const float *post_ln,
                    float ls, int S, int *d_eidx, float *d_ewt, hipStream_t st,
                    const ZzDecFinalArgs *pend_in = nullptr, ZzDecFinalArgs *pend_out = nullptr);
int zz_block_decode_fits(int moe_id, int dense_id, int S);   // the checks zz_block_decode makes
// tensor in the slot-table layout at *cursor (advanced past it, 256-aligned)
ZzTensor zz_make_tensor(int fmt, int O, int I, int64_t *cursor);

struct ZzRepackArgs {
    const uint8_t *src;         // reference record [gate | up | down]
    int64_t src_gate, src_up, src_down;   // byte offsets in the record
    uint8_t *dst;               // repacked expert
    ZzLayout lay;
};

int zz_launch_prep(const ZzPrepArgs &a, int S, hipStream_t st);
int zz_launch_logits(const ZzLogitArgs &a, int S, hipStream_t st);
int zz_launch_topk(const ZzTopkArgs &a, int S, hipStream_t st);
int zz_launch_expf(const float *x, float *y, int64_t n, hipStream_t st);
int zz_launch_dispatch(const ZzDispatchArgs &a, hipStream_t st);
int zz_launch_dec_logits(const ZzDecRouteArgs &a, hipStream_t st);
int zz_launch_dec_up(const ZzDecUpArgs &a, int S, hipStream_t st);
int zz_launch_dec_down(const ZzDecDownArgs &a, hipStream_t st);
int zz_dec_fits(int S, int K, int MI);   // the decode path's LDS holds S*K hidden rows
int zz_dec_fits2(int S, int K, int MI, int MID);   // ... and S dense hidden rows of MID
int zz_launch_dec_final(const ZzDecFinalArgs &a, int S, hipStream_t st);
int zz_dec_fin_fits(int S, int D);   // a deferred combine fits the decode router
int zz_launch_dec_norm(float *out, const float *post_ln, const double *ss, int D, float eps, int S, hipStream_t st);
// int8-MFMA grouped GEMM for work items of up to ZZ_MMA_TOKENS tokens
#define ZZ_MMA_TOKENS 64
int zz_launch_up_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st);
int zz_launch_down_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st);
int zz_launch_combine(const ZzCombineArgs &a, int S, hipStream_t st);
int zz_launch_repack(const ZzRepackArgs &a, hipStream_t st);
// the first n tensors of a.lay only (gate, then up, then down)
int zz_launch_repack_n(const ZzRepackArgs &a, int n, hipStream_t st);
// y[S,O] = W[O,I] x[S,I] with f32 activations (gpu.h matmul contract)
int zz_launch_matmul_f32(int fmt, float *y, const uint8_t *W, const float *x, int O, int I,
                         int S, hipStream_t st);
// f32 -> q4_0 / q8_0 blocks in the reference layout (nblk blocks of 32 values)
int zz_launch_quantize(int fmt, const float *w, uint8_t *dst, int64_t nblk, hipStream_t st);
// per-block exact int32 dots of n rows of a repacked tensor against one int8 vector
int zz_launch_blockdots(const uint8_t *expert, ZzTensor t, int row0, int nrows,
                        const int8_t *xq, int32_t *out, hipStream_t st);
