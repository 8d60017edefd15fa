/* zz_gemma.h -- the parts of gemma4.c's forward() around the MoE block, on the GPU
 * (libzzmoe.so, MI355X gfx950): the feed-forward half of layer_fwd and the tied
 * q4_0 embedding / lm_head with greedy selection. With attention as the identity,
 * these and zz_moe.h make up the whole per-token path of gemma4.c:1184-1275.
 *
 * Conventions as zz_moe.h: 1 when done, 0 (or -1 for an id) to decline with the
 * outputs untouched; single caller; _dev forms take device pointers and a
 * hipStream_t (NULL = the library's stream) and are not waited for.
 */
#ifndef ZZ_GEMMA_H
#define ZZ_GEMMA_H

#include <stdint.h>
#include <stddef.h>
#include "zz_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The feed-forward half of one gemma layer (gemma4.c:1003-1030):
 *   res = H;  h2 = MoE(res)                        moe_start/moe_finish, 1010 + 1021
 *   h1 = rmsnorm(dense_mlp(rmsnorm(res, pre_ffn_ln)), post_ffn_ln1)      1012-1020
 *   H  = (res + rmsnorm(h1 + h2, post_ffn_ln)) * layer_scalar           1022-1030
 * moe_layer is a ZZ_GATE_SOFTMAX_PES layer, dense_layer a ZZ_GATE_DENSE layer of
 * the same D (its record: mlp_gate | mlp_up | mlp_down). The dense branch runs on
 * a second stream while the MoE runs, as the reference overlaps them (1003-1009).
 * Returns a block id >= 0, or -1. The layers stay owned by their creator and must
 * outlive the block. */
int zz_ffn_block_create(int moe_layer, int dense_layer, const float *post_ffn_ln,
                        float layer_scalar);
void zz_ffn_block_destroy(int block);

/* H [S, D] in place. eidx/ewt [S*K] (may be NULL) receive the MoE routing. */
int zz_ffn_block_forward_dev(int block, float *d_H, int S, int *d_eidx, float *d_ewt,
                             void *stream);
int zz_ffn_block_forward(int block, float *H, int S, int *eidx, float *ewt);

/* The tied q4_0 embedding table [V, D] (reference layout, q40.h:9-18), which is
 * also the lm_head (gemma4.c:353-354): embed_row scales by embed_scale
 * (gemma4.c:1131-1145); logits are rmsnorm(H, final_norm) quantised q8_0 times the
 * table, softcapped as tanh(v / cap) * cap when softcap > 0 (gemma4.c:1264-1275).
 * V % 64 == 0. Returns a head id >= 0, or -1. */
int zz_head_create(const uint8_t *table, int V, int D, const float *final_norm, float eps,
                   float embed_scale, float softcap);
void zz_head_destroy(int head);

/* H[s] = embed_row(tok[s]) for S tokens (ids outside [0, V) read row 0). */
int zz_head_embed_dev(int head, const int *d_tok, int S, float *d_H, void *stream);
int zz_head_embed(int head, const int *tok, int S, float *H);

/* logits [S, V] of S <= 4 rows of H, and (if argmax is not NULL) the greedy token of
 * each row: the first index of the largest logit (sample at temp <= 0,
 * gemma4.c:2149-2152). */
int zz_head_logits_dev(int head, const float *d_H, int S, float *d_logits, int *d_argmax,
                       void *stream);
int zz_head_logits(int head, const float *H, int S, float *logits, int *argmax);

/* FlashHead, the approximate lm_head of gemma4.c (flash_logits, 1055-1110, with
 * flash_partition, 1112-1131), for a head: the tensors tools/flashhead.py writes into
 * a container (gemma4.c:357-362) -- q4_0 centroids [n_clusters, D] (reference layout),
 * token_map [n_clusters, cluster_size] (-1 = padding), cluster_scale [n_clusters]
 * (read only when !scaled, i.e. when the scale is not folded into the centroids) and
 * force [n_force] (ids always scored). n_clusters <= 16384, 1 <= n_probes <=
 * n_clusters. Attaching keeps a reference-layout copy of the table on the device
 * (V * D * 18/32 bytes) for the probed rows; a second call replaces the tensors.
 * Returns 1, or 0. */
int zz_head_flash(int head, const uint8_t *centroids, int n_clusters, const int32_t *token_map,
                  int cluster_size, int n_probes, const float *cluster_scale, int scaled,
                  const int32_t *force, int n_force);

/* on != 0: zz_head_logits[_dev] and the stacks on this head take the FlashHead path
 * (gemma4.c:1241-1242, `use_flash`): logits of the n_probes best clusters' members and
 * the forced ids, -inf elsewhere, and the greedy token among them. The probed set is
 * the reference's exactly (centroid scores in q40_dot's order; a tie at the boundary
 * replays the reference's quickselect). on = 0 returns to the full head. */
int zz_head_use_flash(int head, int on);

/* *n = the number of rows whose probed set was decided by a quickselect replay (a tie
 * at the boundary score) since zz_init. */
int zz_head_flash_replays(unsigned *n);

/* A stack of FFN blocks under one head: gemma4.c forward() (1184-1275) with the
 * attention of every layer taken as the identity. Returns a stack id >= 0, or -1.
 * The blocks and the head must outlive the stack. */
int zz_stack_create(const int *blocks, int n_blocks, int head);
void zz_stack_destroy(int stack);

/* Prefill: S rows of H [S, D] through every block in order, in place; when d_tok is
 * not NULL, d_tok[0] receives the greedy token of the last row (forward() with
 * last_only, then sample at temp 0). */
int zz_stack_prefill_dev(int stack, float *d_H, int S, int *d_tok, void *stream);

/* Greedy decode: for i = 0 .. n-1, d_tok[i+1] = the greedy token of
 * head(blocks(embed_row(d_tok[i]))). Token ids never leave the device. d_logits
 * (may be NULL) receives the last step's logits [V]. use_graph != 0 replays one
 * captured HIP graph per step (captured once per stack, on the first such call)
 * instead of launching each kernel. */
int zz_stack_decode_dev(int stack, int *d_tok, int n, float *d_logits, int use_graph,
                        void *stream);

/* zz_head_use_flash on the stack's head. */
int zz_stack_use_flash(int stack, int on);

/* A gemma4 container directory (convert_gemma4.py: manifest.txt, dense.bin,
 * experts.bin) made resident as a stack (gemma4.c:260-403 reads the same files):
 * per layer the MoE layer (router_proj, router_scale, router_pes,
 * pre/post_feedforward_layernorm_2 and the layer's experts), the dense branch
 * (mlp_gate, mlp_up, mlp_down, pre_feedforward_layernorm,
 * post_feedforward_layernorm_1) and the block (post_feedforward_layernorm,
 * layer_scalar); the head from embed_tokens, norm, cfg embed_scale and
 * final_logit_softcap, with the container's FlashHead attached when it has one
 * (cfg flash_*, gemma4.c:302-306, 357-362; off until zz_stack_use_flash). Attention
 * weights are not read. Returns a stack id >= 0 that
 * owns all of these (zz_stack_destroy frees them), or -1; *n_layers, *D, *V (each
 * may be NULL) receive the model's shape. */
int zz_gemma_stack_load(const char *dir, int *n_layers, int *D, int *V);

#ifdef __cplusplus
}
#endif

#endif /* ZZ_GEMMA_H */
