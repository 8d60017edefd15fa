// zz_gemma.hip -- gemma4's forward() around the MoE block (include/zz_gemma.h):
//   - the feed-forward half of layer_fwd (gemma4.c:1003-1030): the MoE layer and the
//     dense MLP (a ZZ_GATE_DENSE layer) on two streams, then the layer combine;
//   - the tied q4_0 embedding / lm_head (gemma4.c:1131-1145, 1264-1275) with the
//     greedy token (gemma4.c:2149-2152).
// The lm_head table is held in the slot-table lane order (zz_common.h), so its GEMV
// streams one 16-byte load per lane and chunk like the expert kernels.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_dot_dev.h"
#include "zz_route_dev.h"
#include "../../include/zz_gemma.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

#define ZZ_FAIL(...)               \
    do {                           \
        zz_set_error(__VA_ARGS__); \
        return 0;                  \
    } while (0)

// ------------------------------------------------------------------ kernels
// H = (H + rmsnorm(h1 + h2, w)) * ls (gemma4.c:1022-1030): tmp = h1 + h2, its sum of
// squares in double (gemma4.c:425-428), tmp*r*w left to right, then (res + tmp)*ls.
// One workgroup per token.
__global__ __launch_bounds__(256) void zz_block_combine_kernel(float *H, const float *h1, const float *h2,
                                                               const float *w, float ls, float eps, int D) {
    const int s = blockIdx.x, tid = threadIdx.x;
    __shared__ __attribute__((aligned(16))) float row[ZZ_MAXD];
    __shared__ double red[4];
    float *hr = H + (size_t)s * D;
    const float *a = h1 + (size_t)s * D, *b = h2 + (size_t)s * D;
    double ss = 0.0;
    for (int o = 4 * tid; o < D; o += 1024) {
        const float4 x = *(const float4 *)(a + o), y = *(const float4 *)(b + o);
        const float4 t = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
        *(float4 *)&row[o] = t;
        ss += (double)t.x * t.x + (double)t.y * t.y + (double)t.z * t.z + (double)t.w * t.w;
    }
    ss = zz_block_sum(ss, red);
    const float r = 1.0f / sqrtf((float)(ss / D) + eps);
    for (int o = 4 * tid; o < D; o += 1024) {
        const float4 t = *(const float4 *)&row[o], wv = *(const float4 *)(w + o), h = *(const float4 *)(hr + o);
        *(float4 *)(hr + o) = make_float4((h.x + (t.x * r) * wv.x) * ls, (h.y + (t.y * r) * wv.y) * ls,
                                          (h.z + (t.z * r) * wv.z) * ls, (h.w + (t.w * r) * wv.w) * ls);
    }
}

// embed_row (gemma4.c:1131-1145): h = (d * (q - 8)) * embed_scale for row tok[s] of
// the lane-order table. Thread u owns block u/4, weights k = 8(u%4)..+7: one 4-byte
// word (byte m: nibbles k = 8qq+m and 8qq+m+4, stored as q ^ 8) and the block scale.
__global__ __launch_bounds__(256) void zz_embed_kernel(const uint8_t *tb, ZzTensor T, const int *tok, float scale,
                                                       float *H) {
    const int s = blockIdx.x, D = T.I, nb = D / ZZ_BLK;
    int t = tok[s];
    t = t < 0 || t >= T.O ? 0 : t;
    const int g = t >> 4, r = t & 15;
    for (int u = threadIdx.x; u < 4 * nb; u += 256) {
        const int b = u >> 2, qq = u & 3;
        const unsigned w = *(const unsigned *)(tb + zz_qlane(T, g, b, 16 * qq + r));
        const float d = zz_h2f(*(const uint16_t *)(tb + zz_sidx(T, g, b, r)));
        float v[8];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int n0 = (int)((w >> (8 * m)) & 15u) ^ 8, n1 = (int)((w >> (8 * m + 4)) & 15u) ^ 8;
            v[m] = (d * (float)(n0 - 8)) * scale;
            v[m + 4] = (d * (float)(n1 - 8)) * scale;
        }
        float *h = H + (size_t)s * D + b * ZZ_BLK + 8 * qq;
        *(float4 *)h = make_float4(v[0], v[1], v[2], v[3]);
        *(float4 *)(h + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__device__ __forceinline__ unsigned zz_ord_bits(float f) {       // order-preserving
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// lm_head GEMV: one wave per 16-row group of the table over the whole K range, lane
// l = 16qq + r as in the slot table. Weight chunks come in batches of HD_C, the next
// batch requested before the current one is used. The q8_0 rows of xn (S <= 4) are
// staged in LDS (S*D codes then S*D/32 scales, dynamic). Then the softcap, the
// logits, and the workgroup's best (logit, -index) key per row into part[s][wg]: the
// finish kernel picks the largest key, so the first index of the largest logit wins
// whatever the order the workgroups run in.
#define HD_C 8
__global__ __launch_bounds__(256) void zz_head_kernel(const uint8_t *tb, ZzTensor T, const int8_t *xq,
                                                      const float *xs, int S, float cap, float *logits,
                                                      unsigned long long *part) {
    extern __shared__ __attribute__((aligned(16))) char hd_lds[];
    __shared__ unsigned long long wkey[4][ZZ_DEC_MAXS];
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, r = l & 15, qq = l >> 4;
    const int D = T.I, nb = D / ZZ_BLK, nch = (nb + 3) / 4, V = T.O, g = 4 * blockIdx.x + w;
    int8_t *sq = (int8_t *)hd_lds;                          // [S][D]
    float *ss = (float *)(hd_lds + (size_t)S * D);          // [S][nb]
    const ZzWalk W = zz_walk(T, g, l, r);
    ZzChunk k[HD_C], kn[HD_C];
#pragma unroll
    for (int i = 0; i < HD_C; i++) k[i] = zz_load_chunk<ZZ_FMT_Q40>(tb, W, min(i, nch - 1));
    for (int i = tid; i < S * (D / 16); i += 256) *(uint4 *)(sq + 16 * i) = ld16(xq + 16 * (size_t)i);
    for (int i = tid; i < S * nb; i += 256) ss[i] = xs[i];
    __syncthreads();
    float acc[ZZ_DEC_MAXS] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < nch; c0 += HD_C) {
        if (c0 + HD_C < nch)
#pragma unroll
            for (int i = 0; i < HD_C; i++) kn[i] = zz_load_chunk<ZZ_FMT_Q40>(tb, W, min(c0 + HD_C + i, nch - 1));
#pragma unroll
        for (int i = 0; i < HD_C; i++) {
            const int c = c0 + i;
            if (c >= nch) break;
            const bool full = c < W.nfull;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (j >= 2 && !full) break;
                const int b = 4 * c + j;
                const uint2 wv = zz_chunk_w<ZZ_FMT_Q40>(k[i], j);
                const float dw = zz_chunk_dw(k[i], j, full);
#pragma unroll
                for (int s = 0; s < ZZ_DEC_MAXS; s++) {
                    if (s >= S) break;
                    const uint2 xv = *(const uint2 *)(sq + (size_t)s * D + b * ZZ_BLK + 8 * qq);
                    int d = zz_dot4(wv.x, xv.x, 0);
                    d = zz_dot4(wv.y, xv.y, d);
                    acc[s] = fmaf(dw * ss[s * nb + b], (float)d, acc[s]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < HD_C; i++) k[i] = kn[i];
    }
    const int o = 16 * g + r;
#pragma unroll
    for (int s = 0; s < ZZ_DEC_MAXS; s++) {
        if (s >= S) break;
        float v = acc[s];
        v = zz_rows_sum(v);
        v *= 0.0625f;                                    // the 16*(q - 8) weights
        if (cap > 0.0f) v = tanhf(v / cap) * cap;
        if (qq == 0) logits[(size_t)s * V + o] = v;
        unsigned long long key = ((unsigned long long)zz_ord_bits(v) << 32) | (0xffffffffu - (unsigned)o);
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) {
            const unsigned long long k2 = __shfl_xor(key, m, 64);
            key = k2 > key ? k2 : key;
        }
        if (l == 0) wkey[w][s] = key;
    }
    __syncthreads();
    if (tid < S) {
        unsigned long long key = wkey[0][tid];
        for (int q = 1; q < 4; q++) key = wkey[q][tid] > key ? wkey[q][tid] : key;
        part[(size_t)tid * gridDim.x + blockIdx.x] = key;
    }
}

// argmax[s] = the index of the largest of the n partial keys of row s
__global__ __launch_bounds__(256) void zz_head_argmax_kernel(const unsigned long long *part, int n, int *argmax) {
    __shared__ unsigned long long red[4];
    const int s = blockIdx.x, tid = threadIdx.x;
    unsigned long long key = 0ull;
    for (int i = tid; i < n; i += 256) {
        const unsigned long long k = part[(size_t)s * n + i];
        key = k > key ? k : key;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long k2 = __shfl_xor(key, m, 64);
        key = k2 > key ? k2 : key;
    }
    if ((tid & 63) == 0) red[tid >> 6] = key;
    __syncthreads();
    if (tid == 0) {
        for (int q = 1; q < 4; q++) key = red[q] > key ? red[q] : key;
        key = red[0] > key ? red[0] : key;
        argmax[s] = (int)(0xffffffffu - (unsigned)(key & 0xffffffffu));
    }
}

// ------------------------------------------------------------------ ffn blocks
struct FfnBlock {
    int moe, dense, D;
    float ls, eps;
    int fuse = 1;                                      // fused decode path (ZZ_BLOCK_FUSE=0: off)
    float *post_ln = nullptr;
    float *h1 = nullptr, *h2 = nullptr, *hh = nullptr;   // hh: host-form staging of H
    size_t cap = 0;                                    // tokens h1/h2/hh hold
    hipStream_t ds = nullptr;                          // the dense branch's stream
    hipEvent_t fork = nullptr, join = nullptr;
};
static std::vector<FfnBlock *> g_blocks;

static void free_block(FfnBlock *B) {
    if (!B) return;
    zz_lib_mem_bump();
    if (B->ds) (void)hipStreamSynchronize(B->ds);
    void *ps[] = {B->post_ln, B->h1, B->h2, B->hh};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    if (B->fork) (void)hipEventDestroy(B->fork);
    if (B->join) (void)hipEventDestroy(B->join);
    if (B->ds) (void)hipStreamDestroy(B->ds);
    delete B;
}

static FfnBlock *get_block(int id) {
    if (!zz_lib_ready() || id < 0 || id >= (int)g_blocks.size()) return nullptr;
    return g_blocks[id];
}

extern "C" int zz_ffn_block_create(int moe_layer, int dense_layer, const float *post_ffn_ln, float layer_scalar) {
    const zz_moe_desc *m = zz_layer_desc(moe_layer), *d = zz_layer_desc(dense_layer);
    if (!m || !d || !post_ffn_ln || m->gating != ZZ_GATE_SOFTMAX_PES || d->gating != ZZ_GATE_DENSE ||
        m->D != d->D) {
        zz_set_error("zz_ffn_block_create: needs a gemma MoE layer and a dense layer of one D, and post_ffn_ln");
        return -1;
    }
    FfnBlock *B = new FfnBlock();
    B->moe = moe_layer;
    B->dense = dense_layer;
    B->D = m->D;
    B->ls = layer_scalar;
    B->eps = m->eps;
    const char *fz = getenv("ZZ_BLOCK_FUSE");
    B->fuse = !(fz && fz[0] == '0');
    bool ok = hipMalloc(&B->post_ln, sizeof(float) * m->D) == hipSuccess &&
              hipMemcpy(B->post_ln, post_ffn_ln, sizeof(float) * m->D, hipMemcpyHostToDevice) == hipSuccess &&
              hipStreamCreateWithFlags(&B->ds, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&B->fork, hipEventDisableTiming) == hipSuccess &&
              hipEventCreateWithFlags(&B->join, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        zz_set_error("zz_ffn_block_create: device allocation failed");
        free_block(B);
        return -1;
    }
    for (size_t i = 0; i < g_blocks.size(); i++)
        if (!g_blocks[i]) { g_blocks[i] = B; return (int)i; }
    g_blocks.push_back(B);
    return (int)g_blocks.size() - 1;
}

extern "C" void zz_ffn_block_destroy(int id) {
    FfnBlock *B = get_block(id);
    if (!B) return;
    (void)hipStreamSynchronize(zz_lib_stream());
    free_block(B);
    g_blocks[id] = nullptr;
}

static int block_grow(FfnBlock *B, int S, hipStream_t st) {
    if ((size_t)S <= B->cap) return 1;
    ZZ_CHECK(hipStreamSynchronize(st));
    ZZ_CHECK(hipStreamSynchronize(B->ds));
    float **bufs[] = {&B->h1, &B->h2, &B->hh};
    for (float **p : bufs) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    B->cap = 0;
    zz_lib_mem_bump();
    const size_t n = sizeof(float) * (size_t)S * B->D;
    ZZ_CHECK(hipMalloc(&B->h1, n));
    ZZ_CHECK(hipMalloc(&B->h2, n));
    ZZ_CHECK(hipMalloc(&B->hh, n));
    B->cap = (size_t)S;
    return 1;
}

static int block_forward(FfnBlock *B, float *d_H, int S, int *d_eidx, float *d_ewt, hipStream_t st) {
    if (S <= 0 || !d_H) ZZ_FAIL("zz_ffn_block_forward: bad arguments");
    if (!block_grow(B, S, st)) return 0;
    // decode rows: the dense branch rides in the routed layer's launches
    if (B->fuse) {
        const int r = zz_block_decode(B->moe, B->dense, d_H, B->h1, B->h2, B->post_ln, B->ls, S, d_eidx, d_ewt, st);
        if (r >= 0) return r;
    }
    // the dense branch forks off the caller's stream and joins before the combine
    ZZ_CHECK(hipEventRecord(B->fork, st));
    ZZ_CHECK(hipStreamWaitEvent(B->ds, B->fork, 0));
    if (!zz_moe_forward_dev(B->moe, d_H, B->h2, S, d_eidx, d_ewt, st)) return 0;
    if (!zz_moe_forward_dev(B->dense, d_H, B->h1, S, nullptr, nullptr, B->ds)) return 0;
    ZZ_CHECK(hipEventRecord(B->join, B->ds));
    ZZ_CHECK(hipStreamWaitEvent(st, B->join, 0));
    hipLaunchKernelGGL(zz_block_combine_kernel, dim3(S), dim3(256), 0, st, d_H, B->h1, B->h2, B->post_ln, B->ls,
                       B->eps, B->D);
    if (hipGetLastError() != hipSuccess) ZZ_FAIL("zz_ffn_block_forward: combine launch failed");
    return 1;
}

extern "C" int zz_ffn_block_forward_dev(int id, float *d_H, int S, int *d_eidx, float *d_ewt, void *stream) {
    FfnBlock *B = get_block(id);
    if (!B) ZZ_FAIL("zz_ffn_block_forward_dev: no such block");
    return block_forward(B, d_H, S, d_eidx, d_ewt, stream ? (hipStream_t)stream : zz_lib_stream());
}

extern "C" int zz_ffn_block_forward(int id, float *H, int S, int *eidx, float *ewt) {
    FfnBlock *B = get_block(id);
    if (!B || !H || S <= 0) ZZ_FAIL("zz_ffn_block_forward: bad arguments");
    const zz_moe_desc *m = zz_layer_desc(B->moe);
    if (!m) ZZ_FAIL("zz_ffn_block_forward: the MoE layer is gone");
    hipStream_t st = zz_lib_stream();
    if (!block_grow(B, S, st)) return 0;
    int *d_ix = nullptr;
    float *d_wt = nullptr;
    const size_t P = (size_t)S * m->K;
    if ((eidx && hipMalloc(&d_ix, sizeof(int) * P) != hipSuccess) ||
        (ewt && hipMalloc(&d_wt, sizeof(float) * P) != hipSuccess)) {
        if (d_ix) (void)hipFree(d_ix);
        ZZ_FAIL("zz_ffn_block_forward: allocation failed");
    }
    std::vector<float> h((size_t)S * B->D);
    int ok = hipMemcpyAsync(B->hh, H, sizeof(float) * h.size(), hipMemcpyHostToDevice, st) == hipSuccess &&
             block_forward(B, B->hh, S, d_ix, d_wt, st) &&
             hipMemcpyAsync(h.data(), B->hh, sizeof(float) * h.size(), hipMemcpyDeviceToHost, st) == hipSuccess &&
             hipStreamSynchronize(st) == hipSuccess &&
             (!eidx || hipMemcpy(eidx, d_ix, sizeof(int) * P, hipMemcpyDeviceToHost) == hipSuccess) &&
             (!ewt || hipMemcpy(ewt, d_wt, sizeof(float) * P, hipMemcpyDeviceToHost) == hipSuccess);
    if (d_ix) (void)hipFree(d_ix);
    if (d_wt) (void)hipFree(d_wt);
    if (!ok) ZZ_FAIL("zz_ffn_block_forward: failed (%s)", hipGetErrorString(hipGetLastError()));
    memcpy(H, h.data(), sizeof(float) * h.size());
    return 1;
}

// ------------------------------------------------------------------ heads
struct Head {
    int V, D;
    float eps, escale, cap;
    ZzTensor T;
    uint8_t *table = nullptr;       // lane-order q4_0 [V, D]
    float *fnorm = nullptr;
    int8_t *xq = nullptr;           // [4, D] q8_0 of rmsnorm(H, final_norm)
    float *xs = nullptr;            // [4, D/32]
    int *xsum = nullptr;            // [4, D/32]
    unsigned long long *part = nullptr;   // [4][V/64] per-workgroup argmax keys
    // FlashHead (zz_flash.hip), once attached; use_flash routes the logits through it
    bool use_flash = false;
    ZzFlashArgs fl{};               // its device tensors and buffers (fl.rtab: the
                                    // table in reference layout, [V, D])
};
static std::vector<Head *> g_heads;

static void free_flash(ZzFlashArgs &f, bool keep_table) {
    zz_lib_mem_bump();
    void *ps[] = {(void *)f.cent, (void *)f.tmap, (void *)f.cscale, (void *)f.force,
                  f.fsim, f.sel, f.part};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    uint8_t *rtab = (uint8_t *)f.rtab;
    if (rtab && !keep_table) (void)hipFree(rtab);
    f = ZzFlashArgs{};
    if (keep_table) f.rtab = rtab;
}

static void free_head(Head *h) {
    if (!h) return;
    zz_lib_mem_bump();
    void *ps[] = {h->table, h->fnorm, h->xq, h->xs, h->xsum, h->part};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    free_flash(h->fl, false);
    delete h;
}

static Head *get_head(int id) {
    if (!zz_lib_ready() || id < 0 || id >= (int)g_heads.size()) return nullptr;
    return g_heads[id];
}

extern "C" int zz_head_create(const uint8_t *table, int V, int D, const float *final_norm, float eps,
                              float embed_scale, float softcap) {
    if (!zz_lib_ready() || !table || !final_norm || V <= 0 || V % 64 || D <= 0 || D % 64 || D > ZZ_MAXD) {
        zz_set_error("zz_head_create: bad arguments (V %% 64 == 0, D %% 64 == 0, D <= %d)", ZZ_MAXD);
        return -1;
    }
    Head *h = new Head();
    h->V = V;
    h->D = D;
    h->eps = eps;
    h->escale = embed_scale;
    h->cap = softcap;
    int64_t cur = 0;
    h->T = zz_make_tensor(ZZ_FMT_Q40, V, D, &cur);
    const size_t src_bytes = (size_t)V * (D / ZZ_BLK) * 18, nb = D / ZZ_BLK;
    hipStream_t st = zz_lib_stream();
    uint8_t *staging = nullptr;
    bool ok = hipMalloc(&h->table, (size_t)cur) == hipSuccess && hipMalloc(&staging, src_bytes) == hipSuccess &&
              hipMalloc(&h->fnorm, sizeof(float) * D) == hipSuccess &&
              hipMalloc(&h->xq, (size_t)ZZ_DEC_MAXS * D) == hipSuccess &&
              hipMalloc(&h->xs, sizeof(float) * ZZ_DEC_MAXS * nb) == hipSuccess &&
              hipMalloc(&h->xsum, sizeof(int) * ZZ_DEC_MAXS * nb) == hipSuccess &&
              hipMalloc(&h->part, sizeof(unsigned long long) * ZZ_DEC_MAXS * (V / 64)) == hipSuccess &&
              hipMemcpy(h->fnorm, final_norm, sizeof(float) * D, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(staging, table, src_bytes, hipMemcpyHostToDevice) == hipSuccess;
    if (ok) {
        ZzRepackArgs a;
        memset(&a, 0, sizeof a);
        a.src = staging;
        a.dst = h->table;
        a.lay.gate = h->T;
        a.lay.bytes = cur;
        ok = zz_launch_repack_n(a, 1, st) && hipStreamSynchronize(st) == hipSuccess;
    }
    if (staging) (void)hipFree(staging);
    if (!ok) {
        zz_set_error("zz_head_create: device allocation or upload failed");
        free_head(h);
        return -1;
    }
    for (size_t i = 0; i < g_heads.size(); i++)
        if (!g_heads[i]) { g_heads[i] = h; return (int)i; }
    g_heads.push_back(h);
    return (int)g_heads.size() - 1;
}

extern "C" void zz_head_destroy(int id) {
    Head *h = get_head(id);
    if (!h) return;
    (void)hipStreamSynchronize(zz_lib_stream());
    free_head(h);
    g_heads[id] = nullptr;
}

extern "C" int zz_head_embed_dev(int id, const int *d_tok, int S, float *d_H, void *stream) {
    Head *h = get_head(id);
    if (!h || !d_tok || !d_H || S <= 0) ZZ_FAIL("zz_head_embed_dev: bad arguments");
    hipStream_t st = stream ? (hipStream_t)stream : zz_lib_stream();
    hipLaunchKernelGGL(zz_embed_kernel, dim3(S), dim3(256), 0, st, h->table, h->T, d_tok, h->escale, d_H);
    if (hipGetLastError() != hipSuccess) ZZ_FAIL("zz_head_embed_dev: launch failed");
    return 1;
}

extern "C" int zz_head_embed(int id, const int *tok, int S, float *H) {
    Head *h = get_head(id);
    if (!h || !tok || !H || S <= 0) ZZ_FAIL("zz_head_embed: bad arguments");
    hipStream_t st = zz_lib_stream();
    int *d_tok = nullptr;
    float *d_H = nullptr;
    int ok = hipMalloc(&d_tok, sizeof(int) * S) == hipSuccess &&
             hipMalloc(&d_H, sizeof(float) * (size_t)S * h->D) == hipSuccess &&
             hipMemcpy(d_tok, tok, sizeof(int) * S, hipMemcpyHostToDevice) == hipSuccess &&
             zz_head_embed_dev(id, d_tok, S, d_H, st) && hipStreamSynchronize(st) == hipSuccess &&
             hipMemcpy(H, d_H, sizeof(float) * (size_t)S * h->D, hipMemcpyDeviceToHost) == hipSuccess;
    if (d_tok) (void)hipFree(d_tok);
    if (d_H) (void)hipFree(d_H);
    if (!ok) ZZ_FAIL("zz_head_embed: failed");
    return 1;
}

extern "C" int zz_head_logits_dev(int id, const float *d_H, int S, float *d_logits, int *d_argmax, void *stream) {
    Head *h = get_head(id);
    if (!h || !d_H || !d_logits || S <= 0 || S > ZZ_DEC_MAXS) ZZ_FAIL("zz_head_logits_dev: bad arguments (S <= %d)", ZZ_DEC_MAXS);
    hipStream_t st = stream ? (hipStream_t)stream : zz_lib_stream();
    // rmsnorm(H, final_norm) and its q8_0 rows, as matvec quantises xn (gemma4.c:445-460)
    ZzPrepArgs pa;
    memset(&pa, 0, sizeof pa);
    pa.D = h->D;
    pa.gemma = 1;
    pa.eps = h->eps;
    pa.in = d_H;
    pa.pre_ln = h->fnorm;
    pa.xq = h->xq;
    pa.xs = h->xs;
    pa.xsum = h->xsum;
    pa.diag = zz_lib_diag();
    if (!zz_launch_prep(pa, S, st)) ZZ_FAIL("zz_head_logits_dev: norm launch failed");
    if (h->use_flash) {                          // gemma4.c:1241-1242
        ZzFlashArgs fa = h->fl;
        fa.xq = h->xq;
        fa.xs = h->xs;
        fa.logits = d_logits;
        fa.diag = zz_lib_diag();
        if (!zz_launch_flash(fa, S, st)) ZZ_FAIL("zz_head_logits_dev: FlashHead launch failed");
        if (d_argmax)
            hipLaunchKernelGGL(zz_head_argmax_kernel, dim3(S), dim3(256), 0, st, fa.part, zz_flash_probe_groups(fa),
                               d_argmax);
        if (hipGetLastError() != hipSuccess) ZZ_FAIL("zz_head_logits_dev: launch failed");
        return 1;
    }
    const size_t lds = (size_t)S * h->D + sizeof(float) * (size_t)S * (h->D / ZZ_BLK);
    hipLaunchKernelGGL(zz_head_kernel, dim3(h->V / 64), dim3(256), lds, st, h->table, h->T, h->xq, h->xs, S, h->cap,
                       d_logits, h->part);
    if (d_argmax)
        hipLaunchKernelGGL(zz_head_argmax_kernel, dim3(S), dim3(256), 0, st, h->part, h->V / 64, d_argmax);
    if (hipGetLastError() != hipSuccess) ZZ_FAIL("zz_head_logits_dev: launch failed");
    return 1;
}

extern "C" int zz_head_logits(int id, const float *H, int S, float *logits, int *argmax) {
    Head *h = get_head(id);
    if (!h || !H || !logits || S <= 0 || S > ZZ_DEC_MAXS) ZZ_FAIL("zz_head_logits: bad arguments");
    hipStream_t st = zz_lib_stream();
    float *d_H = nullptr, *d_l = nullptr;
    int *d_a = nullptr;
    int ok = hipMalloc(&d_H, sizeof(float) * (size_t)S * h->D) == hipSuccess &&
             hipMalloc(&d_l, sizeof(float) * (size_t)S * h->V) == hipSuccess &&
             hipMalloc(&d_a, sizeof(int) * S) == hipSuccess &&
             hipMemcpy(d_H, H, sizeof(float) * (size_t)S * h->D, hipMemcpyHostToDevice) == hipSuccess &&
             zz_head_logits_dev(id, d_H, S, d_l, d_a, st) && hipStreamSynchronize(st) == hipSuccess &&
             hipMemcpy(logits, d_l, sizeof(float) * (size_t)S * h->V, hipMemcpyDeviceToHost) == hipSuccess &&
             (!argmax || hipMemcpy(argmax, d_a, sizeof(int) * S, hipMemcpyDeviceToHost) == hipSuccess);
    if (d_H) (void)hipFree(d_H);
    if (d_l) (void)hipFree(d_l);
    if (d_a) (void)hipFree(d_a);
    if (!ok) ZZ_FAIL("zz_head_logits: failed");
    return 1;
}

// ------------------------------------------------------------------ stacks
extern "C" int zz_head_flash(int id, const uint8_t *centroids, int n_clusters, const int32_t *token_map,
                             int cluster_size, int n_probes, const float *cluster_scale, int scaled,
                             const int32_t *force, int n_force) {
    Head *h = get_head(id);
    if (!h || !centroids || !token_map || n_clusters < 1 || n_clusters > ZZ_FLASH_MAXNC || cluster_size < 1 ||
        n_probes < 1 || n_probes > n_clusters || n_force < 0 || (n_force > 0 && !force) || (!scaled && !cluster_scale))
        ZZ_FAIL("zz_head_flash: bad arguments (1 <= n_probes <= n_clusters <= %d)", ZZ_FLASH_MAXNC);
    hipStream_t st = zz_lib_stream();
    ZZ_CHECK(hipStreamSynchronize(st));
    free_flash(h->fl, true);                     // a new attachment replaces the old one
    h->use_flash = false;
    ZzFlashArgs &f = h->fl;
    const int nb = h->D / ZZ_BLK;
    const size_t rb = (size_t)18 * nb;
    f.V = h->V; f.D = h->D; f.NC = n_clusters; f.CS = cluster_size; f.NP = n_probes; f.nforce = n_force;
    f.scaled = scaled ? 1 : 0; f.cap = h->cap;
    const int groups = zz_flash_probe_groups(f);
    uint8_t *rtab = (uint8_t *)f.rtab, *cent = nullptr;
    int *tmap = nullptr, *fo = nullptr;
    float *cs = nullptr;
    bool ok = true;
    if (!rtab) {                                 // the table in reference layout, once
        ok = hipMalloc(&rtab, rb * h->V) == hipSuccess && zz_launch_flash_unpack(h->table, h->T, rtab, st);
        f.rtab = rtab;
    }
    ok = ok && hipMalloc(&cent, rb * n_clusters) == hipSuccess &&
         hipMalloc(&tmap, sizeof(int) * (size_t)n_clusters * cluster_size) == hipSuccess &&
         hipMalloc(&cs, sizeof(float) * n_clusters) == hipSuccess &&
         hipMalloc(&fo, sizeof(int) * (size_t)(n_force > 0 ? n_force : 1)) == hipSuccess;
    f.cent = cent; f.tmap = tmap; f.cscale = cs; f.force = fo;
    ok = ok && hipMalloc(&f.fsim, sizeof(float) * ZZ_DEC_MAXS * n_clusters) == hipSuccess &&
         hipMalloc(&f.sel, sizeof(int) * ZZ_DEC_MAXS * n_probes) == hipSuccess &&
         hipMalloc(&f.part, sizeof(unsigned long long) * ZZ_DEC_MAXS * groups) == hipSuccess &&
         hipMemcpy(cent, centroids, rb * n_clusters, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(tmap, token_map, sizeof(int) * (size_t)n_clusters * cluster_size, hipMemcpyHostToDevice) ==
             hipSuccess &&
         (scaled || hipMemcpy(cs, cluster_scale, sizeof(float) * n_clusters, hipMemcpyHostToDevice) == hipSuccess) &&
         (n_force == 0 || hipMemcpy(fo, force, sizeof(int) * n_force, hipMemcpyHostToDevice) == hipSuccess) &&
         hipStreamSynchronize(st) == hipSuccess;
    if (!ok) {
        free_flash(h->fl, false);
        ZZ_FAIL("zz_head_flash: device allocation or upload failed");
    }
    return 1;
}

static void drop_graphs_of_head(int head);

extern "C" int zz_head_use_flash(int id, int on) {
    Head *h = get_head(id);
    if (!h || (on && !h->fl.cent)) ZZ_FAIL("zz_head_use_flash: no such head, or no FlashHead attached");
    if (h->use_flash != (on != 0)) {
        (void)hipStreamSynchronize(zz_lib_stream());
        drop_graphs_of_head(id);                 // captured steps hold the other path
    }
    h->use_flash = on != 0;
    return 1;
}

extern "C" int zz_head_flash_replays(unsigned *n) {
    unsigned *d = zz_lib_diag();
    if (!n || !d) ZZ_FAIL("zz_head_flash_replays: not ready");
    ZZ_CHECK(hipMemcpy(n, d + 4, sizeof(unsigned), hipMemcpyDeviceToHost));
    return 1;
}

struct Stack {
    std::vector<int> blocks;
    int head, D, V;
    float *h = nullptr;             // [D] the decode row
    float *alt = nullptr;           // [ZZ_DEC_MAXS, D] the residual stream's second buffer
    float *logits = nullptr;        // [V]
    int *cur = nullptr;             // the current token
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;  // one decode step, captured on first use
    unsigned long long gen = 0;     // zz_lib_mem_gen() the graph was captured at
    unsigned long long warm = 0;    // zz_lib_mem_gen() after the last eager step
    // what a container load created for this stack, destroyed with it
    std::vector<int> own_layers, own_blocks;
    int own_head = -1;
};
static std::vector<Stack *> g_stacks;

// owned: also destroy what the stack owns (not at shutdown, which frees everything)
static void free_stack(Stack *k, bool owned = false) {
    if (!k) return;
    if (owned) {
        for (int b : k->own_blocks) zz_ffn_block_destroy(b);
        for (int l : k->own_layers) zz_moe_layer_destroy(l);
        if (k->own_head >= 0) zz_head_destroy(k->own_head);
    }
    if (k->exec) (void)hipGraphExecDestroy(k->exec);
    if (k->graph) (void)hipGraphDestroy(k->graph);
    void *ps[] = {k->h, k->alt, k->logits, k->cur};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    delete k;
}

static Stack *get_stack(int id) {
    if (!zz_lib_ready() || id < 0 || id >= (int)g_stacks.size()) return nullptr;
    return g_stacks[id];
}

static void drop_graph(Stack *k) {
    if (k->exec) (void)hipGraphExecDestroy(k->exec);
    if (k->graph) (void)hipGraphDestroy(k->graph);
    k->exec = nullptr;
    k->graph = nullptr;
}

static void drop_graphs_of_head(int head) {
    for (Stack *k : g_stacks)
        if (k && k->head == head) drop_graph(k);
    zz_lib_mem_bump();
}

extern "C" int zz_stack_use_flash(int id, int on) {
    Stack *k = get_stack(id);
    if (!k) ZZ_FAIL("zz_stack_use_flash: no such stack");
    return zz_head_use_flash(k->head, on);
}

extern "C" int zz_stack_create(const int *blocks, int n, int head) {
    Head *h = get_head(head);
    if (!blocks || n <= 0 || !h) {
        zz_set_error("zz_stack_create: bad arguments");
        return -1;
    }
    for (int i = 0; i < n; i++) {
        FfnBlock *B = get_block(blocks[i]);
        if (!B || B->D != h->D) {
            zz_set_error("zz_stack_create: block %d is missing or not of the head's D", blocks[i]);
            return -1;
        }
    }
    Stack *k = new Stack();
    k->blocks.assign(blocks, blocks + n);
    k->head = head;
    k->D = h->D;
    k->V = h->V;
    if (hipMalloc(&k->h, sizeof(float) * h->D) != hipSuccess ||
        hipMalloc(&k->alt, sizeof(float) * ZZ_DEC_MAXS * h->D) != hipSuccess ||
        hipMalloc(&k->logits, sizeof(float) * h->V) != hipSuccess || hipMalloc(&k->cur, sizeof(int)) != hipSuccess) {
        zz_set_error("zz_stack_create: device allocation failed");
        free_stack(k);
        return -1;
    }
    for (size_t i = 0; i < g_stacks.size(); i++)
        if (!g_stacks[i]) { g_stacks[i] = k; return (int)i; }
    g_stacks.push_back(k);
    return (int)g_stacks.size() - 1;
}

extern "C" void zz_stack_destroy(int id) {
    Stack *k = get_stack(id);
    if (!k) return;
    (void)hipDeviceSynchronize();
    g_stacks[id] = nullptr;
    free_stack(k, true);
}

int zz_stack_adopt(int id, const std::vector<int> &layers, const std::vector<int> &blocks, int head) {
    Stack *k = get_stack(id);
    if (!k) return 0;
    k->own_layers = layers;
    k->own_blocks = blocks;
    k->own_head = head;
    return 1;
}

// Decode rows through the blocks. Where every block takes the fused decode path and
// the rows fit the router's LDS, each block's combine is deferred into the next
// block's router kernel, which forms the combined rows in every workgroup and stores
// them once: one launch less per block. The router cannot update the rows in place
// (its other workgroups still read them), so the residual stream alternates between
// d_H and k->alt; the last block's combine runs as its own kernel into d_H.
static int stack_blocks(Stack *k, float *d_H, int S, hipStream_t st) {
    bool chain = S <= ZZ_DEC_MAXS && zz_dec_fin_fits(S, k->D);
    for (int b : k->blocks) {
        FfnBlock *B = get_block(b);
        if (!B) ZZ_FAIL("zz_stack: block %d is gone", b);
        chain = chain && B->fuse && zz_block_decode_fits(B->moe, B->dense, S);
    }
    if (!chain) {
        for (int b : k->blocks)
            if (!block_forward(get_block(b), d_H, S, nullptr, nullptr, st)) return 0;
        return 1;
    }
    ZzDecFinalArgs pend;
    bool have = false;
    for (int b : k->blocks) {
        FfnBlock *B = get_block(b);
        if (!block_grow(B, S, st)) return 0;
        float *rows = d_H;
        if (have) {
            pend.Hout = pend.H == d_H ? k->alt : d_H;
            rows = pend.Hout;
        }
        ZzDecFinalArgs next;
        const int r = zz_block_decode(B->moe, B->dense, rows, B->h1, B->h2, B->post_ln, B->ls, S, nullptr,
                                      nullptr, st, have ? &pend : nullptr, &next);
        if (r < 0) ZZ_FAIL("zz_stack: block %d left the decode path", b);
        if (r == 0) return 0;
        pend = next;
        have = true;
    }
    pend.Hout = d_H;
    if (!zz_launch_dec_final(pend, S, st)) ZZ_FAIL("zz_stack: final combine launch failed");
    return 1;
}

extern "C" int zz_stack_prefill_dev(int id, float *d_H, int S, int *d_tok, void *stream) {
    Stack *k = get_stack(id);
    if (!k || !d_H || S <= 0) ZZ_FAIL("zz_stack_prefill_dev: bad arguments");
    hipStream_t st = stream ? (hipStream_t)stream : zz_lib_stream();
    if (!stack_blocks(k, d_H, S, st)) return 0;
    if (d_tok && !zz_head_logits_dev(k->head, d_H + (size_t)(S - 1) * k->D, 1, k->logits, d_tok, st)) return 0;
    return 1;
}

// one decode step: cur -> embed -> blocks -> head -> cur
static int stack_step(Stack *k, hipStream_t st) {
    return zz_head_embed_dev(k->head, k->cur, 1, k->h, st) && stack_blocks(k, k->h, 1, st) &&
           zz_head_logits_dev(k->head, k->h, 1, k->logits, k->cur, st);
}

extern "C" int zz_stack_decode_dev(int id, int *d_tok, int n, float *d_logits, int use_graph, void *stream) {
    Stack *k = get_stack(id);
    if (!k || !d_tok || n < 0) ZZ_FAIL("zz_stack_decode_dev: bad arguments");
    hipStream_t st = stream ? (hipStream_t)stream : zz_lib_stream();
    ZZ_CHECK(hipMemcpyAsync(k->cur, d_tok, sizeof(int), hipMemcpyDeviceToDevice, st));
    for (int i = 0; i < n; i++) {
        // a graph holds raw device pointers: once any buffer it may reference was
        // freed or reallocated (a longer prefill grows the workspaces, a FlashHead is
        // attached or switched), it is dropped and captured again
        if (k->exec && k->gen != zz_lib_mem_gen()) drop_graph(k);
        if (use_graph && !k->exec && k->warm == zz_lib_mem_gen()) {
            // an eager step ran on the current buffers, so every workspace already
            // holds one row: the captured step allocates nothing and waits on nothing
            const unsigned long long gen = zz_lib_mem_gen();
            const int prof = zz_lib_prof_set(0);           // no timing events in the graph
            const hipError_t b = hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed);
            const int ok = b == hipSuccess && stack_step(k, st);
            hipGraph_t g = nullptr;
            const hipError_t e = b == hipSuccess ? hipStreamEndCapture(st, &g) : b;
            zz_lib_prof_set(prof);
            if (!ok || e != hipSuccess || zz_lib_mem_gen() != gen) {
                if (g) (void)hipGraphDestroy(g);
                ZZ_FAIL("zz_stack_decode_dev: capture failed (%s%s)", hipGetErrorString(e),
                        zz_lib_mem_gen() != gen ? ", buffers reallocated during capture" : "");
            }
            k->graph = g;
            if (hipGraphInstantiate(&k->exec, g, nullptr, nullptr, 0) != hipSuccess) {
                drop_graph(k);
                ZZ_FAIL("zz_stack_decode_dev: graph instantiation failed");
            }
            k->gen = gen;
        }
        if (use_graph && k->exec) {
            ZZ_CHECK(hipGraphLaunch(k->exec, st));
        } else {
            if (!stack_step(k, st)) return 0;
            k->warm = zz_lib_mem_gen();
        }
        ZZ_CHECK(hipMemcpyAsync(d_tok + i + 1, k->cur, sizeof(int), hipMemcpyDeviceToDevice, st));
    }
    if (d_logits && n > 0)
        ZZ_CHECK(hipMemcpyAsync(d_logits, k->logits, sizeof(float) * k->V, hipMemcpyDeviceToDevice, st));
    return 1;
}

// released by gpu_shutdown (zz_api.hip)
void zz_gemma_shutdown() {
    for (Stack *&k : g_stacks) { free_stack(k); k = nullptr; }
    g_stacks.clear();
    for (FfnBlock *&B : g_blocks) { free_block(B); B = nullptr; }
    g_blocks.clear();
    for (Head *&h : g_heads) { free_head(h); h = nullptr; }
    g_heads.clear();
}
