// zz_decode.hip -- decode-sized batches (S <= 4 tokens), four launches:
//   1. zz_dec_logits_kernel: one workgroup per expert computes that expert's
//      certified router logit for every token (gemma: with the input rmsnorm from
//      the same loads) and quantises a share of the expert input; in a stack it
//      first forms the previous block's combined rows (the deferred combine);
//   2. zz_dec_up_kernel: per (token, slot) pair and 32-row block of the hidden,
//      wave 0 selects the token's experts (certified top-k); one workgroup per
//      token then forms and writes the gate weights; gate/up GEMV of the chosen
//      expert, the activation and the int8 re-quantisation of the hidden
//      (a dense branch's rows ride in the same grid);
//   3. zz_dec_down_kernel: down GEMV for all (token, slot) pairs of a row tile
//      and the gate-weighted combine in slot order (gemma4.c:652), with per-tile
//      sums of squares for the post-norm;
//   4. zz_dec_norm_kernel (gemma's post-norm, gemma4.c:807-808) or, for a fused
//      block, zz_dec_final_kernel (both post-norms and the block combine).
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_route_dev.h"
#include "zz_topk_wave.h"
#include "zz_dot_dev.h"

#define DEC_MAXS ZZ_DEC_MAXS

// expert id kept inside the slot table whatever the router produced
__device__ __forceinline__ int zz_clamp_e(int e, int E) { return e < 0 || e >= E ? 0 : e; }

// The layer combine of token s (gemma4.c:807-808, 1020, 1022-1030): the two
// post-norms from their per-tile sums, their sum t, then
// Hout[s] = (H[s] + rmsnorm(t)·post)·ls. All 256 threads take part; row (LDS, D
// floats) ends holding Hout[s], which `store` also writes to a.Hout. Each thread
// reads H before it writes Hout, so H == Hout is allowed. The first 1024·NJ
// elements' six operands are all loaded before the norms are formed; the rest of a
// longer row streams.
template <int NJ>
__device__ void zz_dec_final_row(const ZzDecFinalArgs &a, int s, float *row, double *red, bool store) {
    const int tid = threadIdx.x, D = a.D, G = a.G;
    const float *o2 = a.out + (size_t)s * D, *o1 = a.yd + (size_t)s * D, *hr = a.H + (size_t)s * D;
    float4 y[NJ], w2[NJ], x[NJ], w1[NJ], h[NJ], wv[NJ], t[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int o = min(4 * tid + 1024 * j, D - 4);        // clamped: loads stay in range
        y[j] = *(const float4 *)(o2 + o);
        w2[j] = *(const float4 *)(a.post2 + o);
        x[j] = *(const float4 *)(o1 + o);
        w1[j] = *(const float4 *)(a.post1 + o);
        h[j] = *(const float4 *)(hr + o);
        wv[j] = *(const float4 *)(a.post + o);
    }
    // every wave forms both norm factors itself: the same sums in the same order, whose
    // totals every lane holds
    const double *ss2 = a.ss + (size_t)s * G, *ss1 = a.ssd + (size_t)s * G;
    double q2 = 0.0, q1 = 0.0;
    for (int k = tid & 63; k < G; k += 64) {
        q2 += ss2[k];
        q1 += ss1[k];
    }
    q2 = zz_group_sum<64>(q2);
    q1 = zz_group_sum<64>(q1);
    const float r2 = 1.0f / sqrtf((float)(q2 / D) + a.eps), r1 = 1.0f / sqrtf((float)(q1 / D) + a.eps);
    auto tsum = [&](float4 yv, float4 v2, float4 xv, float4 v1) {
        const float4 h2 = make_float4((yv.x * r2) * v2.x, (yv.y * r2) * v2.y, (yv.z * r2) * v2.z, (yv.w * r2) * v2.w);
        const float4 h1 = make_float4((xv.x * r1) * v1.x, (xv.y * r1) * v1.y, (xv.z * r1) * v1.z, (xv.w * r1) * v1.w);
        return make_float4(h1.x + h2.x, h1.y + h2.y, h1.z + h2.z, h1.w + h2.w);
    };
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        t[j] = tsum(y[j], w2[j], x[j], w1[j]);
        if (4 * tid + 1024 * j < D)
            sq += (double)t[j].x * t[j].x + (double)t[j].y * t[j].y + (double)t[j].z * t[j].z + (double)t[j].w * t[j].w;
    }
    for (int o = 4 * tid + 1024 * NJ; o < D; o += 1024) {
        const float4 tv = tsum(*(const float4 *)(o2 + o), *(const float4 *)(a.post2 + o),
                               *(const float4 *)(o1 + o), *(const float4 *)(a.post1 + o));
        *(float4 *)&row[o] = tv;
        sq += (double)tv.x * tv.x + (double)tv.y * tv.y + (double)tv.z * tv.z + (double)tv.w * tv.w;
    }
    sq = zz_block_sum(sq, red);
    const float r = 1.0f / sqrtf((float)(sq / D) + a.eps);
    float *ho = a.Hout + (size_t)s * D;
    auto fin = [&](float4 tv, float4 w, float4 hv) {
        return make_float4((hv.x + (tv.x * r) * w.x) * a.ls, (hv.y + (tv.y * r) * w.y) * a.ls,
                           (hv.z + (tv.z * r) * w.z) * a.ls, (hv.w + (tv.w * r) * w.w) * a.ls);
    };
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int o = 4 * tid + 1024 * j;
        if (o < D) {
            const float4 v = fin(t[j], wv[j], h[j]);
            *(float4 *)&row[o] = v;
            if (store) *(float4 *)(ho + o) = v;
        }
    }
    for (int o = 4 * tid + 1024 * NJ; o < D; o += 1024) {
        const float4 v = fin(*(const float4 *)&row[o], *(const float4 *)(a.post + o), *(const float4 *)(hr + o));
        *(float4 *)&row[o] = v;
        if (store) *(float4 *)(ho + o) = v;
    }
    __syncthreads();
}

// Decode router, part 1: one workgroup per expert e (the dense branch, which has
// no router: 16 workgroups that only norm and quantise). Gemma: per token, one set of
// loads (x row, router row e, router scale) gives both the rmsnorm factor and the
// rounded products of the router logit. The mean square is certified to round to
// the float of the reference's serial double sum (gemma4.c:425-428), else that sum
// is replayed; the logit gets the tight bound of zz_tight_block_scan. lfm/maple:
// wave s computes token s's logit. Then the workgroup quantises its share of the
// expert input (blocks e, e + E, ...).
// RB >= ceil(D/256): loads per thread and token, all issued before any is used.
// FIN: the input rows are first formed from the previous block's combine (a.fa)
// in LDS, and read from there.
template <int RB, bool FIN>
__global__ __launch_bounds__(256) void zz_dec_logits_kernel(ZzDecRouteArgs a) {
    const ZzPrepArgs &pp = a.prep;
    const ZzLogitArgs &lg = a.lg;
    const int S = a.S, D = pp.D, nb = D / ZZ_BLK, tid = threadIdx.x, e = blockIdx.x;
    const bool gem = pp.gemma;
    // gemma: the D rounded products (padded); lfm/maple/ling: one product buffer per
    // token's wave
    __shared__ __attribute__((aligned(16))) char sbuf[(ZZ_MAXD + ZZ_MAXD / 32) * 4 > DEC_MAXS * ZZ_DBUF * 8
                                                          ? (ZZ_MAXD + ZZ_MAXD / 32) * 4
                                                          : DEC_MAXS * ZZ_DBUF * 8];
    float *buf = (float *)sbuf;
    __shared__ double red[12];
    __shared__ float rr[DEC_MAXS];
    __shared__ float cert;
    __shared__ __attribute__((aligned(16))) float hrow[FIN ? ZZ_DEC_FIN_MAXF : 4];
    const float *xin = FIN ? hrow : pp.in;
    auto combine = [&] {
        for (int s = 0; s < S; s++) zz_dec_final_row<(RB + 3) / 4>(a.fa, s, hrow + (size_t)s * D, red, e == 0);
    };
    const float rs = 1.0f / sqrtf((float)D);
    if (a.dense && e == 0 && tid < S) {                      // one expert, weight 1
        pp.route_eidx[tid] = 0;
        pp.route_ewt[tid] = 1.0f;
    }
    if (gem) {
        const int R = (D + 255) >> 8;                         // <= RB
        float wr[RB], sr[RB];
#pragma unroll
        for (int j = 0; j < RB; j++) {                        // clamped: loads stay in range
            const int i = min(tid + 256 * j, D - 1);
            wr[j] = a.dense ? 0.0f : lg.router[(size_t)e * D + i];
            sr[j] = a.dense ? 0.0f : pp.router_scale[i];
        }
        const bool hb = !a.dense && lg.bias;                  // the Zipf offset, read with them
        const float bz = hb ? lg.bias[e] : 0.0f;
#pragma unroll
        for (int j = 0; j < RB; j++) sr[j] = sr[j] * rs;
        if (FIN) combine();                                   // the router rows are in flight
        for (int s = 0; s < S; s++) {
            const float *x = xin + (size_t)s * D;
            float xr[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) xr[j] = x[min(tid + 256 * j, D - 1)];
            double sq = 0.0;
#pragma unroll
            for (int j = 0; j < RB; j++)
                if (j < R && tid + 256 * j < D) sq += (double)xr[j] * (double)xr[j];
            // every square is exact in double; each term meets at most R - 1 + 6 + 3
            // roundings here and D - 1 in the reference's serial sum
            sq = zz_block_sum(sq, red);
            const double m = (double)(R + 10);
            const double g = zz_gamma(D, ZZ_U64) + zz_gamma(m, ZZ_U64);
            const double b = g * sq / (1.0 - zz_gamma(m, ZZ_U64)) * 1.0000001 + 1e-300;
            const float lo = (float)((sq - b) / (double)D), hi = (float)((sq + b) / (double)D);
            if (tid == 0) {
                if (lo == hi) {
                    cert = lo;
                } else {
                    double t = 0.0;                           // serial replay, reference order
                    for (int i = 0; i < D; i++) t += (double)x[i] * (double)x[i];
                    cert = (float)(t / (double)D);
                    if (e == 0) atomicAdd(pp.diag + 0, 1u);
                }
            }
            __syncthreads();
            const float r = 1.0f / sqrtf(cert + pp.eps);
            if (tid == 0) rr[s] = r;
            if (a.dense) continue;                            // no router
#pragma unroll
            for (int j = 0; j < RB; j++) {
                const int i = tid + 256 * j;
                if (j < R && i < D) {
                    const float xv = (xr[j] * r) * sr[j];     // xn as zz_prep_kernel forms it
                    if (e == 0) pp.xn[(size_t)s * D + i] = xv;   // for the exact replay
                    buf[zz_pad32(i)] = wr[j] * xv;
                }
            }
            __syncthreads();
            zz_tight_block_scan<RB>(buf, D, hb, bz, red, lg.cen + (size_t)s * lg.E + e,
                                lg.bnd + (size_t)s * lg.E + e);
        }
    } else {
        if (FIN) combine();
        if ((tid >> 6) < S) zz_logit_wave_f64(lg, tid >> 6, e, (double *)sbuf + (tid >> 6) * ZZ_DBUF);
    }
    // the expert input quantisation: block g on workgroup g % E, lanes 8(g / E)..+7;
    // dual: blocks S*nb.. are the dense branch's input (same rms factor, its own norm)
    __syncthreads();
    const int NQ = S * nb * (a.dual ? 2 : 1);
    for (int g0 = e + gridDim.x * (tid >> 3); g0 - (tid >> 3) * (int)gridDim.x < NQ; g0 += gridDim.x * 32) {
        const int g = min(g0, NQ - 1), m = tid & 7;               // whole waves iterate
        const bool two = g >= S * nb;
        const ZzPrepArgs &P = two ? a.prep2 : pp;
        const int gg = two ? g - S * nb : g, s = gg / nb, b = gg % nb;
        float4 v = *(const float4 *)(xin + (size_t)s * D + b * ZZ_BLK + 4 * m);
        if (gem) {
            const float r = rr[s];
            const float4 w = *(const float4 *)(P.pre_ln + b * ZZ_BLK + 4 * m);
            v = make_float4((v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w);
        }
        float d;
        int qs;
        const unsigned pk = zz_quant8(v, &d, &qs);
        if (g0 < NQ) {
            *(unsigned *)(P.xq + (size_t)s * D + b * ZZ_BLK + 4 * m) = pk;
            if (m == 0) {
                P.xs[(size_t)s * nb + b] = d;
                P.xsum[(size_t)s * nb + b] = qs;
            }
        }
    }
    if (a.dual && e == 0 && tid < S) {                          // the dense rows' routing
        a.prep2.route_eidx[tid] = 0;
        a.prep2.route_ewt[tid] = 1.0f;
    }
}

// ------------------------------------------------------------------ gate/up
// S*K*MI/32 workgroups (+ the fused dense branch's), 512 threads. Workgroup (p, j)
// owns hidden rows 32j..32j+31 of (token, slot) pair p = s*K + slot. Wave 0 first runs the certified top-k of token
// s (zz_topk_wave.h): every workgroup of the token repeats it, so no separate gating
// launch or dispatch list stands between the router and the expert weights; the
// token's first workgroup writes the routing outputs. Then wave w takes row group
// 2j + (w & 1) of gate (w & 3 < 2) or up of the pair's expert over half w/4 of the
// K range.
// Lane l = 16*qq + r is the slot table's lane: row r of the group, weights
// 8qq..8qq+7 of every block, so one chunk of 4 blocks is one contiguous 16-byte
// (q4_0) or 32-byte (q8_0) load; tq2 lanes take whole 64-groups of row r. The
// token's activations are requested first, the weights as soon as the expert is
// known. The output is h = act(g, u) quantised to q8_0 (hq, hs, hsum by flat pair).
#define DU_C 12          // chunks (tq2: groups) per lane issued together
#define DEC_SEG (ZZ_MAXD / 16 / 256)          // activation segments per thread

struct ZzDecStage {
    __attribute__((aligned(16))) int8_t xq[ZZ_MAXD];
    float xs[ZZ_MAXD / ZZ_BLK];
    int xsum[ZZ_MAXD / ZZ_BLK];
    float xt;                   // tq2 Sx of the token
};

// The token's activations into LDS in two steps: the issue requests every segment
// before the weight loads, so that waiting for them in the commit leaves the
// weights in flight (loads complete in order); the commit writes LDS (unconditional
// clamped slots, copies of one value: the loads cannot sink past the weights).
struct ZzDecStageRegs {
    uint4 xv[DEC_SEG];
    float sv;
    int cv;
};

__device__ __forceinline__ void zz_dec_stage_issue(const ZzFfnArgs &a, int tk, ZzDecStageRegs &r) {
    const int D = a.D, nb = D / ZZ_BLK, nseg = D / 16, tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < DEC_SEG; k++) r.xv[k] = ld16(a.xq + (size_t)tk * D + 16 * min(tid + 256 * k, nseg - 1));
    r.sv = a.xs[(size_t)tk * nb + min(tid, nb - 1)];
    r.cv = a.xsum[(size_t)tk * nb + min(tid, nb - 1)];
}

__device__ __forceinline__ void zz_dec_stage_commit(const ZzFfnArgs &a, const ZzDecStageRegs &r, ZzDecStage &st) {
    const int nb = a.D / ZZ_BLK, nseg = a.D / 16, tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < DEC_SEG; k++) *(uint4 *)&st.xq[16 * min(tid + 256 * k, nseg - 1)] = r.xv[k];
    st.xs[min(tid, nb - 1)] = r.sv;
    st.xsum[min(tid, nb - 1)] = r.cv;
    __syncthreads();
}

// The dots of one batch of a wave's chunks (h + 2i). The activation operands of a
// chunk (4 blocks' 8 bytes and d_x) are read from LDS one chunk ahead, so LDS
// latency overlaps the dots; no branch inside a chunk.
// dbg(b, d, whole): diagnostics hook with an int32 dot of block b before its scaling,
// a quarter block of the lane (whole = false) or the whole block (tq2); the timed
// build passes a hook that does nothing.
template <int FMT, typename DF>
__device__ __forceinline__ float zz_dec_up_comp(const ZzChunk (&k)[DU_C], const ZzDecStage &st, int nb, int h,
                                                int i0, int qq, float acc, DF dbg) {
    const int nch = (nb + 3) / 4, nfull = nb / 4;
    auto ldx = [&](int c, uint2 (&xv)[4], float4 &xs) {
        c = min(c, nch - 1);               // a short chunk's extra slots stay inside the row
#pragma unroll
        for (int j = 0; j < 4; j++) xv[j] = *(const uint2 *)&st.xq[(4 * c + j) * ZZ_BLK + 8 * qq];
        xs = *(const float4 *)&st.xs[4 * c];
    };
    auto chunk = [&](const ZzChunk &kk, const uint2 (&xv)[4], const float4 &xs, int c) {
        if (c >= nch) return;
        const bool full = c < nfull;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j >= 2 && !full) break;
            const uint2 w = zz_chunk_w<FMT>(kk, j);
            int d = zz_dot4(w.x, xv[j].x, 0);
            d = zz_dot4(w.y, xv[j].y, d);
            dbg(4 * c + j, d, false);
            const float sx = j == 0 ? xs.x : j == 1 ? xs.y : j == 2 ? xs.z : xs.w;
            acc = fmaf(zz_chunk_dw(kk, j, full) * sx, (float)d, acc);
        }
    };
    uint2 xa[4], xb[4];
    float4 sa, sb;
    ldx(h + 2 * i0, xa, sa);
#pragma unroll
    for (int i = 0; i < DU_C; i++) {
        const int c = h + 2 * (i0 + i);
        if (i % 2 == 0) {
            if (i + 1 < DU_C) ldx(c + 2, xb, sb);
            chunk(k[i], xa, sa, c);
        } else {
            if (i + 1 < DU_C) ldx(c + 2, xa, sa);
            chunk(k[i], xb, sb, c);
        }
    }
    return acc;
}

// the wave's partial dot of row r of group g over its half h of the K range; hook()
// runs once the wave's first weight loads are in flight
template <int FMT, typename HOOK, typename DF>
__device__ __forceinline__ float zz_dec_up_part(const ZzFfnArgs &a, const ZzDecStageRegs &sr, ZzDecStage &st,
                                                const uint8_t *E, const ZzTensor &T, int g, int h, int l,
                                                HOOK hook, DF dbg) {
    const int nb = a.D / ZZ_BLK, r = l & 15, qq = l >> 4;
    float acc = 0.0f;
    // the first batch of loads, the staging commit (waits only for the activations,
    // requested first), then batches past the first (K > 2 * DU_C chunks) in a loop
    // without a barrier
    if (FMT == ZZ_FMT_TQ2) {
        const int ng = nb / 2;                                  // lane's groups qq + 4h + 8i
        uint4 c[DU_C];
        auto load = [&](int i0) {
#pragma unroll
            for (int i = 0; i < DU_C; i++)                     // clamped: loads stay in range
                c[i] = ld16(E + zz_tq2off(T, 16 * g + r, min(qq + 4 * h + 8 * (i0 + i), ng - 1)));
        };
        auto comp = [&](int i0) {
#pragma unroll
            for (int i = 0; i < DU_C; i++) {
                const int gp = qq + 4 * h + 8 * (i0 + i);
                if (gp >= ng) continue;
                const int8_t *x = &st.xq[gp * 64];
                const int d0 = zz_dot_tq2(c[i], 0, ld16(x), ld16(x + 16));
                const int d1 = zz_dot_tq2(c[i], 1, ld16(x + 32), ld16(x + 48));
                dbg(2 * gp, d0, true);
                dbg(2 * gp + 1, d1, true);
                acc = fmaf(st.xs[2 * gp], (float)d0, acc);
                acc = fmaf(st.xs[2 * gp + 1], (float)d1, acc);
            }
        };
        load(0);
        hook();
        zz_dec_stage_commit(a, sr, st);
        comp(0);
        for (int i0 = DU_C; 4 * h + 8 * i0 < ng; i0 += DU_C) {
            load(i0);
            comp(i0);
        }
        return acc;
    }
    const int nch = (nb + 3) / 4;                               // lane's chunks h + 2i
    const ZzWalk W = zz_walk(T, g, l, r);
    ZzChunk k[DU_C];
    auto load = [&](int i0) {
#pragma unroll
        for (int i = 0; i < DU_C; i++) k[i] = zz_load_chunk<FMT>(E, W, min(h + 2 * (i0 + i), nch - 1));
    };
    load(0);
    hook();
    zz_dec_stage_commit(a, sr, st);
    acc = zz_dec_up_comp<FMT>(k, st, nb, h, 0, qq, acc, dbg);
    for (int i0 = DU_C; h + 2 * i0 < nch; i0 += DU_C) {
        load(i0);
        acc = zz_dec_up_comp<FMT>(k, st, nb, h, i0, qq, acc, dbg);
    }
    return FMT == ZZ_FMT_Q40 ? acc * 0.0625f : acc;            // the 16*(q - 8) weights
}

template <bool DBG>
__global__ __launch_bounds__(512) void zz_dec_up_kernel(ZzDecUpArgs a) {
    // workgroup (p, j) of the routed pairs is number p*(MI/32) + j; the fused dense
    // branch's rows (one per token, expert 0, no routing) follow, numbered the same way
    const int nr = a.pk * (a.f.MI / ZZ_BLK);
    const bool dn = (int)blockIdx.x >= nr;
    const ZzFfnArgs &f = dn ? a.fd : a.f;
    const int nbx = f.MI / ZZ_BLK, rel = dn ? (int)blockIdx.x - nr : (int)blockIdx.x;
    const int p = rel / nbx, j = rel - p * nbx;
    const int K = dn ? 1 : a.tk.K, s = p / K, js = p - s * K;
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, h = w >> 2, q = w & 3;
    extern __shared__ __attribute__((aligned(16))) char tk_lds[];
    __shared__ ZzDecStage st;
    __shared__ float part[2][4][16];                // [half][gate g0, g1, up g0, g1][row]
    __shared__ float hb[ZZ_BLK];
    ZzDecStageRegs sr;
    zz_dec_stage_issue(f, s, sr);
    const bool routed = !a.dense && !dn;
    // wave 0 selects the token's experts; the gate weights, needed only by the down
    // kernel, are formed by one workgroup per token (the writer) once its weight loads
    // are in flight, so no workgroup waits for them before its own loads
    const bool writer = j == 0 && js == 0;
    if (w == 0 && routed) zz_topk_wave_any(a.tk, s, tk_lds, writer, false);
    __syncthreads();
    const int e = routed ? zz_clamp_e(((const ZzTopkWaveHdr *)tk_lds)->idx[js], a.tk.E) : 0;
    const ZzTensor &T = q >= 2 ? f.lay.up : f.lay.gate;
    const int g = 2 * j + (q & 1);
    const uint8_t *E = f.experts + (size_t)e * f.estride;
    // tq2's row alphas of hidden row 32j + tid (tq2.h:154), read with the weights
    float ag = 1.0f, au = 1.0f;
    if (T.fmt == ZZ_FMT_TQ2 && tid < ZZ_BLK) {
        ag = ((const float *)(E + f.lay.gate.off_s))[32 * j + tid];
        au = ((const float *)(E + f.lay.up.off_s))[32 * j + tid];
    }
    auto gates = [&] {
        if (w == 0 && routed && writer) zz_topk_wave_gates(a.tk, s, tk_lds, true);
    };
    // diagnostics: pair p, row 16g + r of the wave's tensor (gate for q < 2), block b;
    // the quarters of a q4_0 / q8_0 block sit in lanes r, r + 16, r + 32, r + 48
    auto dbg = [&](int b, int d, bool whole) {
        if constexpr (DBG) {
            if (!whole) {
                d += __shfl_xor(d, 16);
                d += __shfl_xor(d, 32);
            }
            if (routed && (whole || l < 16))
                f.dbg_up[(((size_t)p * 2 + (q >= 2 ? 1 : 0)) * f.MI + 16 * g + (l & 15)) * (f.D / ZZ_BLK) + b] = d;
        }
    };
    float acc;
    if (T.fmt == ZZ_FMT_Q40) acc = zz_dec_up_part<ZZ_FMT_Q40>(f, sr, st, E, T, g, h, l, gates, dbg);
    else if (T.fmt == ZZ_FMT_Q80) acc = zz_dec_up_part<ZZ_FMT_Q80>(f, sr, st, E, T, g, h, l, gates, dbg);
    else acc = zz_dec_up_part<ZZ_FMT_TQ2>(f, sr, st, E, T, g, h, l, gates, dbg);
    acc = zz_rows_sum(acc);                                     // sum over the 4 k-quarters
    if (l < 16) part[h][q][l] = acc;
    if (T.fmt == ZZ_FMT_TQ2 && tid == 0) {          // tq2.h:101-106, serial
        const int nb = f.D / ZZ_BLK;
        double tot = 0.0;
        for (int b = 0; b < nb; b++) tot += (double)st.xs[b] * (double)st.xsum[b];
        st.xt = (float)tot;
    }
    __syncthreads();
    if (tid < ZZ_BLK) {                                         // hidden row 32j + tid
        const int gg = tid >> 4, r = tid & 15;
        float gv = part[0][gg][r] + part[1][gg][r];
        float uv = part[0][2 + gg][r] + part[1][2 + gg][r];
        if (T.fmt == ZZ_FMT_TQ2) {                              // tq2.h:154
            gv = ag * (gv - st.xt);
            uv = au * (uv - st.xt);
        }
        hb[tid] = zz_act(f.act, gv, uv, f.clamp);
    }
    __syncthreads();
    if (w == 0) {                                               // q8_0 of the block (gemma4.c:646)
        const int m = l & 7;
        const float4 v = *(const float4 *)&hb[4 * m];
        float d;
        int qs;
        const unsigned pk = zz_quant8(v, &d, &qs);
        const int nbM = f.MI / ZZ_BLK;
        if (l < 8) *(unsigned *)(f.hq + (size_t)p * f.MI + 32 * j + 4 * m) = pk;
        if (l == 0) {
            f.hs[(size_t)p * nbM + j] = d;
            f.hsum[(size_t)p * nbM + j] = qs;
        }
    }
}

// ------------------------------------------------------------------ down + combine
// grid D/16, 512 threads: the workgroup owns the 16 output rows of row group g of
// down. First every (token, slot) pair's q8_0 hidden is staged in LDS. Wave w
// takes the pairs w, w+8, ... and walks their units (pair,
// chunk) in order, DD_C units' loads at a time; lane l = 16*qq + r as in the
// gate/up kernel. With fewer pairs than waves (LFM's top-4 at S = 1), the 8 / P
// waves w = p + P*sub of pair p take its chunks sub, sub + 8/P, ... and their
// partial sums meet in LDS in wave order. A pair's partial dots are summed over the 4 k-quarters when its
// last unit is done. The 16 x P expert outputs are then combined per token in slot
// order, out = fma(w_j, y_j, out) as gemma4.c:652.
#define DD_C 12
#define DD_W 8                        // waves
#define DD_QB 4                       // hidden 16-byte segments per thread requested ahead
#define DD_SB 2                       // hidden block scales per thread requested ahead
#define DD_DN 4                       // fused dense-branch chunks per wave (its K <= 4096)

struct ZzDecPairs {                 // per (token, slot) pair, flat order s*K + j
    int e[DEC_MAXS * ZZ_MAXK];      // expert (clamped into the table)
    float w[DEC_MAXS * ZZ_MAXK];    // gate weight
};

// LDS bytes of the staged hidden rows of P pairs: int8 codes, block scales and sums
static inline size_t zz_dec_down_lds(int P, int MI) { return (size_t)P * MI + 8 * (size_t)P * (MI / ZZ_BLK); }

template <int FMT, bool DBG>
__global__ __launch_bounds__(512) void zz_dec_down_kernel(ZzDecDownArgs a) {
    const ZzFfnArgs &f = a.f;
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, r = l & 15, qq = l >> 4;
    const int g = blockIdx.x;
    const ZzTensor &T = f.lay.down;
    const int MI = f.MI, nb = MI / ZZ_BLK, D = f.D, S = a.S, K = a.K, P = S * K;
    const int nch = FMT == ZZ_FMT_TQ2 ? (nb / 2 + 3) / 4 : (nb + 3) / 4;   // units per pair
    const int npw = (P - w + DD_W - 1) / DD_W;                  // this wave's pairs
    // split: nw waves per pair; wave w takes pair w % P, chunks w / P + nw * i
    const int nw = P < DD_W ? DD_W / P : 1, sub = w / P;
    const bool split = nw > 1, active = w < P * nw;
    const int U = split ? (active ? (nch - sub + nw - 1) / nw : 0) : npw * nch;
    __shared__ ZzDecPairs pr;
    __shared__ float yv[DEC_MAXS * ZZ_MAXK][16];
    __shared__ float htot[DEC_MAXS * ZZ_MAXK];
    __shared__ float dpart[DD_W][DEC_MAXS][16];                 // fused dense branch, per wave
    __shared__ float ypart[DD_W][16];                           // split pairs: per wave
    extern __shared__ __attribute__((aligned(16))) char dd_lds[];
    int8_t *sh_q = (int8_t *)dd_lds;                            // [P][MI] by flat pair
    float *sh_s = (float *)(dd_lds + (size_t)P * MI);           // [P][nb]
    int *sh_c = (int *)(sh_s + P * nb);                         // [P][nb]
    // fused dense branch (nd rows): its hidden [nd][MID] and scales [nd][MID/32]
    constexpr bool DN = FMT != ZZ_FMT_TQ2;
    const int nd = DN ? a.nd : 0, MID = a.fd.MI, nbd = MID / ZZ_BLK, nchd = (nbd + 3) / 4;
    int8_t *sh_qd = (int8_t *)(sh_c + P * nb);
    float *sh_sd = (float *)(sh_qd + (size_t)nd * MID);
    if (tid < P) {
        pr.e[tid] = zz_clamp_e(a.eidx[tid], a.E);
        pr.w[tid] = a.ewt[tid];         // read now: the combine at the end would wait for it
    }
    __syncthreads();
    // the pairs' q8_0 hidden (codes, scales, sums by flat pair), requested before the
    // weights (the wait for them then leaves the weight loads in flight; loads
    // complete in order); the LDS writes are unconditional, clamped slots holding
    // copies, so the loads cannot sink past the weights
    const int nseg = P * MI / 16, nsc = P * nb;
    uint4 hv[DD_QB];
    float sv[DD_SB];
    int cv[DD_SB];
#pragma unroll
    for (int k = 0; k < DD_QB; k++) hv[k] = ld16(f.hq + 16 * (size_t)min(tid + 512 * k, nseg - 1));
#pragma unroll
    for (int k = 0; k < DD_SB; k++) {
        const int i = min(tid + 512 * k, nsc - 1);
        sv[k] = f.hs[i];
        cv[k] = f.hsum[i];
    }
    ZzChunk k[DD_C];
    uint4 c[DD_C];
    const ZzWalk W = zz_walk(T, g, l, r);
    auto load_units = [&](int u0) {
#pragma unroll
        for (int i = 0; i < DD_C; i++) {                        // clamped: loads stay in range
            const int u = min(u0 + i, max(U - 1, 0));
            const int fp = split ? w % P : w + DD_W * (u / nch);
            const int ch = split ? min(sub + nw * u, nch - 1) : u % nch;
            const uint8_t *E = f.experts + (size_t)pr.e[min(fp, P - 1)] * f.estride;
            if (FMT == ZZ_FMT_TQ2) c[i] = ld16(E + zz_tq2off(T, 16 * g + r, min(qq + 4 * ch, nb / 2 - 1)));
            else k[i] = zz_load_chunk<FMT>(E, W, ch);
        }
    };
    // diagnostics: flat pair fp, row 16g + r of down, block b (quarters as in gate/up)
    auto dbg = [&](int fp, int b, int d, bool whole) {
        if constexpr (DBG) {
            if (!whole) {
                d += __shfl_xor(d, 16);
                d += __shfl_xor(d, 32);
            }
            if (whole || qq == 0) f.dbg_dn[((size_t)fp * D + 16 * g + r) * nb + b] = d;
        }
    };
    float acc = 0.0f;
    int cur = -1;
    auto comp_units = [&](int u0) {
#pragma unroll
        for (int i = 0; i < DD_C; i++) {
            const int u = u0 + i;
            if (u >= U) continue;
            const int fp = split ? w % P : w + DD_W * (u / nch);
            const int ch = split ? sub + nw * u : u % nch;
            if (fp != cur) {                                    // wave-uniform
                if (cur >= 0) {
                    acc = zz_rows_sum(acc);
                    if (qq == 0) yv[cur][r] = FMT == ZZ_FMT_Q40 ? acc * 0.0625f : acc;
                }
                cur = fp;
                acc = 0.0f;
            }
            const int8_t *hx = sh_q + (size_t)fp * MI;
            const float *hsx = sh_s + fp * nb;
            if (FMT == ZZ_FMT_TQ2) {
                const int gp = qq + 4 * ch;
                if (gp < nb / 2) {
                    const int8_t *x = hx + gp * 64;
                    const int d0 = zz_dot_tq2(c[i], 0, *(const uint4 *)x, *(const uint4 *)(x + 16));
                    const int d1 = zz_dot_tq2(c[i], 1, *(const uint4 *)(x + 32), *(const uint4 *)(x + 48));
                    dbg(fp, 2 * gp, d0, true);
                    dbg(fp, 2 * gp + 1, d1, true);
                    acc = fmaf(hsx[2 * gp], (float)d0, acc);
                    acc = fmaf(hsx[2 * gp + 1], (float)d1, acc);
                }
            } else {
                const int cbs = zz_cbs(T, 4 * ch);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (j >= cbs) continue;
                    const int b = 4 * ch + j;
                    const uint2 wv = zz_chunk_w<FMT>(k[i], j);
                    const uint2 xv = *(const uint2 *)(hx + b * ZZ_BLK + 8 * qq);
                    int d = zz_dot4(wv.x, xv.x, 0);
                    d = zz_dot4(wv.y, xv.y, d);
                    dbg(fp, b, d, false);
                    acc = fmaf(zz_chunk_dw(k[i], j, cbs == 4) * hsx[b], (float)d, acc);
                }
            }
        }
    };
    __builtin_amdgcn_sched_barrier(0);                          // hidden loads issue first
    load_units(0);
    // the fused dense branch's chunks of this wave (w, w+8, ...), requested after the
    // routed pairs' first units so that waiting for those leaves these in flight
    ZzChunk kd[DD_DN];
    ZzWalk Wd;
    if (nd) {
        Wd = zz_walk(a.fd.lay.down, g, l, r);
#pragma unroll
        for (int i = 0; i < DD_DN; i++) kd[i] = zz_load_chunk<FMT>(a.fd.experts, Wd, min(w + DD_W * i, nchd - 1));
    }
#pragma unroll
    for (int k = 0; k < DD_QB; k++) *(uint4 *)(sh_q + 16 * (size_t)min(tid + 512 * k, nseg - 1)) = hv[k];
#pragma unroll
    for (int k = 0; k < DD_SB; k++) {
        const int i = min(tid + 512 * k, nsc - 1);
        sh_s[i] = sv[k];
        sh_c[i] = cv[k];
    }
    for (int i = tid + 512 * DD_QB; i < nseg; i += 512) *(uint4 *)(sh_q + 16 * (size_t)i) = ld16(f.hq + 16 * (size_t)i);
    for (int i = tid + 512 * DD_SB; i < nsc; i += 512) {
        sh_s[i] = f.hs[i];
        sh_c[i] = f.hsum[i];
    }
    for (int i = tid; i < nd * MID / 16; i += 512) *(uint4 *)(sh_qd + 16 * (size_t)i) = ld16(a.fd.hq + 16 * (size_t)i);
    for (int i = tid; i < nd * nbd; i += 512) sh_sd[i] = a.fd.hs[i];
    __syncthreads();
    if (FMT == ZZ_FMT_TQ2 && tid < P) {                         // tq2.h:101-106, serial
        double t = 0.0;
        for (int b = 0; b < nb; b++) t += (double)sh_s[tid * nb + b] * (double)sh_c[tid * nb + b];
        htot[tid] = (float)t;
    }
    comp_units(0);
    for (int u0 = DD_C; u0 < U; u0 += DD_C) {
        load_units(u0);
        comp_units(u0);
    }
    if (cur >= 0) {
        acc = zz_rows_sum(acc);
        const float y = FMT == ZZ_FMT_Q40 ? acc * 0.0625f : acc;   // 16*(q - 8) weights
        if (qq == 0) {
            if (split) ypart[w][r] = y;
            else yv[cur][r] = y;
        }
    } else if (split && qq == 0) {
        ypart[w][r] = 0.0f;                                     // a pair with fewer chunks than waves
    }
    if (nd) {                                                   // this wave's dense chunks
        float ad[DEC_MAXS] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < DD_DN; i++) {
            const int cd = w + DD_W * i;
            if (cd >= nchd) break;                              // wave-uniform
            const int cbs = zz_cbs(a.fd.lay.down, 4 * cd);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (j >= cbs) break;
                const int b = 4 * cd + j;
                const uint2 wv = zz_chunk_w<FMT>(kd[i], j);
                const float dw = zz_chunk_dw(kd[i], j, cbs == 4);
#pragma unroll
                for (int q = 0; q < DEC_MAXS; q++) {
                    if (q >= nd) break;
                    const uint2 xv = *(const uint2 *)(sh_qd + (size_t)q * MID + b * ZZ_BLK + 8 * qq);
                    int d = zz_dot4(wv.x, xv.x, 0);
                    d = zz_dot4(wv.y, xv.y, d);
                    ad[q] = fmaf(dw * sh_sd[q * nbd + b], (float)d, ad[q]);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < DEC_MAXS; q++) {
            float v = ad[q];
            v = zz_rows_sum(v);
            if (qq == 0 && q < nd) dpart[w][q][r] = v;
        }
    }
    __syncthreads();
    if (split) {                                                // uniform
        if (tid < P * 16) {                                     // pair p's waves in order
            const int q = tid >> 4, rr = tid & 15;
            float v = ypart[q][rr];
            for (int sb = 1; sb < nw; sb++) v += ypart[q + P * sb][rr];
            yv[q][rr] = v;
        }
        __syncthreads();
    }
    if (nd && tid < nd * 16) {                                  // dense rows 16g.., waves in order
        const int q = tid >> 4, rr = tid & 15;
        float v = dpart[0][q][rr];
#pragma unroll
        for (int ww = 1; ww < DD_W; ww++) v += dpart[ww][q][rr];
        if (FMT == ZZ_FMT_Q40) v *= 0.0625f;
        a.yd[(size_t)q * D + g * 16 + rr] = v;
        double t = (double)v * (double)v;
        t = zz_group_sum<16>(t);
        if (rr == 0) a.ssd[(size_t)q * gridDim.x + g] = t;
    }
    if (tid < S * 16) {
        const int s = tid >> 4, rr = tid & 15, o = g * 16 + rr;
        float v = 0.0f;
        for (int j = 0; j < K; j++) {
            const int fp = s * K + j;
            float y = yv[fp][rr];
            if (FMT == ZZ_FMT_TQ2) {
                const float alpha = ((const float *)(f.experts + (size_t)pr.e[fp] * f.estride + T.off_s))[o];
                y = alpha * (y - htot[fp]);        // tq2.h:154
            }
            v = fmaf(pr.w[fp], y, v);
        }
        a.out[(size_t)s * D + o] = v;
        if (a.ss) {                               // this tile's sum of squares, for the post-norm
            double q = (double)v * (double)v;
            q = zz_group_sum<16>(q);
            if (rr == 0) a.ss[(size_t)s * gridDim.x + g] = q;
        }
    }
}

// gemma post-norm of the decode rows: out = rmsnorm(out, post_ffn_ln2)
// (gemma4.c:807-808). grid (D/256, S): every workgroup sums the token's G per-tile
// sums of squares (double, fixed order: lane-strided, then a fixed butterfly) while
// its 256 outputs and weights are in flight, then scales them.
__global__ __launch_bounds__(256) void zz_dec_norm_kernel(float *out, const float *post_ln, const double *ss, int G,
                                                          int D, float eps) {
    __shared__ float rn;
    const int tid = threadIdx.x, s = blockIdx.y, i = min(256 * blockIdx.x + tid, D - 1);
    float *o = out + (size_t)s * D;
    const float v = o[i], w = post_ln[i];
    if (tid < 64) {
        double q = 0.0;
        for (int k = tid; k < G; k += 64) q += ss[(size_t)s * G + k];
        q = zz_group_sum<64>(q);
        if (tid == 0) rn = 1.0f / sqrtf((float)(q / D) + eps);
    }
    __syncthreads();
    if (256 * blockIdx.x + tid < D) o[i] = (v * rn) * w;
}

int zz_launch_dec_logits(const ZzDecRouteArgs &a, hipStream_t st) {
    const int R = (a.prep.D + 255) / 256;
    const dim3 g(a.dense ? 16 : a.lg.E);
    if (a.fin) {                                     // zz_dec_fin_fits holds
        if (R <= 12) hipLaunchKernelGGL((zz_dec_logits_kernel<12, true>), g, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((zz_dec_logits_kernel<16, true>), g, dim3(256), 0, st, a);
    }
    else if (R <= 4) hipLaunchKernelGGL((zz_dec_logits_kernel<4, false>), g, dim3(256), 0, st, a);
    else if (R <= 8) hipLaunchKernelGGL((zz_dec_logits_kernel<8, false>), g, dim3(256), 0, st, a);
    else if (R <= 12) hipLaunchKernelGGL((zz_dec_logits_kernel<12, false>), g, dim3(256), 0, st, a);
    else if (R <= 16) hipLaunchKernelGGL((zz_dec_logits_kernel<16, false>), g, dim3(256), 0, st, a);
    else if (R <= 24) hipLaunchKernelGGL((zz_dec_logits_kernel<24, false>), g, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((zz_dec_logits_kernel<32, false>), g, dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

// a deferred combine fits the router's LDS rows (and its RB <= 16 forms)
int zz_dec_fin_fits(int S, int D) {
    return S > 0 && D % 4 == 0 && D <= 4096 && (long)S * D <= ZZ_DEC_FIN_MAXF;
}

int zz_launch_dec_up(const ZzDecUpArgs &a, int S, hipStream_t st) {
    const int n = S * a.tk.K * (a.f.MI / ZZ_BLK) + a.nd * (a.nd ? a.fd.MI / ZZ_BLK : 0);
    if (a.f.dbg_up) hipLaunchKernelGGL(zz_dec_up_kernel<true>, dim3(n), dim3(512), zz_topk_wave_bytes(a.tk.E), st, a);
    else hipLaunchKernelGGL(zz_dec_up_kernel<false>, dim3(n), dim3(512), zz_topk_wave_bytes(a.tk.E), st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_dec_fits(int S, int K, int MI) { return zz_dec_down_lds(S * K, MI) <= ZZ_DEC_LDS; }

// a dense branch of intermediate MID fused in: its S hidden rows and scales beside the
// routed pairs', and at most DD_DN of its chunks per wave
static inline size_t zz_dec_dense_lds(int S, int MID) { return (size_t)S * MID + 4 * (size_t)S * (MID / ZZ_BLK); }
int zz_dec_fits2(int S, int K, int MI, int MID) {
    return zz_dec_down_lds(S * K, MI) + zz_dec_dense_lds(S, MID) <= ZZ_DEC_LDS &&
           (MID / ZZ_BLK + 3) / 4 <= DD_W * DD_DN;
}

int zz_launch_dec_down(const ZzDecDownArgs &a, hipStream_t st) {
    const dim3 grid(a.f.D / 16);
    const int nd = a.nd && a.f.lay.down.fmt != ZZ_FMT_TQ2 ? a.nd : 0;
    const size_t lds = zz_dec_down_lds(a.S * a.K, a.f.MI) + (nd ? zz_dec_dense_lds(nd, a.fd.MI) : 0);
    if (nd ? !zz_dec_fits2(a.S, a.K, a.f.MI, a.fd.MI) : !zz_dec_fits(a.S, a.K, a.f.MI)) return 0;
    const int fmt = a.f.lay.down.fmt;
    if (fmt != ZZ_FMT_Q40 && fmt != ZZ_FMT_Q80 && fmt != ZZ_FMT_TQ2) return 0;
    if (a.f.dbg_dn) {
        if (fmt == ZZ_FMT_Q40) hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_Q40, true>), grid, dim3(512), lds, st, a);
        else if (fmt == ZZ_FMT_Q80) hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_Q80, true>), grid, dim3(512), lds, st, a);
        else hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_TQ2, true>), grid, dim3(512), lds, st, a);
    } else {
        if (fmt == ZZ_FMT_Q40) hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_Q40, false>), grid, dim3(512), lds, st, a);
        else if (fmt == ZZ_FMT_Q80) hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_Q80, false>), grid, dim3(512), lds, st, a);
        else hipLaunchKernelGGL((zz_dec_down_kernel<ZZ_FMT_TQ2, false>), grid, dim3(512), lds, st, a);
    }
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dec_norm(float *out, const float *post_ln, const double *ss, int D, float eps, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_norm_kernel, dim3((D + 255) / 256, S), dim3(256), 0, st, out, post_ln, ss, D / 16, D, eps);
    return hipGetLastError() == hipSuccess;
}

// The tail of a gemma FFN block whose dense branch ran fused into the routed layer's
// decode kernels: the two post-norms from their per-tile sums (each formed as
// zz_dec_norm_kernel forms it), then the layer combine as zz_block_combine_kernel
// forms it (gemma4.c:807-808, 1020, 1022-1030). One workgroup per token.
__global__ __launch_bounds__(256) void zz_dec_final_kernel(ZzDecFinalArgs a) {
    __shared__ __attribute__((aligned(16))) float row[ZZ_MAXD];
    __shared__ double red[4];
    zz_dec_final_row<4>(a, blockIdx.x, row, red, true);
}

int zz_launch_dec_final(const ZzDecFinalArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_final_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}
