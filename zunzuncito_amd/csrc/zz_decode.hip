// zz_decode.hip -- decode-sized batches (S <= 4 tokens):
//   1. zz_dec_logits_kernel: one workgroup per expert computes that expert's
//      certified router logit for every token (gemma: with the input rmsnorm from
//      the same loads) and quantises a share of the expert input;
//   2. zz_dec_gate_kernel: one workgroup runs the top-k gating and builds the
//      dispatch lists (gemma4.c:750-790 for a handful of rows);
//   3. zz_dec_up_kernel: gate/up GEMV with the activation and the int8
//      re-quantisation of the hidden, per expert work item;
//   4. zz_dec_down_kernel: down GEMV for all (token, slot) pairs of a row tile
//      and the gate-weighted combine (gemma4.c:652); gemma's post-norm
//      (gemma4.c:807-808) follows as a one-workgroup-per-token kernel.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_route_dev.h"
#include "zz_topk_wave.h"
#include "zz_dot_dev.h"

#define DEC_MAXS ZZ_DEC_MAXS

// expert id kept inside the slot table whatever the router produced
__device__ __forceinline__ int zz_clamp_e(int e, int E) { return e < 0 || e >= E ? 0 : e; }

// Decode router, part 1: one workgroup per expert e. Gemma: per token, one set of
// loads (x row, router row e, router scale) gives both the rmsnorm factor and the
// rounded products of the router logit. The mean square is certified to round to
// the float of the reference's serial double sum (gemma4.c:425-428), else that sum
// is replayed; the logit gets the tight bound of zz_tight_block_scan. lfm/maple:
// wave s computes token s's logit. Then the workgroup quantises its share of the
// expert input (blocks e, e + E, ...).
// RB >= ceil(D/256): loads per thread and token, all issued before any is used.
template <int RB>
__global__ __launch_bounds__(256) void zz_dec_logits_kernel(ZzDecRouteArgs a) {
    const ZzPrepArgs &pp = a.prep;
    const ZzLogitArgs &lg = a.lg;
    const int S = a.S, D = pp.D, nb = D / ZZ_BLK, tid = threadIdx.x, e = blockIdx.x;
    const bool gem = pp.gemma;
    __shared__ __attribute__((aligned(16))) float buf[ZZ_MAXD + ZZ_MAXD / 32];
    __shared__ double red[12];
    __shared__ float rr[DEC_MAXS];
    __shared__ float cert;
    const float rs = 1.0f / sqrtf((float)D);
    if (gem) {
        const int R = (D + 255) >> 8;                         // <= RB
        const float *w = lg.router + (size_t)e * D;
        float wr[RB], sr[RB];
#pragma unroll
        for (int j = 0; j < RB; j++) {                        // clamped: loads stay in range
            const int i = min(tid + 256 * j, D - 1);
            wr[j] = w[i];
            sr[j] = pp.router_scale[i];
        }
#pragma unroll
        for (int j = 0; j < RB; j++) sr[j] = sr[j] * rs;
        for (int s = 0; s < S; s++) {
            const float *x = pp.in + (size_t)s * D;
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
            zz_tight_block_scan<RB>(buf, D, lg.bias, e, red, lg.cen + (size_t)s * lg.E + e,
                                lg.bnd + (size_t)s * lg.E + e);
        }
    } else if ((tid >> 6) < S) {
        zz_logit_wave_f64(lg, tid >> 6, e);
    }
    // the expert input quantisation, block g on workgroup g % gridDim.x
    __syncthreads();
    for (int g = e + gridDim.x * tid; g < S * nb; g += gridDim.x * 256) {
        const int s = g / nb, b = g % nb;
        const float *x = pp.in + (size_t)s * D + b * ZZ_BLK;
        float v[ZZ_BLK];
#pragma unroll
        for (int j = 0; j < ZZ_BLK; j += 4) {
            const float4 t = *(const float4 *)(x + j);
            v[j] = t.x; v[j + 1] = t.y; v[j + 2] = t.z; v[j + 3] = t.w;
        }
        if (gem) {
            const float r = rr[s];
#pragma unroll
            for (int j = 0; j < ZZ_BLK; j += 4) {
                const float4 w = *(const float4 *)(pp.pre_ln + b * ZZ_BLK + j);
                v[j] = (v[j] * r) * w.x; v[j + 1] = (v[j + 1] * r) * w.y;
                v[j + 2] = (v[j + 2] * r) * w.z; v[j + 3] = (v[j + 3] * r) * w.w;
            }
        }
        int qs;
        const float d = zz_quant_block(v, pp.xq + (size_t)s * D + b * ZZ_BLK, &qs);
        pp.xs[(size_t)s * nb + b] = d;
        pp.xsum[(size_t)s * nb + b] = qs;
    }
}

// Decode router, part 2 (one workgroup, one wave per token): certified top-k
// gating (zz_topk_wave.h), then the dispatch of the S*K pairs.
__global__ __launch_bounds__(256) void zz_dec_gate_kernel(ZzDecRouteArgs a) {
    extern __shared__ __attribute__((aligned(16))) char tk_lds[];
    const int S = a.S, tid = threadIdx.x, w = tid >> 6;
    zz_topk_wave_any(a.tk, w, tk_lds + w * zz_topk_wave_bytes(a.tk.E));
    __syncthreads();
    // dispatch of P = S*K <= 64 pairs: stable ranking by (expert, pair index)
    const ZzDispatchArgs &dp = a.dp;
    const int K = dp.K, P = S * K;
    __shared__ int pe[DEC_MAXS * ZZ_MAXK], pf[DEC_MAXS * ZZ_MAXK];
    if (tid < P) {
        const int e = dp.eidx[tid];
        pe[tid] = e < 0 || e >= dp.E ? 0 : e;     // never index past the expert tables
    }
    __syncthreads();
    int ep = 0, rank = 0, start = 0, cnt = 0, first = 1;
    if (tid < P) {
        ep = pe[tid];
        for (int q = 0; q < P; q++) {
            const int eq = pe[q];
            rank += eq < ep || (eq == ep && q < tid);
            start += eq < ep;
            cnt += eq == ep;
            first &= !(q < tid && eq == ep);
        }
        pf[tid] = first;                          // first occurrence of its expert
    }
    __syncthreads();
    if (tid < P) {
        int urank = 0;                            // union order: first-seen
        for (int q = 0; q < tid; q++) urank += pf[q];
        dp.ptok[rank] = tid / K;
        dp.pslot[rank] = tid % K;
        dp.pwt[rank] = dp.ewt[tid];
        dp.ppos[tid] = rank;
        if (first) {
            dp.uniq[urank] = ep;
            dp.uoff[urank] = start;
            dp.ucnt[urank] = cnt;
            ZzItem it;
            it.e = ep;
            it.u = urank;
            it.p0 = start;
            it.n = cnt;                            // cnt <= S <= 4 fits one item
            dp.items[urank] = it;
        }
        if (tid == P - 1) {
            const int nu = urank + first;
            dp.meta[0] = nu;
            dp.meta[1] = nu;
        }
    }
}

// ------------------------------------------------------------------ gate/up
// grid (MI/32, items): the workgroup owns hidden rows 32*blockIdx.x .. +31 of one
// expert item (<= ZZ_DEC_MAXS tokens). Waves 0-3 take the 32 gate rows, waves 4-7
// the 32 up rows, 8 lanes per row; lane `sub` takes blocks sub, sub+8, ... and
// issues DU_J of them at once, before the activations are staged in LDS, so the
// weight stream is in flight from the first cycle.
#define DU_J 12

// one workgroup-wide staging of the item's activations into LDS
struct ZzDecStage {
    __attribute__((aligned(16))) int8_t xq[DEC_MAXS][ZZ_MAXD];
    float xs[DEC_MAXS][ZZ_MAXD / ZZ_BLK];
    int xsum[DEC_MAXS][ZZ_MAXD / ZZ_BLK];
    int tok[DEC_MAXS];
    float xt[DEC_MAXS];         // tq2 Sx of each token
};

__device__ __forceinline__ void zz_dec_stage(const ZzFfnArgs &a, const ZzItem &item, ZzDecStage &st) {
    const int D = a.D, nb = D / ZZ_BLK;
    for (int t = 0; t < item.n; t++) {
        const int tk = st.tok[t];
        for (int i = 16 * threadIdx.x; i < D; i += 16 * blockDim.x)
            *(uint4 *)&st.xq[t][i] = ld16(a.xq + (size_t)tk * D + i);
        for (int b = threadIdx.x; b < nb; b += blockDim.x) {
            st.xs[t][b] = a.xs[(size_t)tk * nb + b];
            st.xsum[t][b] = a.xsum[(size_t)tk * nb + b];
        }
    }
    __syncthreads();
}

// Partial dots of one lane for one row: weights of DU_J blocks (tq2: groups) are
// loaded first, then the activations are staged (once per workgroup), then used.
template <int FMT>
__device__ __forceinline__ void zz_dec_up_part(const ZzFfnArgs &a, const ZzItem &item, ZzDecStage &st,
                                               const uint8_t *E, const ZzTensor &T, int row, int sub,
                                               float (&acc)[DEC_MAXS]) {
    const int nb = a.D / ZZ_BLK, n = item.n;
    const int nu = FMT == ZZ_FMT_TQ2 ? nb / 2 : nb;          // units: blocks or 64-groups
#pragma unroll
    for (int t = 0; t < DEC_MAXS; t++) acc[t] = 0.0f;
    for (int u0 = 0; u0 < nu; u0 += 8 * DU_J) {
        uint4 w0[DU_J], w1[DU_J];
        float dw[DU_J];
#pragma unroll
        for (int j = 0; j < DU_J; j++) {
            const int u = min(u0 + sub + 8 * j, nu - 1);       // clamped: loads stay in range
            const uint8_t *qp = E + zz_qoff(T, row, u);
            w0[j] = ld16(qp);
            if (FMT == ZZ_FMT_Q80) w1[j] = ld16(qp + 16);
            if (FMT != ZZ_FMT_TQ2) dw[j] = zz_h2f(*(const uint16_t *)(E + zz_soff(T, row, u)));
        }
        if (u0 == 0) zz_dec_stage(a, item, st);               // uniform: every wave passes here
#pragma unroll
        for (int j = 0; j < DU_J; j++) {
            const int u = u0 + sub + 8 * j;
            if (u >= nu) continue;
#pragma unroll
            for (int t = 0; t < DEC_MAXS; t++) {
                if (t >= n) continue;
                if (FMT == ZZ_FMT_TQ2) {
                    const int8_t *x = &st.xq[t][u * 64];
                    const int d0 = zz_dot_tq2(w0[j], 0, ld16(x), ld16(x + 16));
                    const int d1 = zz_dot_tq2(w0[j], 1, ld16(x + 32), ld16(x + 48));
                    acc[t] = fmaf(st.xs[t][2 * u], (float)d0, acc[t]);
                    acc[t] = fmaf(st.xs[t][2 * u + 1], (float)d1, acc[t]);
                } else {
                    const int8_t *x = &st.xq[t][u * ZZ_BLK];
                    const uint4 x0 = ld16(x), x1 = ld16(x + 16);
                    const int d = FMT == ZZ_FMT_Q80 ? zz_dot_q80(w0[j], w1[j], x0, x1)
                                                    : zz_dot_q40(w0[j], x0, x1) - 8 * st.xsum[t][u];
                    acc[t] = fmaf(dw[j] * st.xs[t][u], (float)d, acc[t]);
                }
            }
        }
    }
}

__global__ __launch_bounds__(512) void zz_dec_up_kernel(ZzFfnArgs a) {
    const int it = blockIdx.y;
    if (it >= a.meta[1]) return;
    const ZzItem item = a.items[it];
    const int tid = threadIdx.x, rr = tid >> 3, sub = tid & 7, rb = blockIdx.x;
    const bool up = rr >= 32;
    const ZzTensor &T = up ? a.lay.up : a.lay.gate;
    const int row = rb * 32 + (rr & 31);
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    __shared__ ZzDecStage st;
    __shared__ float gu[DEC_MAXS][64];
    __shared__ float hb[DEC_MAXS][ZZ_BLK + 1];
    if (tid < item.n) st.tok[tid] = a.ptok[item.p0 + tid];
    __syncthreads();
    float acc[DEC_MAXS];
    if (T.fmt == ZZ_FMT_Q40) zz_dec_up_part<ZZ_FMT_Q40>(a, item, st, E, T, row, sub, acc);
    else if (T.fmt == ZZ_FMT_Q80) zz_dec_up_part<ZZ_FMT_Q80>(a, item, st, E, T, row, sub, acc);
    else zz_dec_up_part<ZZ_FMT_TQ2>(a, item, st, E, T, row, sub, acc);
    if (T.fmt == ZZ_FMT_TQ2 && tid < item.n) {      // tq2.h:101-106, serial
        const int nb = a.D / ZZ_BLK;
        double tot = 0.0;
        for (int b = 0; b < nb; b++) tot += (double)st.xs[tid][b] * (double)st.xsum[tid][b];
        st.xt[tid] = (float)tot;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < DEC_MAXS; t++) {
        float v = acc[t];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        if (T.fmt == ZZ_FMT_TQ2 && t < item.n) {
            const float alpha = ((const float *)(E + T.off_s))[row];
            v = alpha * (v - st.xt[t]);                        // tq2.h:154
        }
        if (sub == 0) gu[t][rr] = v;
    }
    __syncthreads();
    if (tid < item.n * ZZ_BLK) {
        const int t = tid >> 5, r = tid & 31;
        hb[t][r] = zz_act(a.act, gu[t][r], gu[t][32 + r], a.clamp);
    }
    __syncthreads();
    if (tid < item.n) {                                         // one thread per token block
        float v[ZZ_BLK];
#pragma unroll
        for (int r = 0; r < ZZ_BLK; r++) v[r] = hb[tid][r];
        const size_t p = (size_t)item.p0 + tid;
        int qs;
        const float d = zz_quant_block(v, a.hq + p * a.MI + rb * ZZ_BLK, &qs);
        a.hs[p * (a.MI / ZZ_BLK) + rb] = d;
        a.hsum[p * (a.MI / ZZ_BLK) + rb] = qs;
    }
}

// ------------------------------------------------------------------ down + combine
// grid D/8: the workgroup owns 8 output rows, 32 lanes per row. A row's work is
// P * nu units (pair, block) -- nu blocks of 32 (q4_0 / q8_0) or 64-groups (tq2)
// per (token, slot) pair; lane q takes units q, q+32, ..., DD_U at a time with
// every load issued before any is used. Unit results meet in LDS and each
// (row, pair) sum runs in block order; the 8 x P expert outputs are then combined
// per token in slot order, out = fma(w_j, y_j, out) as gemma4.c:652.
#define DD_RW 8
#define DD_U 12
#define DD_UB 1024                    // unit results per row held at once

struct ZzDecPairs {                 // per (token, slot) pair, flat order s*K + j
    int pos[DEC_MAXS * ZZ_MAXK];    // sorted position: row of hq / hs / hsum
    int e[DEC_MAXS * ZZ_MAXK];      // expert (clamped into the table)
};

template <int FMT>
__global__ __launch_bounds__(256) void zz_dec_down_kernel(ZzDecDownArgs a) {
    const ZzFfnArgs &f = a.f;
    const int tid = threadIdx.x, r = tid >> 5, q = tid & 31;
    const int row = blockIdx.x * DD_RW + r;
    const ZzTensor &T = f.lay.down;
    const int MI = f.MI, nb = MI / ZZ_BLK, D = f.D, S = a.S, K = a.K, P = S * K;
    const int nu = FMT == ZZ_FMT_TQ2 ? nb / 2 : nb;
    const int PG = min(P, DD_UB / nu);                          // pairs per group, >= 1
    __shared__ ZzDecPairs pr;
    __shared__ float ub[DD_RW][DD_UB];
    __shared__ float yv[DEC_MAXS * ZZ_MAXK][DD_RW];
    __shared__ float htot[DEC_MAXS * ZZ_MAXK];
    if (tid < P) {
        pr.pos[tid] = a.ppos[tid];
        pr.e[tid] = zz_clamp_e(a.eidx[tid], a.E);
    }
    if (FMT == ZZ_FMT_TQ2 && tid < P) {            // tq2.h:101-106, serial
        const size_t p = (size_t)a.ppos[tid];
        double t = 0.0;
        for (int b = 0; b < nb; b++) t += (double)f.hs[p * nb + b] * (double)f.hsum[p * nb + b];
        htot[tid] = (float)t;
    }
    __syncthreads();
    for (int pg0 = 0; pg0 < P; pg0 += PG) {
        const int np = min(PG, P - pg0), U = np * nu;
        for (int u0 = 0; u0 < U; u0 += 32 * DD_U) {
            uint4 w0[DD_U], w1[DD_U], x0[DD_U], x1[DD_U], x2[DD_U], x3[DD_U];
            float dw[DD_U], s0[DD_U], s1[DD_U];
            int hm[DD_U];
#pragma unroll
            for (int j = 0; j < DD_U; j++) {                     // clamped: loads stay in range
                const int u = min(u0 + q + 32 * j, U - 1);
                const int pp = pg0 + u / nu, b = u % nu;
                const int p = pr.pos[pp];
                const uint8_t *E = f.experts + (size_t)pr.e[pp] * f.estride;
                const uint8_t *qp = E + zz_qoff(T, row, b);
                w0[j] = ld16(qp);
                if (FMT == ZZ_FMT_TQ2) {
                    const int8_t *x = f.hq + (size_t)p * MI + b * 64;
                    x0[j] = ld16(x);
                    x1[j] = ld16(x + 16);
                    x2[j] = ld16(x + 32);
                    x3[j] = ld16(x + 48);
                    s0[j] = f.hs[(size_t)p * nb + 2 * b];
                    s1[j] = f.hs[(size_t)p * nb + 2 * b + 1];
                } else {
                    if (FMT == ZZ_FMT_Q80) w1[j] = ld16(qp + 16);
                    dw[j] = zz_h2f(*(const uint16_t *)(E + zz_soff(T, row, b)));
                    const int8_t *x = f.hq + (size_t)p * MI + b * ZZ_BLK;
                    x0[j] = ld16(x);
                    x1[j] = ld16(x + 16);
                    s0[j] = f.hs[(size_t)p * nb + b];
                    if (FMT == ZZ_FMT_Q40) hm[j] = f.hsum[(size_t)p * nb + b];
                }
            }
#pragma unroll
            for (int j = 0; j < DD_U; j++) {
                const int u = u0 + q + 32 * j;
                float c;
                if (FMT == ZZ_FMT_TQ2) {
                    const int d0 = zz_dot_tq2(w0[j], 0, x0[j], x1[j]);
                    const int d1 = zz_dot_tq2(w0[j], 1, x2[j], x3[j]);
                    c = fmaf(s1[j], (float)d1, s0[j] * (float)d0);
                } else {
                    const int d = FMT == ZZ_FMT_Q80 ? zz_dot_q80(w0[j], w1[j], x0[j], x1[j])
                                                    : zz_dot_q40(w0[j], x0[j], x1[j]) - 8 * hm[j];
                    c = (dw[j] * s0[j]) * (float)d;
                }
                if (u < U) ub[r][u] = c;
            }
        }
        __syncthreads();
        for (int t = tid; t < DD_RW * np; t += 256) {             // (row, pair) sums, block order
            const int rr = t / np, pl = t % np;
            const float *c = &ub[rr][pl * nu];
            float y = 0.0f;
            for (int b = 0; b < nu; b++) y += c[b];
            yv[pg0 + pl][rr] = y;
        }
        __syncthreads();
    }
    if (tid < S * DD_RW) {
        const int s = tid / DD_RW, rr = tid % DD_RW, o = blockIdx.x * DD_RW + rr;
        float v = 0.0f;
        for (int j = 0; j < K; j++) {
            const int fp = s * K + j;
            float y = yv[fp][rr];
            if (FMT == ZZ_FMT_TQ2) {
                const float alpha = ((const float *)(f.experts + (size_t)pr.e[fp] * f.estride + T.off_s))[o];
                y = alpha * (y - htot[fp]);        // tq2.h:154
            }
            v = fmaf(a.ewt[fp], y, v);
        }
        a.out[(size_t)s * D + o] = v;
    }
}

// gemma post-norm of the decode rows: out = rmsnorm(out, post_ffn_ln2)
// (gemma4.c:807-808), one workgroup per token, sum of squares in double
__global__ __launch_bounds__(256) void zz_dec_norm_kernel(float *out, const float *post_ln, int D, float eps) {
    __shared__ double red[4];
    float *o = out + (size_t)blockIdx.x * D;
    double ss = 0.0;
    for (int i = 4 * threadIdx.x; i < D; i += 1024) {
        const float4 v = *(const float4 *)(o + i);
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    ss = zz_block_sum(ss, red);
    const float r = 1.0f / sqrtf((float)(ss / D) + eps);
    for (int i = 4 * threadIdx.x; i < D; i += 1024) {
        float4 v = *(const float4 *)(o + i);
        const float4 w = *(const float4 *)(post_ln + i);
        v = make_float4((v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w);
        *(float4 *)(o + i) = v;
    }
}

int zz_launch_dec_route(const ZzDecRouteArgs &a, hipStream_t st) {
    const int R = (a.prep.D + 255) / 256;
    if (R <= 4) hipLaunchKernelGGL(zz_dec_logits_kernel<4>, dim3(a.lg.E), dim3(256), 0, st, a);
    else if (R <= 8) hipLaunchKernelGGL(zz_dec_logits_kernel<8>, dim3(a.lg.E), dim3(256), 0, st, a);
    else if (R <= 12) hipLaunchKernelGGL(zz_dec_logits_kernel<12>, dim3(a.lg.E), dim3(256), 0, st, a);
    else if (R <= 16) hipLaunchKernelGGL(zz_dec_logits_kernel<16>, dim3(a.lg.E), dim3(256), 0, st, a);
    else if (R <= 24) hipLaunchKernelGGL(zz_dec_logits_kernel<24>, dim3(a.lg.E), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(zz_dec_logits_kernel<32>, dim3(a.lg.E), dim3(256), 0, st, a);
    if (hipGetLastError() != hipSuccess) return 0;
    hipLaunchKernelGGL(zz_dec_gate_kernel, dim3(1), dim3(64 * a.S), a.S * zz_topk_wave_bytes(a.tk.E), st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dec_up(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_up_kernel, dim3(a.MI / 32, max_items), dim3(512), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dec_down(const ZzDecDownArgs &a, hipStream_t st) {
    const dim3 grid(a.f.D / DD_RW);
    switch (a.f.lay.down.fmt) {
    case ZZ_FMT_Q40: hipLaunchKernelGGL(zz_dec_down_kernel<ZZ_FMT_Q40>, grid, dim3(256), 0, st, a); break;
    case ZZ_FMT_Q80: hipLaunchKernelGGL(zz_dec_down_kernel<ZZ_FMT_Q80>, grid, dim3(256), 0, st, a); break;
    case ZZ_FMT_TQ2: hipLaunchKernelGGL(zz_dec_down_kernel<ZZ_FMT_TQ2>, grid, dim3(256), 0, st, a); break;
    default: return 0;
    }
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dec_norm(float *out, const float *post_ln, int D, float eps, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_norm_kernel, dim3(S), dim3(256), 0, st, out, post_ln, D, eps);
    return hipGetLastError() == hipSuccess;
}
