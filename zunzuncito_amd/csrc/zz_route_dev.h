// zz_route_dev.h -- router device functions shared by the batched kernels
// (zz_route.hip) and the fused decode kernels (zz_decode.hip).
#pragma once
#include "zz_common.h"
#include "zz_kernels.h"

// gamma_k = k*u / (1 - k*u), Higham's constant for k roundings of unit roundoff u
__device__ __forceinline__ double zz_gamma(double k, double u) { return k * u / (1.0 - k * u); }
#define ZZ_U32 5.9604644775390625e-08     // 2^-24
#define ZZ_U64 1.1102230246251565e-16     // 2^-53

// -------------------------------------------------------------------------------
// Block-wide reductions over 256 threads (4 waves).
template <typename T>
__device__ __forceinline__ T zz_block_sum(T v, T *red) {
    v = zz_wave_sum(v);
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    T s = red[0] + red[1] + red[2] + red[3];
    return s;
}

// -------------------------------------------------------------------------------
// Router logits: one wave per (token, expert). Lane l takes elements l, l+64, ...
// Gemma: t_i = fl(w_i * xn_i) exactly as the reference rounds them, summed in fp32
// per lane and across the wave; the bound covers both this sum and the
// reference's in-order fp32 chain: |v_ref - c| <= (g_{D-1} + g_m) * sum|t_i|.
// lfm/maple: products are exact in double; the double sum is certified to round
// to the same float as the reference's serial double sum, else replayed serially.
// One router logit (token s, expert e) by one wave; writes cen/bnd from lane 0.
__device__ __forceinline__ void zz_logit_wave(const ZzLogitArgs &a, int s, int e) {
    const int l = threadIdx.x & 63;
    const int D = a.D;
    const float *w = a.router + (size_t)e * D;
    const size_t o = (size_t)s * a.E + e;
    if (a.gating == ZZ_GATE_SOFTMAX_PES) {
        const float *xn = a.xn + (size_t)s * D;
        float c = 0.0f, t = 0.0f;
        for (int i = l; i < D; i += 64) {
            float p = w[i] * xn[i];
            c += p;
            t += fabsf(p);
        }
        c = zz_wave_sum(c);
        t = zz_wave_sum(t);
        if (l == 0) {
            double m = (double)((D + 63) / 64 + 6);
            double gm = zz_gamma(m, ZZ_U32);
            double T = (double)t / (1.0 - gm);               // rigorous upper bound
            double b = (zz_gamma(D - 1, ZZ_U32) + gm) * T * 1.0000001 + 1e-40;
            double cen = (double)c;
            if (a.bias) {                                    // v' = fl(v + bias_e)
                cen += (double)a.bias[e];
                b += 2.0 * ZZ_U32 * (fabs(cen) + b) + 1e-40;
            }
            a.cen[o] = cen;
            a.bnd[o] = b;
        }
    } else {
        const float *xv = a.x + (size_t)s * D;
        double c = 0.0, t = 0.0;
        for (int i = l; i < D; i += 64) {
            double p = (double)w[i] * (double)xv[i];
            c += p;
            t += fabs(p);
        }
        c = zz_wave_sum(c);
        t = zz_wave_sum(t);
        if (l == 0) {
            double m = (double)((D + 63) / 64 + 6);
            double b = (zz_gamma(D - 1, ZZ_U64) + zz_gamma(m, ZZ_U64)) * t * 1.0000001 + 1e-300;
            float lo = (float)(c - b), hi = (float)(c + b), v = lo;
            if (lo != hi) {
                double r = 0.0;                      // serial replay, reference order
                for (int i = 0; i < D; i++) r += (double)w[i] * (double)xv[i];
                v = (float)r;
                atomicAdd(a.diag + 1, 1u);
            }
            a.cen[o] = (double)v;                    // exact float logit
            a.bnd[o] = 0.0;
        }
    }
}

// -------------------------------------------------------------------------------
// Top-k with interval certification. Each expert carries [lo, hi] containing the
// reference's selection score. Candidates are experts whose hi reaches the k-th
// largest lo; a candidate is contested when its interval meets another
// candidate's. No contested candidate => the reference's top-k set and order are
// fixed by the centres. Contested gemma experts are refined (exact prefix-sum
// bound), then replayed serially; contested lfm scores (glibc expf in the
// reference, lfm25.c:648) are flagged for the caller.
struct ZzTopkShared {
    double lo[ZZ_MAXE], hi[ZZ_MAXE];
    int cand[ZZ_MAXE], cont[ZZ_MAXE];
    float sg[ZZ_MAXE];
    int list[ZZ_MAXE];
    int nlist;
    int any;
    int width;                           // some interval has non-zero width
    double lk;
    int idx[ZZ_MAXK];
    float topv[ZZ_MAXK];
    double red[4];
    float prod[2][4096];                 // stage-3 products, waves 0 and 1 (D <= 4096)
};

__device__ void zz_mark_contested(ZzTopkShared &sh, int E, int K) {
    // k-th largest lo (ties broken by index)
    for (int e = threadIdx.x; e < E; e += 256) {
        int rank = 0;
        double le = sh.lo[e];
#pragma unroll 8
        for (int f = 0; f < E; f++) {
            double lf = sh.lo[f];
            rank += (lf > le) || (lf == le && f < e);
        }
        if (rank == K - 1) sh.lk = le;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256) sh.cand[e] = sh.hi[e] >= sh.lk;
    if (threadIdx.x == 0) { sh.any = 0; sh.nlist = 0; }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256) {
        int c = 0;
        if (sh.cand[e]) {
#pragma unroll 8
            for (int f = 0; f < E; f++)
                if (f != e && sh.cand[f] && sh.lo[f] <= sh.hi[e] && sh.lo[e] <= sh.hi[f]) { c = 1; break; }
        }
        sh.cont[e] = c;
        if (c) {
            sh.any = 1;
            int k = atomicAdd(&sh.nlist, 1);
            sh.list[k] = e;
        }
    }
    __syncthreads();
}

// Tight bound for one gemma logit, one wave: exact prefix sums S_k of the rounded
// products in double, then |v_ref - S_D| <= u/(1-u) (sum_{k>=2} |S_k| + (D-1) g_D T).
__device__ void zz_refine_wave(const float *w, const float *xn, int D, const float *bias, int e,
                               double *lo, double *hi) {
    const int l = threadIdx.x & 63;
    const int per = (D + 63) / 64, i0 = l * per, i1 = min(D, i0 + per);
    double loc = 0.0, T = 0.0;
    for (int i = i0; i < i1; i++) {
        float p = w[i] * xn[i];
        loc += (double)p;
        T += fabs((double)p);
    }
    // exclusive scan of lane totals
    double inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        double v = __shfl_up(inc, o, 64);
        if (l >= o) inc += v;
    }
    double run = inc - loc, sabs = 0.0;
    for (int i = i0; i < i1; i++) {
        run += (double)(w[i] * xn[i]);
        if (i >= 1) sabs += fabs(run);
    }
    sabs = zz_wave_sum(sabs);
    T = zz_wave_sum(T);
    double tot = __shfl(inc, 63, 64);
    if (l == 0) {
        double gd = zz_gamma(D, ZZ_U64);
        // double-precision slack on every computed prefix (|S_k err| <= g_D^d T)
        double b = ZZ_U32 / (1.0 - ZZ_U32) * (sabs + (double)D * gd * T + (double)(D - 1) * zz_gamma(D, ZZ_U32) * T);
        b = b * 1.000001 + gd * T + 1e-40;
        double cen = tot;
        if (bias) {
            cen += (double)bias[e];
            b += 2.0 * ZZ_U32 * (fabs(cen) + b) + 1e-40;
        }
        *lo = cen - b;
        *hi = cen + b;
    }
}

// Top-k for token s by a whole 256-thread workgroup.
__device__ void zz_topk_token(const ZzTopkArgs &a, int s, ZzTopkShared &sh) {
    const int E = a.E, K = a.K;
    const double *cen = a.cen + (size_t)s * E, *bnd = a.bnd + (size_t)s * E;
    int contested = 0;
    if (threadIdx.x == 0) sh.width = a.gating == ZZ_GATE_SIGMOID_BIAS;
    __syncthreads();
    if (threadIdx.x < K) {          // valid ids even if NaN scores leave ranks unfilled
        sh.idx[threadIdx.x] = threadIdx.x;
        sh.topv[threadIdx.x] = 0.0f;
    }

    if (a.gating == ZZ_GATE_SIGMOID_BIAS) {
        // s = 1/(1+expf(-v)) with exp evaluated in double and rounded once; glibc's
        // expf is within 1 ulp of that, so each s is within 2 ulps of the
        // reference's and sel = s + bias within 2 ulp(s) + ulp(sel).
        for (int e = threadIdx.x; e < E; e += 256) {
            float v = (float)cen[e];
            float ex = (float)exp(-(double)v);
            float sg = 1.0f / (1.0f + ex);
            float sel = a.bias ? sg + a.bias[e] : sg;
            double sl = 2.0 * (double)ulp_of(sg) + (double)ulp_of(sel);
            sh.sg[e] = sg;
            sh.lo[e] = (double)sel - sl;
            sh.hi[e] = (double)sel + sl;
        }
    } else {
        for (int e = threadIdx.x; e < E; e += 256) {
            sh.lo[e] = cen[e] - bnd[e];
            sh.hi[e] = cen[e] + bnd[e];
            if (bnd[e] > 0.0) sh.width = 1;
        }
    }
    __syncthreads();
    zz_mark_contested(sh, E, K);
    // exact logits (zero-width intervals) can only "overlap" by being equal, which
    // the index tie-break below resolves as the reference does
    if (threadIdx.x == 0 && !sh.width) sh.any = 0;
    __syncthreads();

    if (sh.any && a.gating == ZZ_GATE_SOFTMAX_PES) {
        // stage 2: tight bounds for the contested experts, one wave each
        const float *xn = a.xn + (size_t)s * a.D;
        for (int k = threadIdx.x >> 6; k < sh.nlist; k += 4) {
            int e = sh.list[k];
            double lo = 0, hi = 0;
            zz_refine_wave(a.router + (size_t)e * a.D, xn, a.D, a.bias, e, &lo, &hi);
            if ((threadIdx.x & 63) == 0) {      // both intervals hold v_ref
                sh.lo[e] = fmax(sh.lo[e], lo);
                sh.hi[e] = fmin(sh.hi[e], hi);
            }
        }
        __syncthreads();
        zz_mark_contested(sh, E, K);
        if (sh.any) {
            // stage 3: replay the reference's in-order fp32 chain (gemma4.c:600-601).
            // The wave forms the rounded products in LDS, one lane adds them in order.
            const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
            if (a.D <= 4096 && wv < 2) {
                for (int k = wv; k < sh.nlist; k += 2) {
                    const int e = sh.list[k];
                    const float *w = a.router + (size_t)e * a.D;
                    float *pr = sh.prod[wv];
                    for (int i = l; i < a.D; i += 64) pr[i] = w[i] * xn[i];
                    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    if (l == 0) {
                        float v = 0.0f;
                        for (int i = 0; i < a.D; i += 4) {
                            const float4 p = *(const float4 *)(pr + i);
                            v = v + p.x;
                            v = v + p.y;
                            v = v + p.z;
                            v = v + p.w;
                        }
                        if (a.bias) v = v + a.bias[e];
                        sh.lo[e] = sh.hi[e] = (double)v;
                    }
                    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                }
            } else if (a.D > 4096) {
                for (int k = threadIdx.x; k < sh.nlist; k += 256) {
                    const int e = sh.list[k];
                    const float *w = a.router + (size_t)e * a.D;
                    float v = 0.0f;
                    for (int i = 0; i < a.D; i++) v = v + w[i] * xn[i];
                    if (a.bias) v = v + a.bias[e];
                    sh.lo[e] = sh.hi[e] = (double)v;
                }
            }
            if (threadIdx.x == 0) atomicAdd(a.diag + 2, 1u);
            __syncthreads();
            zz_mark_contested(sh, E, K);       // recomputes the candidate set
            // exact values may tie: ordering below breaks ties by index, as the
            // reference's strict '>' insertion does
        }
    } else if (sh.any && a.gating == ZZ_GATE_SIGMOID_BIAS) {
        contested = 1;
    }

    // rank candidates by (centre desc, index asc); centres of disjoint intervals
    // order exactly as the reference's values do
    for (int e = threadIdx.x; e < E; e += 256) {
        if (!sh.cand[e]) continue;
        double me = 0.5 * (sh.lo[e] + sh.hi[e]);
        int rank = 0;
#pragma unroll 8
        for (int f = 0; f < E; f++) {
            if (!sh.cand[f] || f == e) continue;
            double mf = 0.5 * (sh.lo[f] + sh.hi[f]);
            rank += (mf > me) || (mf == me && f < e);
        }
        if (rank < K) {
            sh.idx[rank] = e;
            sh.topv[rank] = (float)me;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int *idx = a.eidx + (size_t)s * K;
        float *wt = a.ewt + (size_t)s * K;
        if (a.gating == ZZ_GATE_SOFTMAX_PES) {               // gemma4.c:609-612
            float sum = 0.0f, mx = sh.topv[0], w[ZZ_MAXK];
            for (int j = 0; j < K; j++) { w[j] = expf(sh.topv[j] - mx); sum += w[j]; }
            for (int j = 0; j < K; j++) { idx[j] = sh.idx[j]; wt[j] = (w[j] / sum) * a.pes[sh.idx[j]]; }
        } else if (a.gating == ZZ_GATE_SIGMOID_BIAS) {       // lfm25.c:661-667
            float sum = 0.0f, w[ZZ_MAXK];
            for (int j = 0; j < K; j++) { w[j] = sh.sg[sh.idx[j]]; sum += w[j]; }
            for (int j = 0; j < K; j++) {
                float v = w[j];
                if (a.norm_topk) v /= (sum + 1e-6f);
                idx[j] = sh.idx[j];
                wt[j] = v * a.routed_scaling;
            }
            if (a.contested) a.contested[s] = contested;
            if (contested) atomicAdd(a.diag + 3, 1u);
        } else {                                             // maple.c:596-600
            float sum = 0.0f, mx = sh.topv[0], w[ZZ_MAXK];
            for (int j = 0; j < K; j++) { w[j] = expf(sh.topv[j] - mx); sum += w[j]; }
            for (int j = 0; j < K; j++) {
                float v = w[j];
                if (a.norm_topk) v /= (sum + 1e-20f);
                idx[j] = sh.idx[j];
                wt[j] = v;
            }
        }
        if (a.topv) for (int j = 0; j < K; j++) a.topv[(size_t)s * K + j] = sh.topv[j];
    }
}

