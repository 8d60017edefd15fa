// zz_route.hip -- MoE front half on gfx950: input norms + int8 activation
// quantisation, router logits, certified top-k gating, and the batch-union
// dispatch (histogram / prefix / stable scatter as one LDS sort).
//
// Exactness strategy. The reference computes its routing decisions with serial
// CPU arithmetic (an in-order fp32 sum for gemma4.c:600-601, serial double sums
// for lfm25.c:646-647 and maple.c:400-410, a serial double sum of squares in
// rmsnorm gemma4.c:425-428). A GPU reduces in parallel, so it cannot replay those
// roundings cheaply. Instead each value is computed in parallel together with a
// rigorous bound on its distance from the reference's serial result; a decision
// (a rounding to float, the top-k set and order) is taken on the GPU only when
// the bound proves it equals the reference's. Otherwise the few contested values
// are recomputed: first with a tighter bound from exact prefix sums, and as a last
// resort by replaying the reference's serial chain in the reference's order.
#include "zz_common.h"
#include "zz_kernels.h"
#include <float.h>

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

// The float (float)(s/D) that the reference's serial double sum of squares would
// produce, certified from a parallel sum; falls back to the serial replay when
// the bound straddles a rounding boundary (gemma4.c:425-428).
__device__ float zz_certified_meansq(const float *x, int D, double *red, unsigned *fallbacks) {
    double s = 0.0;
    for (int i = threadIdx.x; i < D; i += 256) s += (double)x[i] * (double)x[i];
    s = zz_block_sum(s, red);
    // each term took part in at most D/256 + 8 roundings on the GPU, D-1 in the
    // reference; all terms are non-negative so sum|terms| = the exact sum <= s/(1-g)
    double m = (double)((D + 255) / 256 + 8);
    double g = zz_gamma(D, ZZ_U64) + zz_gamma(m, ZZ_U64);
    double b = g * s / (1.0 - zz_gamma(m, ZZ_U64)) * 1.0000001 + 1e-300;
    float lo = (float)((s - b) / (double)D), hi = (float)((s + b) / (double)D);
    __shared__ float cert;
    __syncthreads();
    if (threadIdx.x == 0) {
        if (lo == hi) {
            cert = lo;
        } else {
            double t = 0.0;                    // serial replay, reference order
            for (int i = 0; i < D; i++) t += (double)x[i] * (double)x[i];
            cert = (float)(t / (double)D);
            atomicAdd(fallbacks, 1u);
        }
    }
    __syncthreads();
    return cert;
}

// -------------------------------------------------------------------------------
// Prep: one workgroup per token. Gemma: router input xn = rmsnorm(x)*scale*D^-1/2
// (gemma4.c:591-593) and expert input X = rmsnorm(x, pre_ffn_ln2) (763-764), both
// from the same certified mean square. Then X is quantised q8_0-style per 32-block
// (q40.h:124-138) with per-block integer sums, and for tq2 the Sx total
// (tq2.h:98-108) is summed serially in the reference's order.
__global__ __launch_bounds__(256) void zz_prep_kernel(ZzPrepArgs a) {
    const int s = blockIdx.x, D = a.D;
    const float *x = a.in + (size_t)s * D;
    __shared__ double red[4];
    __shared__ float xs_l[ZZ_MAXD / ZZ_BLK];
    __shared__ int xsum_l[ZZ_MAXD / ZZ_BLK];
    float r = 1.0f;
    if (a.gemma) {
        float ms = zz_certified_meansq(x, D, red, a.diag + 0);
        r = 1.0f / sqrtf(ms + a.eps);
        float rs = 1.0f / sqrtf((float)D);
        for (int i = threadIdx.x; i < D; i += 256)
            a.xn[(size_t)s * D + i] = (x[i] * r) * (a.router_scale[i] * rs);
    }
    // quantise: each wave takes two 32-blocks per step, one value per lane
    const int nb = D / ZZ_BLK, w = threadIdx.x >> 6, l = threadIdx.x & 63;
    for (int b0 = 2 * w; b0 < nb; b0 += 8) {
        int b = b0 + (l >> 5), j = l & 31;
        float v = 0.0f;
        if (b < nb) {
            v = x[b * ZZ_BLK + j];
            if (a.gemma) v = (v * r) * a.pre_ln[b * ZZ_BLK + j];
        }
        float d;
        int q = zz_quant_lane(v, &d);
        int qs = q;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) qs += __shfl_xor(qs, o, 64);
        if (b < nb) {
            a.xq[(size_t)s * D + b * ZZ_BLK + j] = (int8_t)q;
            if (j == 0) {
                a.xs[(size_t)s * nb + b] = d;
                a.xsum[(size_t)s * nb + b] = qs;
                xs_l[b] = d;
                xsum_l[b] = qs;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && a.xt) {
        double tot = 0.0;                          // tq2.h:101-106, serial
        for (int b = 0; b < nb; b++) tot += (double)xs_l[b] * (double)xsum_l[b];
        a.xt[s] = (float)tot;
    }
}

// -------------------------------------------------------------------------------
// Router logits: one wave per (token, expert). Lane l takes elements l, l+64, ...
// Gemma: t_i = fl(w_i * xn_i) exactly as the reference rounds them, summed in fp32
// per lane and across the wave; the bound covers both this sum and the
// reference's in-order fp32 chain: |v_ref - c| <= (g_{D-1} + g_m) * sum|t_i|.
// lfm/maple: products are exact in double; the double sum is certified to round
// to the same float as the reference's serial double sum, else replayed serially.
__global__ __launch_bounds__(256) void zz_logits_kernel(ZzLogitArgs a) {
    const int s = blockIdx.y, e = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (e >= a.E) return;
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
    double lk;
    int idx[ZZ_MAXK];
    float topv[ZZ_MAXK];
    double red[4];
};

__device__ void zz_mark_contested(ZzTopkShared &sh, int E, int K) {
    // k-th largest lo (ties broken by index)
    for (int e = threadIdx.x; e < E; e += 256) {
        int rank = 0;
        double le = sh.lo[e];
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

__global__ __launch_bounds__(256) void zz_topk_kernel(ZzTopkArgs a) {
    const int s = blockIdx.x, E = a.E, K = a.K;
    __shared__ ZzTopkShared sh;
    const double *cen = a.cen + (size_t)s * E, *bnd = a.bnd + (size_t)s * E;
    int contested = 0;
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
        }
    }
    __syncthreads();
    zz_mark_contested(sh, E, K);

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
            // stage 3: replay the reference's in-order fp32 chain (gemma4.c:600-601)
            for (int k = threadIdx.x; k < sh.nlist; k += 256) {
                int e = sh.list[k];
                const float *w = a.router + (size_t)e * a.D;
                float v = 0.0f;
                for (int i = 0; i < a.D; i++) v = v + w[i] * xn[i];
                if (a.bias) v = v + a.bias[e];
                sh.lo[e] = sh.hi[e] = (double)v;
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

// -------------------------------------------------------------------------------
// Dispatch, one workgroup of 1024 threads. Keys (expert << 14 | flat pair index)
// are bitonic-sorted in LDS: runs of equal expert are that expert's token list in
// ascending token order -- exactly the rows[] of gemma4.c:779-786. The first key
// of each run gives the expert's first-seen position, whose order is the union
// order of gemma4.c:756-761. Also emits the FFN work list: per expert in union
// order, chunks of at most `tch` pairs.
__global__ __launch_bounds__(1024) void zz_dispatch_kernel(ZzDispatchArgs a) {
    extern __shared__ int keys[];
    __shared__ int first[ZZ_MAXE], start[ZZ_MAXE], cnt[ZZ_MAXE], order[ZZ_MAXE];
    __shared__ int nu_s;
    const int P = a.P, E = a.E;
    int N = 1;
    while (N < P) N <<= 1;
    for (int i = threadIdx.x; i < N; i += 1024) {
        int e = i < P ? a.eidx[i] : 0;
        e = e < 0 || e >= E ? 0 : e;        // never index past the expert tables
        keys[i] = i < P ? (e << 14) | i : 0x7fffffff;
    }
    for (int e = threadIdx.x; e < E; e += 1024) { first[e] = 0x7fffffff; start[e] = 0; cnt[e] = 0; }
    __syncthreads();
    for (int k = 2; k <= N; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < N; i += 1024) {
                int ixj = i ^ j;
                if (ixj > i) {
                    int x = keys[i], y = keys[ixj];
                    bool up = (i & k) == 0;
                    if ((x > y) == up) { keys[i] = y; keys[ixj] = x; }
                }
            }
            __syncthreads();
        }
    for (int i = threadIdx.x; i < P; i += 1024) {
        int key = keys[i], e = key >> 14, p = key & 0x3fff;
        a.ptok[i] = p / a.K;
        a.pslot[i] = p % a.K;
        a.pwt[i] = a.ewt[p];
        a.ppos[p] = i;
        if (i == 0 || (keys[i - 1] >> 14) != e) { start[e] = i; first[e] = p; }
        if (i == P - 1 || (keys[i + 1] >> 14) != e) cnt[e] = i + 1;   // run end, for now
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 1024)
        if (cnt[e]) cnt[e] -= start[e];
    __syncthreads();
    // union order: rank experts present by first-seen pair index
    for (int e = threadIdx.x; e < E; e += 1024) {
        if (!cnt[e]) continue;
        int r = 0;
        for (int f = 0; f < E; f++) r += cnt[f] && first[f] < first[e];
        order[r] = e;
    }
    if (threadIdx.x == 0) {
        int nu = 0;
        for (int e = 0; e < E; e++) nu += cnt[e] != 0;
        nu_s = nu;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int nu = nu_s, nitems = 0;
        for (int u = 0; u < nu; u++) {
            int e = order[u];
            a.uniq[u] = e;
            a.uoff[u] = start[e];
            a.ucnt[u] = cnt[e];
            for (int c0 = 0; c0 < cnt[e]; c0 += a.tch) {
                a.items[nitems].e = e;
                a.items[nitems].u = u;
                a.items[nitems].p0 = start[e] + c0;
                a.items[nitems].n = min(a.tch, cnt[e] - c0);
                nitems++;
            }
        }
        a.meta[0] = nu;
        a.meta[1] = nitems;
    }
}

// ------------------------------------------------------------------ launchers
int zz_launch_prep(const ZzPrepArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_prep_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_logits(const ZzLogitArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_logits_kernel, dim3((a.E + 3) / 4, S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_topk(const ZzTopkArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_topk_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dispatch(const ZzDispatchArgs &a, hipStream_t st) {
    int N = 1;
    while (N < a.P) N <<= 1;
    hipLaunchKernelGGL(zz_dispatch_kernel, dim3(1), dim3(1024), sizeof(int) * N, st, a);
    return hipGetLastError() == hipSuccess;
}
