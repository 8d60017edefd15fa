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
// Router logits, one wave per (token, expert).
//
// Gemma: the reference adds t_i = fl(w_i * xn_i) in order in fp32 (gemma4.c:600-601).
// The wave forms the same rounded products and their exact-order prefix sums S_k
// in double, which bounds the reference's chain tightly:
//   |v_ref - S_D| <= u/(1-u) (sum_{k>=2} |S_k| + (D-1) g_D T),  T = sum |t_i|
// (each rounding of the chain is at most u times its partial sum). Products are
// loaded coalesced, 32 per lane, and transposed through LDS so each lane owns a
// contiguous run of the order; a wave scan joins the runs.
// lfm/maple: products are exact in double; the parallel double sum is certified
// to round to the same float as the reference's serial double sum, else replayed
// serially.
#define ZZ_TPER 32                           // elements per lane per chunk
#define ZZ_TBUF (64 * (ZZ_TPER + 1))         // floats of one wave's transpose buffer

__device__ __forceinline__ void zz_wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Centre and bound of a gemma logit from the exact-order prefix data; bias is the
// harness's Zipf offset, v' = fl(v + bias_e).
__device__ __forceinline__ void zz_tight_finish(double sabs, double T, double tot, int D,
                                                const float *bias, int e, double *cen_out,
                                                double *bnd_out) {
    const double gd = zz_gamma(D, ZZ_U64);
    // double-precision slack on every computed prefix (|S_k err| <= g_D^d T)
    double b = ZZ_U32 / (1.0 - ZZ_U32) *
               (sabs + (double)D * gd * T + (double)(D - 1) * zz_gamma(D, ZZ_U32) * T);
    b = b * 1.000001 + gd * T + 1e-40;
    double cen = tot;
    if (bias) {
        cen += (double)bias[e];
        b += 2.0 * ZZ_U32 * (fabs(cen) + b) + 1e-40;
    }
    *cen_out = cen;
    *bnd_out = b;
}

// Gemma logits of NS tokens against one router row, each with its tight bound,
// by one wave. ONFLY: the router input is formed as (x_s * rr[s]) * (rscale * rs),
// the prep kernel's expression, from the raw rows x_s = src + s*D (and written to
// xn_out when that is not null); otherwise src holds the router inputs xn_s.
// The router row is loaded once per chunk for all tokens. buf: ZZ_TBUF floats of
// LDS owned by this wave. Lane 0 writes cen/bnd[s * cstride].
template <int NS, bool ONFLY>
__device__ void zz_tight_wave(const float *w, const float *src, const float *rscale, const float *rr,
                              float rs, int D, const float *bias, int e, float *buf, double *cen,
                              double *bnd, int cstride, float *xn_out) {
    const int l = threadIdx.x & 63;
    double carry[NS], sabs[NS], T[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) carry[s] = sabs[s] = T[s] = 0.0;
    for (int c0 = 0; c0 < D; c0 += 64 * ZZ_TPER) {
        // element c0 + 64j + l; past D the (clamped, in-range) load is discarded
        float wv[ZZ_TPER], sc[ZZ_TPER];
#pragma unroll
        for (int j = 0; j < ZZ_TPER; j++) {
            const int i = min(c0 + 64 * j + l, D - 1);
            wv[j] = w[i];
            if (ONFLY) sc[j] = rscale[i] * rs;
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float *xs = src + (size_t)s * D;
#pragma unroll
            for (int j = 0; j < ZZ_TPER; j++) {
                const int i = min(c0 + 64 * j + l, D - 1);
                const float xv = ONFLY ? (xs[i] * rr[s]) * sc[j] : xs[i];
                if (ONFLY && xn_out && c0 + 64 * j + l < D) xn_out[(size_t)s * D + i] = xv;
                // transposed: lane o = q >> 5 owns elements c0 + 32 o .. +31
                const int q = 64 * j + l;
                buf[(q >> 5) * (ZZ_TPER + 1) + (q & 31)] = wv[j] * xv;
            }
            zz_wave_sync_lds();
            float p[ZZ_TPER];
            double loc = 0.0;
            const int i0 = c0 + l * ZZ_TPER;
#pragma unroll
            for (int k = 0; k < ZZ_TPER; k++) {
                p[k] = i0 + k < D ? buf[l * (ZZ_TPER + 1) + k] : 0.0f;
                loc += (double)p[k];
                T[s] += fabs((double)p[k]);
            }
            double inc = loc;                                 // inclusive scan of lane runs
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const double v = __shfl_up(inc, o, 64);
                if (l >= o) inc += v;
            }
            double run = carry[s] + (inc - loc);
#pragma unroll
            for (int k = 0; k < ZZ_TPER; k++) {
                run += (double)p[k];
                if (i0 + k >= 1 && i0 + k < D) sabs[s] += fabs(run);
            }
            carry[s] += __shfl(inc, 63, 64);
            zz_wave_sync_lds();                               // buf is rewritten next
        }
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const double sa = zz_wave_sum(sabs[s]), t = zz_wave_sum(T[s]);
        if (l == 0) zz_tight_finish(sa, t, carry[s], D, bias, e, cen + (size_t)s * cstride,
                                    bnd + (size_t)s * cstride);
    }
}

// Tight bound of one gemma logit by a whole 256-thread workgroup (decode
// batches), from the D rounded products t_i staged in LDS at buf[zz_pad32(i)] (one
// pad word per 32 against bank conflicts): each thread owns a contiguous run of
// R = ceil(D/256) elements of the order, a block scan joins the runs. red: 12
// doubles of LDS. Thread 0 writes *cen / *bnd. Ends with a barrier (buf and red
// may be reused).
__device__ __forceinline__ int zz_pad32(int i) { return i + (i >> 5); }

__device__ void zz_tight_block_scan(const float *buf, int D, const float *bias, int e, double *red,
                                    double *cen, double *bnd) {
    const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
    const int R = (D + 255) >> 8;                             // <= 32 for D <= 8192
    const int i0 = tid * R;
    float p[32];
    double loc = 0.0, T = 0.0;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        p[k] = k < R && i0 + k < D ? buf[zz_pad32(i0 + k)] : 0.0f;
        loc += (double)p[k];
        T += fabs((double)p[k]);
    }
    double inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double v = __shfl_up(inc, o, 64);
        if (l >= o) inc += v;
    }
    if (l == 63) red[wv] = inc;
    __syncthreads();
    double run = inc - loc, sabs = 0.0;
    for (int q = 0; q < wv; q++) run += red[q];
#pragma unroll
    for (int k = 0; k < 32; k++) {
        run += (double)p[k];
        if (k < R && i0 + k >= 1 && i0 + k < D) sabs += fabs(run);
    }
    sabs = zz_wave_sum(sabs);
    T = zz_wave_sum(T);
    if (l == 0) {
        red[4 + wv] = sabs;
        red[8 + wv] = T;
    }
    __syncthreads();
    if (tid == 0) {
        const double tot = ((red[0] + red[1]) + red[2]) + red[3];
        zz_tight_finish(((red[4] + red[5]) + red[6]) + red[7], ((red[8] + red[9]) + red[10]) + red[11],
                        tot, D, bias, e, cen, bnd);
    }
    __syncthreads();
}

// lfm / maple logit of token s, expert e (router input x), by one wave.
__device__ void zz_logit_wave_f64(const ZzLogitArgs &a, int s, int e) {
    const int l = threadIdx.x & 63;
    const int D = a.D;
    const float *w = a.router + (size_t)e * D;
    const float *xv = a.x + (size_t)s * D;
    const size_t o = (size_t)s * a.E + e;
    double c = 0.0, t = 0.0;
    for (int c0 = 0; c0 < D; c0 += 64 * 16) {
        float wr[16], xr[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {                        // clamped: loads stay in range
            const int i = min(c0 + 64 * j + l, D - 1);
            wr[j] = w[i];
            xr[j] = xv[i];
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (c0 + 64 * j + l < D) {
                const double p = (double)wr[j] * (double)xr[j];
                c += p;
                t += fabs(p);
            }
        }
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

// -------------------------------------------------------------------------------
// Top-k with interval certification. Each expert carries [lo, hi] containing the
// reference's selection score. Candidates are experts whose hi reaches the k-th
// largest lo; a candidate is contested when its interval meets another
// candidate's. No contested candidate => the reference's top-k set and order are
// fixed by the centres. Contested gemma experts are refined (exact prefix-sum
// bound), then replayed serially; contested lfm scores (glibc expf in the
// reference, lfm25.c:648) are flagged for the caller.
struct ZzTopkShared {
    __attribute__((aligned(16))) double lo[ZZ_MAXE + 8], hi[ZZ_MAXE + 8];
    int clist[ZZ_MAXE];                  // candidates (any order)
    int ncand;
    float sg[ZZ_MAXE];
    int list[ZZ_MAXE];                   // contested candidates (any order)
    int nlist;
    int any;
    int width;                           // some interval has non-zero width
    double lk;
    int idx[ZZ_MAXK];
    float topv[ZZ_MAXK];
    float wj[ZZ_MAXK], pj[ZZ_MAXK], wsum;   // gate weights before normalisation
    double red[4];
    __attribute__((aligned(16))) float buf[4 * ZZ_TBUF];   // per-wave transposes; chain replay
};

// Candidates are the experts whose hi reaches lk, the k-th largest lo (ties by
// index); a candidate is contested when its interval meets another candidate's.
// The all-pairs pass for lk reads the lo table 8 entries at a time as broadcast
// LDS loads; the candidate passes run over the (short) candidate list.
__device__ void zz_mark_contested(ZzTopkShared &sh, int E, int K) {
    if (threadIdx.x == 0) {
        sh.lk = -INFINITY;
        sh.ncand = 0;
        sh.nlist = 0;
        sh.any = 0;
    }
    __syncthreads();
    // T adjacent threads share expert e, each ranking it against a slice of lo
    const int T = E <= 32 ? 8 : (E <= 64 ? 4 : (E <= 128 ? 2 : 1));
    const int per = (E + T - 1) / T;
    for (int base = 0; base < E * T; base += 256) {
        const int v = base + threadIdx.x, e = v / T, h = v % T;
        const bool act = e < E;
        const double le = act ? sh.lo[e] : 0.0;
        int rank = 0;
        const int f1 = act ? min(E, (h + 1) * per) : 0;
        for (int f0 = h * per; f0 < f1; f0 += 8) {
            double lf[8];                        // lo has 8 spare entries past ZZ_MAXE
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const double2 w = *(const double2 *)&sh.lo[(f0 & ~1) + j];
                lf[j] = w.x;
                lf[j + 1] = w.y;
            }
            const int fb = f0 & ~1;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int f = fb + j;
                rank += (f >= f0) & (f < f1) & ((lf[j] > le) | ((lf[j] == le) & (f < e)));
            }
        }
        // T is a power of two and the T threads of e are adjacent lanes of one wave
        for (int o = 1; o < T; o <<= 1) rank += __shfl_xor(rank, o, 64);
        if (act && h == 0 && rank == K - 1) sh.lk = le;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256)
        if (sh.hi[e] >= sh.lk) sh.clist[atomicAdd(&sh.ncand, 1)] = e;
    __syncthreads();
    const int nc = sh.ncand;
    for (int i = threadIdx.x; i < nc; i += 256) {
        const int e = sh.clist[i];
        const double le = sh.lo[e], he = sh.hi[e];
        int c = 0;
        for (int j = 0; j < nc; j++) {
            const int f = sh.clist[j];
            c |= (f != e) & (sh.lo[f] <= he) & (le <= sh.hi[f]);
        }
        if (c) {
            sh.any = 1;
            sh.list[atomicAdd(&sh.nlist, 1)] = e;
        }
    }
    __syncthreads();
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
        // every gemma logit already carries its tight bound (zz_tight_wave); what
        // is still contested is settled by replaying the reference's chain
        const float *xn = a.xn + (size_t)s * a.D;
        {
            // replay the reference's in-order fp32 chain (gemma4.c:600-601). The
            // wave forms the rounded products in LDS, one lane adds them in order.
            const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
            if (a.D <= 2 * ZZ_TBUF && wv < 2) {
                for (int k = wv; k < sh.nlist; k += 2) {
                    const int e = sh.list[k];
                    const float *w = a.router + (size_t)e * a.D;
                    float *pr = sh.buf + wv * 2 * ZZ_TBUF;
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
            } else if (a.D > 2 * ZZ_TBUF) {
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
    const int nc = sh.ncand;
    for (int i = threadIdx.x; i < nc; i += 256) {
        const int e = sh.clist[i];
        const double me = 0.5 * (sh.lo[e] + sh.hi[e]);
        int rank = 0;
        for (int j = 0; j < nc; j++) {
            const int f = sh.clist[j];
            const double mf = 0.5 * (sh.lo[f] + sh.hi[f]);
            rank += (f != e) & ((mf > me) | ((mf == me) & (f < e)));
        }
        if (rank < K) {
            sh.idx[rank] = e;
            sh.topv[rank] = (float)me;
        }
    }
    __syncthreads();
    // gate weights: each slot's w_j in parallel, their sum serially in slot order
    // as the reference adds them, then each slot's normalisation
    const int j = threadIdx.x;
    if (j < K) {
        const int e = sh.idx[j];
        sh.wj[j] = a.gating == ZZ_GATE_SIGMOID_BIAS ? sh.sg[e] : expf(sh.topv[j] - sh.topv[0]);
        sh.pj[j] = a.gating == ZZ_GATE_SOFTMAX_PES ? a.pes[e] : 1.0f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (int i = 0; i < K; i++) sum += sh.wj[i];
        sh.wsum = sum;
        if (a.gating == ZZ_GATE_SIGMOID_BIAS) {
            if (a.contested) a.contested[s] = contested;
            if (contested) atomicAdd(a.diag + 3, 1u);
        }
    }
    __syncthreads();
    if (j < K) {
        const float sum = sh.wsum, v = sh.wj[j];
        float out;
        if (a.gating == ZZ_GATE_SOFTMAX_PES) {                     // gemma4.c:609-612
            out = (v / sum) * sh.pj[j];
        } else if (a.gating == ZZ_GATE_SIGMOID_BIAS) {             // lfm25.c:661-667
            float t = v;
            if (a.norm_topk) t /= (sum + 1e-6f);
            out = t * a.routed_scaling;
        } else {                                                   // maple.c:596-600
            float t = v;
            if (a.norm_topk) t /= (sum + 1e-20f);
            out = t;
        }
        a.eidx[(size_t)s * K + j] = sh.idx[j];
        a.ewt[(size_t)s * K + j] = out;
        if (a.topv) a.topv[(size_t)s * K + j] = sh.topv[j];
    }
}

