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

// Centre and bound of a gemma logit from the exact-order prefix data; with hb, bz is
// the harness's Zipf offset bias_e (read by the caller when its loads are issued),
// v' = fl(v + bias_e).
__device__ __forceinline__ void zz_tight_finish(double sabs, double T, double tot, int D,
                                                bool hb, float bz, double *cen_out,
                                                double *bnd_out) {
    const double gd = zz_gamma(D, ZZ_U64);
    // double-precision slack on every computed prefix (|S_k err| <= g_D^d T)
    double b = ZZ_U32 / (1.0 - ZZ_U32) *
               (sabs + (double)D * gd * T + (double)(D - 1) * zz_gamma(D, ZZ_U32) * T);
    b = b * 1.000001 + gd * T + 1e-40;
    double cen = tot;
    if (hb) {
        cen += (double)bz;
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
    const float bz = bias ? bias[e] : 0.0f;
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
            const double inc = zz_wave_incl_scan_add(loc);    // inclusive scan of lane runs
            double run = carry[s] + (inc - loc);
#pragma unroll
            for (int k = 0; k < ZZ_TPER; k++) {
                run += (double)p[k];
                if (i0 + k >= 1 && i0 + k < D) sabs[s] += fabs(run);
            }
            carry[s] += zz_lane_f64(inc, 63);
            zz_wave_sync_lds();                               // buf is rewritten next
        }
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const double sa = zz_wave_sum(sabs[s]), t = zz_wave_sum(T[s]);
        if (l == 0) zz_tight_finish(sa, t, carry[s], D, bias != nullptr, bz, cen + (size_t)s * cstride,
                                    bnd + (size_t)s * cstride);
    }
}

// Tight bound of one gemma logit by a whole 256-thread workgroup (decode
// batches), from the D rounded products t_i staged in LDS at buf[zz_pad32(i)] (one
// pad word per 32 against bank conflicts): each thread owns a contiguous run of
// R = ceil(D/256) elements of the order, a block scan joins the runs. red: 12
// doubles of LDS; RB >= R is the compile-time run capacity. Thread 0 writes
// *cen / *bnd. Ends with a barrier (buf and red may be reused).
__device__ __forceinline__ int zz_pad32(int i) { return i + (i >> 5); }

template <int RB>
__device__ void zz_tight_block_scan(const float *buf, int D, bool hb, float bz, double *red,
                                    double *cen, double *bnd) {
    const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
    const int R = (D + 255) >> 8;                             // R <= RB
    const int i0 = tid * R;
    float p[RB];
    double loc = 0.0, T = 0.0;
#pragma unroll
    for (int k = 0; k < RB; k++) p[k] = buf[zz_pad32(min(i0 + k, D - 1))];   // all reads issued first
#pragma unroll
    for (int k = 0; k < RB; k++) {
        if (!(k < R && i0 + k < D)) p[k] = 0.0f;
        loc += (double)p[k];
        T += fabs((double)p[k]);
    }
    const double inc = zz_wave_incl_scan_add(loc);
    if (l == 63) red[wv] = inc;
    __syncthreads();
    double run = inc - loc, sabs = 0.0;
    for (int q = 0; q < wv; q++) run += red[q];
#pragma unroll
    for (int k = 0; k < RB; k++) {
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
                        tot, D, hb, bz, cen, bnd);
    }
    __syncthreads();
}

// -------------------------------------------------------------------------------
// lfm / maple / ling logits. The reference sums the exact double products
// p_i = (double)w_i * (double)x_i in order: one double chain (lfm25.c:650-653;
// maple.c:744 through w_dot_f32, maple.c:400-410) or eight chains by i % 8 combined
// pairwise (ling.c:722-727); the logit is the float of that sum. The first addition
// (0 + p_0) is exact and each later one errs by at most u |v_i|, so the chain's sum
// lies within u (1+u)^D sum_{i>=1} |S_i| of the exact prefix-sum end S_D. The wave
// forms the products once, transposes them through LDS so that each lane owns a
// contiguous run of the order, and joins the runs by a wave scan: that gives the
// prefix sums S_i (to gamma_40 T, T = sum |p_i|) and the centre S_D (to gamma_30 T).
// When every value the bound allows rounds to one float, that float is the
// reference's logit; otherwise one lane replays the chain from the products staged
// in LDS, chunk by chunk.
#define ZZ_DPER 16                           // products per lane per chunk
#define ZZ_DBUF (64 * (ZZ_DPER + 1))         // doubles of one wave's product buffer

// The exact products of elements c0 .. c0 + 64*ZZ_DPER - 1 into the wave's buffer,
// element c0 + q at tb[(q / ZZ_DPER) * (ZZ_DPER + 1) + q % ZZ_DPER] (0 past D).
// Loads are coalesced (element c0 + 64 j + l on lane l). Ends synchronised.
__device__ __forceinline__ void zz_stage_products(const float *w, const float *x, int D, int c0, double *tb) {
    const int l = threadIdx.x & 63;
    float wv[ZZ_DPER], xr[ZZ_DPER];
#pragma unroll
    for (int j = 0; j < ZZ_DPER; j++) {                   // clamped: loads stay in range
        const int i = min(c0 + 64 * j + l, D - 1);
        wv[j] = w[i];
        xr[j] = x[i];
    }
#pragma unroll
    for (int j = 0; j < ZZ_DPER; j++) {
        const int q = 64 * j + l;
        tb[(q / ZZ_DPER) * (ZZ_DPER + 1) + q % ZZ_DPER] =
            c0 + q < D ? (double)wv[j] * (double)xr[j] : 0.0;
    }
    zz_wave_sync_lds();
}

// logit of token s, expert e (router input x), by one wave; tb: ZZ_DBUF doubles of
// LDS owned by this wave. Lane 0 writes cen (the exact float logit) and bnd = 0.
__device__ void zz_logit_wave_f64(const ZzLogitArgs &a, int s, int e, double *tb) {
    const int l = threadIdx.x & 63, D = a.D;
    const float *w = a.router + (size_t)e * D, *xv = a.x + (size_t)s * D;
    const size_t o = (size_t)s * a.E + e;
    const bool grp = a.gating == ZZ_GATE_GROUPED;
    double carry = 0.0, sabs = 0.0, T = 0.0;
    for (int c0 = 0; c0 < D; c0 += 64 * ZZ_DPER) {
        zz_stage_products(w, xv, D, c0, tb);
        const int i0 = c0 + l * ZZ_DPER;
        double p[ZZ_DPER], loc = 0.0;
#pragma unroll
        for (int k = 0; k < ZZ_DPER; k++) {
            p[k] = tb[l * (ZZ_DPER + 1) + k];
            loc += p[k];
            T += fabs(p[k]);
        }
        const double inc = zz_wave_incl_scan_add(loc);     // inclusive scan of the runs
        if (!grp) {
            double run = carry + (inc - loc);
#pragma unroll
            for (int k = 0; k < ZZ_DPER; k++) {
                run += p[k];
                if (i0 + k >= 1 && i0 + k < D) sabs += fabs(run);
            }
        }
        carry += zz_lane_f64(inc, 63);
        zz_wave_sync_lds();                                // tb is rewritten next
    }
    sabs = zz_wave_sum(sabs);
    T = zz_wave_sum(T);
    // the centre's own error: runs of ZZ_DPER, 6 scan levels, one add per chunk
    const double gc = zz_gamma(ZZ_DPER + 6 + (D + 64 * ZZ_DPER - 1) / (64 * ZZ_DPER) + 2, ZZ_U64) * T;
    double b;
    if (grp) {
        // eight chains of D/8 terms, each within gamma_{D/8} of its exact sum, then
        // three levels of pairwise adds: within gamma_{D/8 + 3} T in all
        b = zz_gamma(D / 8 + 3, ZZ_U64) * T + gc;
    } else {
        // the prefix sums' slack: each S_i within gamma_{D + 40} T (far more than the
        // run, scan and carry depth)
        b = ZZ_U64 * (1.0 + zz_gamma(D + 2, ZZ_U64)) * (sabs + (double)D * zz_gamma(D + 40, ZZ_U64) * T) + gc;
    }
    b = b * 1.000001 + 1e-300;
    const float lo = (float)(carry - b), hi = (float)(carry + b);
    float v = lo;
    if (__builtin_amdgcn_readfirstlane(lo != hi)) {
        // replay, reference order, from the products staged chunk by chunk
        double r = 0.0, q0 = 0.0, q1 = 0.0, q2 = 0.0, q3 = 0.0, q4 = 0.0, q5 = 0.0, q6 = 0.0, q7 = 0.0;
        for (int c0 = 0; c0 < D; c0 += 64 * ZZ_DPER) {
            zz_stage_products(w, xv, D, c0, tb);
            if (l == 0) {
                const int n = min(64 * ZZ_DPER, D - c0);
                if (grp) {                                 // D % 8 == 0, c0 % 8 == 0
                    for (int i = 0; i < n; i += 8) {
                        const double *t = tb + (i / ZZ_DPER) * (ZZ_DPER + 1) + i % ZZ_DPER;
                        q0 += t[0]; q1 += t[1]; q2 += t[2]; q3 += t[3];
                        q4 += t[4]; q5 += t[5]; q6 += t[6]; q7 += t[7];
                    }
                } else {
                    for (int i = 0; i < n; i += ZZ_DPER) {
                        const double *t = tb + (i / ZZ_DPER) * (ZZ_DPER + 1);
                        const int m = min(ZZ_DPER, n - i);
#pragma unroll
                        for (int k = 0; k < ZZ_DPER; k++)
                            if (k < m) r += t[k];
                    }
                }
            }
            zz_wave_sync_lds();
        }
        if (grp) r = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7));
        v = (float)r;
        if (l == 0) atomicAdd(a.diag + 1, 1u);
    }
    if (l == 0) {
        a.cen[o] = (double)v;                    // exact float logit
        a.bnd[o] = 0.0;
    }
}
