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
// doubles of LDS; RB >= R is the compile-time run capacity. Thread 0 writes
// *cen / *bnd. Ends with a barrier (buf and red may be reused).
__device__ __forceinline__ int zz_pad32(int i) { return i + (i >> 5); }

template <int RB>
__device__ void zz_tight_block_scan(const float *buf, int D, const float *bias, int e, double *red,
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
            if (a.gating == ZZ_GATE_GROUPED) {   // ling.c:722-727: 8 accumulators, D % 8 == 0
                double q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int i = 0; i < D; i += 8)
                    for (int k = 0; k < 8; k++) q[k] += (double)w[i + k] * (double)xv[i + k];
                r = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
            } else {
                for (int i = 0; i < D; i++) r += (double)w[i] * (double)xv[i];
            }
            v = (float)r;
            atomicAdd(a.diag + 1, 1u);
        }
        a.cen[o] = (double)v;                    // exact float logit
        a.bnd[o] = 0.0;
    }
}
