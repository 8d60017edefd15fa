// zz_decode.hip -- decode-sized batches (S <= 4 tokens) in three launches:
//   1. zz_dec_route_kernel: every workgroup quantises a slice of the expert input
//      and computes the certified logits of 4 experts for all tokens; the last
//      workgroup to arrive (device-scope ticket) runs the top-k gating and builds
//      the dispatch lists (gemma4.c:750-790 for a handful of rows).
//   2. the dot4 gate/up GEMV (zz_ffn.hip) over the work items.
//   3. zz_dec_down_kernel: down GEMV for all (token, slot) pairs of a row tile,
//      the gate-weighted combine in registers (gemma4.c:652) and, for gemma, the
//      post-norm (gemma4.c:807-808) finished by the last workgroup.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_route_dev.h"

#define DEC_MAXS 4

// rmsnorm factor of one row, the mean square certified as in zz_prep_kernel
__device__ float zz_row_rms(const float *x, int D, float eps, double *red, float *cert, unsigned *diag) {
    const int tid = threadIdx.x;
    double sq = 0.0;
    for (int i = 4 * tid; i < D; i += 1024) {
        const float4 v = *(const float4 *)(x + i);
        sq += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    sq = zz_block_sum(sq, red);
    const double m = (double)(D / 1024 + 12);
    const double g = zz_gamma(D, ZZ_U64) + zz_gamma(m, ZZ_U64);
    const double b = g * sq / (1.0 - zz_gamma(m, ZZ_U64)) * 1.0000001 + 1e-300;
    const float lo = (float)((sq - b) / (double)D), hi = (float)((sq + b) / (double)D);
    if (tid == 0) {
        if (lo == hi) {
            *cert = lo;
        } else {
            double t = 0.0;
            for (int i = 0; i < D; i++) t += (double)x[i] * (double)x[i];
            *cert = (float)(t / (double)D);
            atomicAdd(diag, 1u);
        }
    }
    __syncthreads();
    return 1.0f / sqrtf(*cert + eps);
}

__global__ __launch_bounds__(256) void zz_dec_route_kernel(ZzDecRouteArgs a) {
    const ZzPrepArgs &pp = a.prep;
    const int S = a.S, D = pp.D, nb = D / ZZ_BLK, tid = threadIdx.x, l = tid & 63;
    const bool gem = pp.gemma;
    __shared__ double red[4];
    __shared__ float cert;
    __shared__ float rr[DEC_MAXS];
    __shared__ int last;
    __shared__ ZzTopkShared sh;
    if (gem) {
        for (int s = 0; s < S; s++) {
            const float r = zz_row_rms(pp.in + (size_t)s * D, D, pp.eps, red, &cert, pp.diag);
            if (tid == 0) rr[s] = r;
            __syncthreads();
        }
    }
    // (a) this workgroup's slice of the expert input quantisation and of xn
    const float rs = 1.0f / sqrtf((float)D);
    for (int g = blockIdx.x * 256 + tid; g < S * nb; g += gridDim.x * 256) {
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
            for (int j = 0; j < ZZ_BLK; j++) {
                const int i = b * ZZ_BLK + j;
                pp.xn[(size_t)s * D + i] = (v[j] * r) * (pp.router_scale[i] * rs);
                v[j] = (v[j] * r) * pp.pre_ln[i];
            }
        }
        int qs;
        const float d = zz_quant_block(v, pp.xq + (size_t)s * D + b * ZZ_BLK, &qs);
        pp.xs[(size_t)s * nb + b] = d;
        pp.xsum[(size_t)s * nb + b] = qs;
    }
    // (b) logits of this workgroup's experts; xn is formed on the fly from x
    const ZzLogitArgs &lg = a.lg;
    const int e = blockIdx.x * 4 + (tid >> 6);
    if (e < lg.E) {
        const float *w = lg.router + (size_t)e * D;
        for (int s = 0; s < S; s++) {
            const size_t o = (size_t)s * lg.E + e;
            const float *x = pp.in + (size_t)s * D;
            if (gem) {
                const float r = rr[s];
                float c = 0.0f, t = 0.0f;
                for (int i = l; i < D; i += 64) {
                    const float xn = (x[i] * r) * (pp.router_scale[i] * rs);
                    const float p = w[i] * xn;
                    c += p;
                    t += fabsf(p);
                }
                c = zz_wave_sum(c);
                t = zz_wave_sum(t);
                if (l == 0) {
                    const double m = (double)((D + 63) / 64 + 6);
                    const double gm = zz_gamma(m, ZZ_U32);
                    const double T = (double)t / (1.0 - gm);
                    double b = (zz_gamma(D - 1, ZZ_U32) + gm) * T * 1.0000001 + 1e-40;
                    double cen = (double)c;
                    if (lg.bias) {
                        cen += (double)lg.bias[e];
                        b += 2.0 * ZZ_U32 * (fabs(cen) + b) + 1e-40;
                    }
                    lg.cen[o] = cen;
                    lg.bnd[o] = b;
                }
            } else {
                zz_logit_wave(lg, s, e);
            }
        }
    }
    // (c) the last workgroup to finish does the gating and the dispatch
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(a.ticket, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int s = 0; s < S; s++) {
        zz_topk_token(a.tk, s, sh);
        __syncthreads();
    }
    // dispatch of P = S*K <= 64 pairs: stable ranking by (expert, pair index)
    const ZzDispatchArgs &dp = a.dp;
    const int K = dp.K, P = S * K;
    __shared__ int pe[DEC_MAXS * ZZ_MAXK];
    __shared__ int firsts;
    if (tid < P) pe[tid] = dp.eidx[tid];
    if (tid == 0) firsts = 0;
    __syncthreads();
    if (tid < P) {
        const int ep = pe[tid];
        int rank = 0, start = 0, cnt = 0, first = 1, urank = 0;
        for (int q = 0; q < P; q++) {
            const int eq = pe[q];
            rank += eq < ep || (eq == ep && q < tid);
            start += eq < ep;
            cnt += eq == ep;
            if (q < tid && eq == ep) first = 0;
        }
        if (first)
            for (int q = 0; q < tid; q++) {
                int f = 1;
                for (int q2 = 0; q2 < q; q2++) f &= pe[q2] != pe[q];
                urank += f;
            }
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
            atomicAdd(&firsts, 1);
        }
    }
    __syncthreads();
    if (tid == 0) {
        dp.meta[0] = firsts;
        dp.meta[1] = firsts;
        *a.ticket = 0u;                            // ready for the next call
    }
}

// grid D/64: wave w owns 16 output rows; lane (row l%16, quarter l/16) takes the
// blocks b = quarter, quarter+4, ... of each (token, slot)'s down row.
__global__ __launch_bounds__(256) void zz_dec_down_kernel(ZzDecDownArgs a) {
    const ZzFfnArgs &f = a.f;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r = l & 15, q = l >> 4;
    const int g16 = blockIdx.x * 4 + w, row = g16 * 16 + r;
    const ZzTensor &T = f.lay.down;
    const int MI = f.MI, nb = MI / ZZ_BLK, D = f.D, S = a.S, K = a.K;
    const bool tq = T.fmt == ZZ_FMT_TQ2, q8 = T.fmt == ZZ_FMT_Q80;
    __shared__ double red[4];
    __shared__ int last;
    float outv[DEC_MAXS];
    double ss[DEC_MAXS];
    for (int s = 0; s < S; s++) {
        float acc_out = 0.0f;
        for (int j = 0; j < K; j++) {
            const int p = a.ppos[s * K + j], e = a.eidx[s * K + j];
            const float wt = a.ewt[s * K + j];
            const uint8_t *E = f.experts + (size_t)e * f.estride;
            const int8_t *hq = f.hq + (size_t)p * MI;
            const float *hs = f.hs + (size_t)p * nb;
            float part = 0.0f;
            if (tq) {
                // 64-weight groups: quarter q takes groups q, q+4, ...
                for (int g = q; g < nb / 2; g += 4) {
                    const uint4 c = *(const uint4 *)(E + zz_qoff(T, row, g));
                    const int8_t *x = hq + g * 64;
                    const uint4 x0 = *(const uint4 *)x, x1 = *(const uint4 *)(x + 16);
                    const uint4 x2 = *(const uint4 *)(x + 32), x3 = *(const uint4 *)(x + 48);
                    int d0 = 0, d1 = 0;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const unsigned m = 0x03030303u;
                        const int sa = 4 * h, sb = 4 * h + 2;
                        const uint4 xa = h ? x2 : x0, xb = h ? x3 : x1;
                        int d = zz_dot4((c.x >> sa) & m, xa.x, 0);
                        d = zz_dot4((c.y >> sa) & m, xa.y, d);
                        d = zz_dot4((c.z >> sa) & m, xa.z, d);
                        d = zz_dot4((c.w >> sa) & m, xa.w, d);
                        d = zz_dot4((c.x >> sb) & m, xb.x, d);
                        d = zz_dot4((c.y >> sb) & m, xb.y, d);
                        d = zz_dot4((c.z >> sb) & m, xb.z, d);
                        d = zz_dot4((c.w >> sb) & m, xb.w, d);
                        // c - 1 per weight: subtract the block's sum of x
                        d -= f.hsum[(size_t)p * nb + 2 * g + h];
                        if (h) d1 = d; else d0 = d;
                    }
                    part = fmaf(hs[2 * g], (float)d0, part);
                    part = fmaf(hs[2 * g + 1], (float)d1, part);
                }
            } else {
#pragma unroll 2
                for (int b = q; b < nb; b += 4) {
                    const uint8_t *qp = E + zz_qoff(T, row, b);
                    const float dw = zz_h2f(*(const uint16_t *)(E + zz_soff(T, row, b)));
                    const int8_t *x = hq + b * ZZ_BLK;
                    const uint4 x0 = *(const uint4 *)x, x1 = *(const uint4 *)(x + 16);
                    const uint4 w0 = *(const uint4 *)qp;
                    int d;
                    if (q8) {
                        const uint4 w1 = *(const uint4 *)(qp + 16);
                        d = zz_dot4(w0.x, x0.x, 0);
                        d = zz_dot4(w0.y, x0.y, d);
                        d = zz_dot4(w0.z, x0.z, d);
                        d = zz_dot4(w0.w, x0.w, d);
                        d = zz_dot4(w1.x, x1.x, d);
                        d = zz_dot4(w1.y, x1.y, d);
                        d = zz_dot4(w1.z, x1.z, d);
                        d = zz_dot4(w1.w, x1.w, d);
                    } else {
                        const unsigned m = 0x0F0F0F0Fu;
                        d = zz_dot4(w0.x & m, x0.x, 0);
                        d = zz_dot4(w0.y & m, x0.y, d);
                        d = zz_dot4(w0.z & m, x0.z, d);
                        d = zz_dot4(w0.w & m, x0.w, d);
                        d = zz_dot4((w0.x >> 4) & m, x1.x, d);
                        d = zz_dot4((w0.y >> 4) & m, x1.y, d);
                        d = zz_dot4((w0.z >> 4) & m, x1.z, d);
                        d = zz_dot4((w0.w >> 4) & m, x1.w, d);
                        d -= 8 * f.hsum[(size_t)p * nb + b];
                    }
                    part = fmaf(dw * hs[b], (float)d, part);
                }
            }
            part += __shfl_xor(part, 16, 64);
            part += __shfl_xor(part, 32, 64);
            if (tq) part *= ((const float *)(E + T.off_s))[row];
            acc_out = fmaf(wt, part, acc_out);     // out += w * y, slot order
        }
        outv[s] = acc_out;
        ss[s] = (double)acc_out * (double)acc_out;
    }
    if (q == 0)
        for (int s = 0; s < S; s++) a.out[(size_t)s * D + row] = outv[s];
    if (!a.gemma) return;
    // post-norm: per-workgroup partial sums of squares, reduced by the last one
    for (int s = 0; s < S; s++) {
        double v = q == 0 ? ss[s] : 0.0;
        v = zz_block_sum(v, red);
        if (tid == 0) a.part[(size_t)s * gridDim.x + blockIdx.x] = v;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(a.ticket, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    __shared__ float rs_s[DEC_MAXS];
    if (tid == 0) {
        for (int s = 0; s < S; s++) {
            double t = 0.0;
            for (int b = 0; b < (int)gridDim.x; b++) t += a.part[(size_t)s * gridDim.x + b];
            rs_s[s] = 1.0f / sqrtf((float)(t / D) + a.eps);
        }
        *a.ticket = 0u;
    }
    __syncthreads();
    for (int s = 0; s < S; s++)
        for (int o = 4 * tid; o < D; o += 1024) {
            float4 v = *(float4 *)(a.out + (size_t)s * D + o);
            const float4 wl = *(const float4 *)(a.post_ln + o);
            const float r = rs_s[s];
            v = make_float4((v.x * r) * wl.x, (v.y * r) * wl.y, (v.z * r) * wl.z, (v.w * r) * wl.w);
            *(float4 *)(a.out + (size_t)s * D + o) = v;
        }
}

int zz_launch_dec_route(const ZzDecRouteArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_route_kernel, dim3((a.lg.E + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dec_down(const ZzDecDownArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(zz_dec_down_kernel, dim3(a.f.D / 64), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}
