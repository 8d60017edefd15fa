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
// the bound proves it equals the reference's. Gemma logits carry a tight bound
// from their exact-order prefix sums; the rare values still contested are
// recomputed by replaying the reference's serial chain in the reference's order.
// Batches of 16+ tokens compute the gemma chains exactly instead (tiled kernel).
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_route_dev.h"
#include "zz_topk_wave.h"
#include <float.h>

// Prep: one workgroup per token. Gemma: the mean square is certified to round to
// the float the reference's serial double sum gives (gemma4.c:425-428), else that
// sum is replayed serially; then the router input xn = rmsnorm(x)*scale*D^-1/2
// (gemma4.c:591-593), unless there is no router (the dense branch, which routes
// every row to its one expert with weight 1 here). The expert input X (gemma: rmsnorm(x, pre_ffn_ln2),
// gemma4.c:763-764; lfm/maple: x) is quantised q8_0-style (q40.h:124-138), one
// 32-block per thread, with per-block integer sums; for tq2 the Sx total
// (tq2.h:98-108) is summed serially in the reference's order.
#define PREP_R 8           // float4 per thread: D <= 8192
__global__ __launch_bounds__(256) void zz_prep_kernel(ZzPrepArgs a) {
    const int s = blockIdx.x, D = a.D, tid = threadIdx.x, nb = D / ZZ_BLK, n4 = D / 4;
    const float *x = a.in + (size_t)s * D;
    __shared__ double red[4];
    __shared__ float xs_l[ZZ_MAXD / ZZ_BLK];
    __shared__ int xsum_l[ZZ_MAXD / ZZ_BLK];
    __shared__ float cert;
    // the row, its norm weights and router scale: every load issued first. Float4 i
    // of the row is value 4i..4i+3: block i/8, lane i%8 of the block's 8 lanes.
    const int R = (n4 + 255) >> 8;
    float4 xv[PREP_R], wv[PREP_R], sv[PREP_R];
#pragma unroll
    for (int k = 0; k < PREP_R; k++) {
        if (k >= R) break;
        const int i = min(tid + 256 * k, n4 - 1);
        xv[k] = *(const float4 *)(x + 4 * i);
        if (a.gemma) wv[k] = *(const float4 *)(a.pre_ln + 4 * i);
        if (a.gemma && a.router_scale) sv[k] = *(const float4 *)(a.router_scale + 4 * i);
    }
    if (a.route_eidx && tid == 0) {                // dense branch: one expert, weight 1
        a.route_eidx[s] = 0;
        a.route_ewt[s] = 1.0f;
    }
    float r = 1.0f;
    if (a.gemma) {
        double sq = 0.0;
#pragma unroll
        for (int k = 0; k < PREP_R; k++) {
            if (k >= R) break;
            if (tid + 256 * k < n4) {
                const float4 v = xv[k];
                sq += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
            }
        }
        sq = zz_block_sum(sq, red);
        // GPU: each term in <= R + 12 roundings; reference: D - 1 in order.
        // All terms are non-negative, so the exact sum is <= sq / (1 - g_m).
        const double m = (double)(R + 12);
        const double g = zz_gamma(D, ZZ_U64) + zz_gamma(m, ZZ_U64);
        const double b = g * sq / (1.0 - zz_gamma(m, ZZ_U64)) * 1.0000001 + 1e-300;
        const float lo = (float)((sq - b) / (double)D), hi = (float)((sq + b) / (double)D);
        if (tid == 0) {
            if (lo == hi) {
                cert = lo;
            } else {
                double t = 0.0;                    // serial replay, reference order
                for (int i = 0; i < D; i++) t += (double)x[i] * (double)x[i];
                cert = (float)(t / (double)D);
                atomicAdd(a.diag + 0, 1u);
            }
        }
        __syncthreads();
        r = 1.0f / sqrtf(cert + a.eps);
        if (a.router_scale) {                      // the router input (no router: no xn)
            const float rs = 1.0f / sqrtf((float)D);
#pragma unroll
            for (int k = 0; k < PREP_R; k++) {
                if (k >= R) break;
                const int i = tid + 256 * k;
                if (i < n4) {
                    const float4 v = xv[k], sc = sv[k];
                    *(float4 *)(a.xn + (size_t)s * D + 4 * i) =
                        make_float4((v.x * r) * (sc.x * rs), (v.y * r) * (sc.y * rs), (v.z * r) * (sc.z * rs),
                                    (v.w * r) * (sc.w * rs));
                }
            }
        }
    }
    // q8_0 of the expert input, 8 lanes per block (every lane of a wave takes part)
#pragma unroll
    for (int k = 0; k < PREP_R; k++) {
        if (k >= R) break;
        const int i = tid + 256 * k;
        float4 v = xv[k];
        if (a.gemma) {
            const float4 w = wv[k];
            v = make_float4((v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w);
        }
        float d;
        int qs;
        const unsigned pk = zz_quant8(v, &d, &qs);
        if (i < n4) {
            *(unsigned *)(a.xq + (size_t)s * D + 4 * i) = pk;
            if ((i & 7) == 0) {
                const int b = i >> 3;
                a.xs[(size_t)s * nb + b] = d;
                a.xsum[(size_t)s * nb + b] = qs;
                xs_l[b] = d;
                xsum_l[b] = qs;
            }
        }
    }
    if (a.xt) {
        __syncthreads();
        if (tid == 0) {
            double tot = 0.0;                      // tq2.h:101-106, serial
            for (int b = 0; b < nb; b++) tot += (double)xs_l[b] * (double)xsum_l[b];
            a.xt[s] = (float)tot;
        }
    }
}

__global__ __launch_bounds__(256) void zz_logits_kernel(ZzLogitArgs a) {
    __shared__ __attribute__((aligned(16))) float buf[4 * ZZ_TBUF];
    const int s = blockIdx.y, e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= a.E) return;
    if (a.gating == ZZ_GATE_SOFTMAX_PES) {
        const size_t o = (size_t)s * a.E + e;
        zz_tight_wave<1, false>(a.router + (size_t)e * a.D, a.xn + (size_t)s * a.D, nullptr, nullptr,
                                1.0f, a.D, a.bias, e, buf + (threadIdx.x >> 6) * ZZ_TBUF, a.cen + o,
                                a.bnd + o, a.E, nullptr);
    } else {
        zz_logit_wave_f64(a, s, e);
    }
}

// -------------------------------------------------------------------------------
// Router logits for batches: the reference's own serial chains, exactly. One
// thread owns one (token, expert) pair and walks k = 0..D-1 in order:
//   gemma  v = v + fl(w_k * xn_k) in fp32, unfused (gemma4.c:600-601 as compiled:
//          vmulps then in-order vaddss);
//   lfm / maple  v = v + (double)w_k * x_k in double, then (float)v
//          (lfm25.c:646-647, maple.c:400-410);
//   ling   eight double accumulators by k % 8, combined pairwise (ling.c:722-727).
// A workgroup is 16 tokens x 16 experts; 64-wide K chunks of both operands are
// staged in LDS so each router row and each input row is read once per tile.
// Many independent chains (one per thread) hide the add latency.
#define LG_T 16
#define LG_E 16
#define LG_K 64
__global__ __launch_bounds__(256) void zz_logits_exact_kernel(ZzLogitArgs a) {
    const int tid = threadIdx.x, tt = tid / LG_E, te = tid % LG_E;
    const int s0 = blockIdx.x * LG_T, e0 = blockIdx.y * LG_E;
    const int s = s0 + tt, e = e0 + te, D = a.D;
    const bool gem = a.gating == ZZ_GATE_SOFTMAX_PES;
    const float *X = gem ? a.xn : a.x;
    __shared__ float xs_t[2][LG_T][LG_K + 4];
    __shared__ float ws_t[2][LG_E][LG_K + 4];
    // staging: each thread moves LG_V float4 of each tile per chunk (rows clamped
    // into range: a row past the end holds copies, its chains are not stored)
    constexpr int LG_V = LG_T * LG_K / 4 / 256;
    const int lr = tid / (LG_K / 4 / LG_V), lc = (tid % (LG_K / 4 / LG_V)) * 4 * LG_V;
    const float *xsrc = X + (size_t)min(s0 + lr, a.S - 1) * D + lc;
    const float *wsrc = a.router + (size_t)min(e0 + lr, a.E - 1) * D + lc;
    float4 xv[LG_V], wv[LG_V];
#pragma unroll
    for (int v = 0; v < LG_V; v++) {
        xv[v] = *(const float4 *)(xsrc + 4 * v);
        wv[v] = *(const float4 *)(wsrc + 4 * v);
    }
#pragma unroll
    for (int v = 0; v < LG_V; v++) {
        *(float4 *)&xs_t[0][lr][lc + 4 * v] = xv[v];
        *(float4 *)&ws_t[0][lr][lc + 4 * v] = wv[v];
    }
    __syncthreads();
    float vf = 0.0f;
    double vd = 0.0;
    double v8[8] = {0, 0, 0, 0, 0, 0, 0, 0};         // grouped: ling.c's 8 accumulators
    const bool grp = a.gating == ZZ_GATE_GROUPED;
    int buf = 0;
    for (int k0 = 0; k0 < D; k0 += LG_K) {
        const int k1 = min(k0 + LG_K, D - LG_K);    // the last chunk reloads itself
#pragma unroll
        for (int v = 0; v < LG_V; v++) {
            xv[v] = *(const float4 *)(xsrc + k1 + 4 * v);
            wv[v] = *(const float4 *)(wsrc + k1 + 4 * v);
        }
        const float *xr = xs_t[buf][tt], *wr = ws_t[buf][te];
        if (gem) {
#pragma unroll 16
            for (int k = 0; k < LG_K; k += 4) {
                const float4 x4 = *(const float4 *)(xr + k), w4 = *(const float4 *)(wr + k);
                vf = vf + w4.x * x4.x;
                vf = vf + w4.y * x4.y;
                vf = vf + w4.z * x4.z;
                vf = vf + w4.w * x4.w;
            }
        } else if (grp) {
            // element k0 + k goes to accumulator k % 8 (k0 is a multiple of LG_K)
#pragma unroll 16
            for (int k = 0; k < LG_K; k += 8) {
                const float4 xa = *(const float4 *)(xr + k), wa = *(const float4 *)(wr + k);
                const float4 xb = *(const float4 *)(xr + k + 4), wb = *(const float4 *)(wr + k + 4);
                v8[0] = v8[0] + (double)wa.x * (double)xa.x;
                v8[1] = v8[1] + (double)wa.y * (double)xa.y;
                v8[2] = v8[2] + (double)wa.z * (double)xa.z;
                v8[3] = v8[3] + (double)wa.w * (double)xa.w;
                v8[4] = v8[4] + (double)wb.x * (double)xb.x;
                v8[5] = v8[5] + (double)wb.y * (double)xb.y;
                v8[6] = v8[6] + (double)wb.z * (double)xb.z;
                v8[7] = v8[7] + (double)wb.w * (double)xb.w;
            }
        } else {
#pragma unroll 16
            for (int k = 0; k < LG_K; k += 4) {
                const float4 x4 = *(const float4 *)(xr + k), w4 = *(const float4 *)(wr + k);
                vd = vd + (double)w4.x * (double)x4.x;
                vd = vd + (double)w4.y * (double)x4.y;
                vd = vd + (double)w4.z * (double)x4.z;
                vd = vd + (double)w4.w * (double)x4.w;
            }
        }
#pragma unroll
        for (int v = 0; v < LG_V; v++) {
            *(float4 *)&xs_t[buf ^ 1][lr][lc + 4 * v] = xv[v];
            *(float4 *)&ws_t[buf ^ 1][lr][lc + 4 * v] = wv[v];
        }
        __syncthreads();
        buf ^= 1;
    }
    if (s < a.S && e < a.E) {
        const size_t o = (size_t)s * a.E + e;
        if (gem) {
            if (a.bias) vf = vf + a.bias[e];       // harness logit offset, after the dot
            a.cen[o] = (double)vf;
        } else {
            if (grp) vd = ((v8[0] + v8[1]) + (v8[2] + v8[3])) + ((v8[4] + v8[5]) + (v8[6] + v8[7]));
            a.cen[o] = (double)(float)vd;
        }
        a.bnd[o] = 0.0;                             // exact: no interval
    }
}

// Top-k gating, one wave per token (zz_topk_wave.h), four tokens per workgroup.
__global__ __launch_bounds__(256) void zz_topk_kernel(ZzTopkArgs a, int S) {
    extern __shared__ __attribute__((aligned(16))) char tk_lds[];
    const int w = threadIdx.x >> 6, s = blockIdx.x * 4 + w;
    if (s >= S) return;
    zz_topk_wave_any(a, s, tk_lds + w * zz_topk_wave_bytes(a.E));
}

// -------------------------------------------------------------------------------
// Dispatch, one workgroup of 512 threads. Each expert gets a bitmask over tokens;
// a pair's place in its expert's list is the expert's start plus the number of
// earlier tokens that chose it (a popcount) -- the stable counting sort that gives
// exactly rows[] of gemma4.c:779-786, ascending tokens. The smallest pair index
// of each expert orders the union as first-seen (gemma4.c:756-761). Also emits
// the FFN work list: per expert in union order, chunks of at most `tch` pairs.
// exclusive prefix sum over the 512 threads of a workgroup: a shuffle scan per wave,
// then the wave totals (two barriers)
__device__ __forceinline__ int zz_block_excl_scan(int v, int *tmp) {
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int n = __shfl_up(x, off, 64);
        if (l >= off) x += n;
    }
    if (l == 63) tmp[w] = x;
    __syncthreads();
    int base = 0;
    for (int q = 0; q < w; q++) base += tmp[q];
    __syncthreads();                           // tmp is free again for the next scan
    return base + x - v;
}

#define DP_PT 16                      // pairs per thread: S*K <= 8192 = 512 * DP_PT
// One workgroup: the per-expert token bitmasks give each expert's count, its pairs'
// positions (a stable counting sort by expert, gemma4.c:779-786) and its first pair;
// the union order is the order of first pairs (gemma4.c:756-761), read off a bitmap
// over the pairs by prefix popcounts.
// LDS: mask and word prefixes [E][W] (W = S/32 words), first-pair bitmap [P/32],
// pair experts [P] (then the inverse permutation) and weights by position [P].
__global__ __launch_bounds__(512) void zz_dispatch_kernel(ZzDispatchArgs a) {
    extern __shared__ unsigned dsm[];
    __shared__ int cnt[ZZ_MAXE], start[ZZ_MAXE], first[ZZ_MAXE], order[ZZ_MAXE], tmp[16];
    __shared__ int fbase[DP_PT * 512 / 32];      // first pairs before each bitmap word
    const int P = a.P, E = a.E, K = a.K, S = P / K, W = (S + 31) / 32, PW = (P + 31) / 32, t = threadIdx.x;
    unsigned *mask = dsm, *wpre = dsm + E * W, *fb = wpre + E * W;
    int *pe = (int *)(fb + PW);                  // pair -> expert, later position -> pair
    float *pwl = (float *)(pe + P);              // position -> weight
    for (int i = t; i < E * W; i += 512) mask[i] = 0u;
    for (int i = t; i < PW; i += 512) fb[i] = 0u;
    // every pair's expert and weight in registers first: one round of loads
    int ev[DP_PT];
    float wv[DP_PT];
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = min(t + 512 * k, P - 1);
        const int e = a.eidx[p];
        ev[k] = e < 0 || e >= E ? 0 : e;            // never index past the expert tables
        wv[k] = a.ewt[p];
    }
#pragma unroll
    for (int k = 0; k < DP_PT; k++)
        if (t + 512 * k < P) pe[t + 512 * k] = ev[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = t + 512 * k, s = p / K;
        if (p < P) atomicOr(&mask[ev[k] * W + (s >> 5)], 1u << (s & 31));
    }
    __syncthreads();
    // per expert: word prefix counts, the count, and the first pair that routes to
    // it (its lowest token, that token's slot holding e)
    for (int e = t; e < E; e += 512) {
        int run = 0, s0 = -1;
        for (int w = 0; w < W; w++) {
            const unsigned m = mask[e * W + w];
            wpre[e * W + w] = run;
            if (s0 < 0 && m) s0 = 32 * w + __ffs(m) - 1;
            run += __popc(m);
        }
        cnt[e] = run;
        int f = 0x7fffffff;
        if (s0 >= 0) {
            for (int j = K - 1; j >= 0; j--)
                if (pe[s0 * K + j] == e) f = s0 * K + j;
            atomicOr(&fb[f >> 5], 1u << (f & 31));
        }
        first[e] = f;
    }
    const int st = zz_block_excl_scan(t < E ? cnt[t] : 0, tmp);   // its barrier orders the above
    if (t < E) start[t] = st;
    // union rank of each present expert: first pairs below its own
    const int fw = t < PW ? __popc(fb[t]) : 0;
    const int fpre = zz_block_excl_scan(fw, tmp);
    if (t < PW) fbase[t] = fpre;
    __syncthreads();
    // positions; the sorted lists are then written in position order (coalesced)
    // through the inverse permutation, which reuses the pair-expert array
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int p = t + 512 * k;
        if (p < P) {
            const int e = ev[k], s = p / K, w = s >> 5, bit = s & 31;
            const int pos = start[e] + wpre[e * W + w] + __popc(mask[e * W + w] & ((1u << bit) - 1u));
            a.ppos[p] = pos;
            pe[pos] = p;
            pwl[pos] = wv[k];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < DP_PT; k++) {
        const int i = t + 512 * k;
        if (i < P) {
            const int p = pe[i], s = p / K;
            a.ptok[i] = s;
            a.pslot[i] = p - s * K;
            a.pwt[i] = pwl[i];
        }
    }
    const bool present = t < E && cnt[t] != 0;
    if (present) {
        const int f = first[t];
        order[fbase[f >> 5] + __popc(fb[f >> 5] & ((1u << (f & 31)) - 1u))] = t;
    }
    const int nu = __syncthreads_count(present);
    const int ce = t < nu ? cnt[order[t]] : 0;
    const int nit = (ce + a.tch - 1) / a.tch;
    const int i0 = zz_block_excl_scan(nit, tmp);
    if (t < nu) {
        const int e = order[t];
        a.uniq[t] = e;
        a.uoff[t] = start[e];
        a.ucnt[t] = ce;
        for (int c = 0; c < nit; c++) {
            ZzItem it;
            it.e = e;
            it.u = t;
            it.p0 = start[e] + c * a.tch;
            it.n = min(a.tch, ce - c * a.tch);
            a.items[i0 + c] = it;
        }
    }
    if (t == nu - 1 || (nu == 0 && t == 0)) {
        a.meta[0] = nu;
        a.meta[1] = i0 + nit;
    }
}

// ------------------------------------------------------------------ launchers
int zz_launch_prep(const ZzPrepArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_prep_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_logits(const ZzLogitArgs &a, int S, hipStream_t st) {
    if (S >= 16 && a.D % LG_K == 0) {
        ZzLogitArgs b = a;
        b.S = S;
        hipLaunchKernelGGL(zz_logits_exact_kernel, dim3((S + LG_T - 1) / LG_T, (a.E + LG_E - 1) / LG_E),
                           dim3(256), 0, st, b);
    } else {
        hipLaunchKernelGGL(zz_logits_kernel, dim3((a.E + 3) / 4, S), dim3(256), 0, st, a);
    }
    return hipGetLastError() == hipSuccess;
}

int zz_launch_topk(const ZzTopkArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_topk_kernel, dim3((S + 3) / 4), dim3(256), 4 * zz_topk_wave_bytes(a.E), st, a, S);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_dispatch(const ZzDispatchArgs &a, hipStream_t st) {
    const int W = (a.P / a.K + 31) / 32, PW = (a.P + 31) / 32;
    const size_t lds = sizeof(unsigned) * (2 * (size_t)a.E * W + PW) + 8 * (size_t)a.P;
    hipLaunchKernelGGL(zz_dispatch_kernel, dim3(1), dim3(512), lds, st, a);
    return hipGetLastError() == hipSuccess;
}
