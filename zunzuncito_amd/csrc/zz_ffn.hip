// zz_ffn.hip -- expert FFN on gfx950: slot-table repack, gate/up GEMV with the
// fused activation and int8 re-quantisation of the hidden, down GEMV, and the
// gate-weighted combine (+ gemma's post-norm).
//
// The per-block integer dots are exact int32 (v_dot4_i32_i8): q4_0 uses the
// unsigned nibbles and subtracts 8*sum(x) (q40.h:30-32), tq2 uses the unsigned
// codes and subtracts Sx once per row (tq2.h:29-37), q8_0 is signed x signed.
// Across blocks the fp32 accumulation order is this kernel's own; the layer
// output matches the reference within the fp32 tolerance, the integers exactly.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_dot_dev.h"

#define ZZ_TCH 8   // pairs (token, expert) per FFN work item

// Partial row dot of one lane: blocks b = sub, sub+4, ... of row `row` of tensor T
// against the int8 activations of up to ZZ_TCH tokens. Returns per-token partial
// sums of d_w * d_x * int32 (q4_0 / q8_0) or d_x * int32 (tq2, alpha applied later).
template <int NT>
__device__ __forceinline__ void zz_row_partial(const uint8_t *E, const ZzTensor &T, int row, int sub,
                                               int nt, const int8_t *const *xq,
                                               const float *const *xs, const int *const *xsum,
                                               float (&acc)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
    if (T.fmt == ZZ_FMT_TQ2) {
        const int ng = T.I / 64;
        for (int g = sub; g < ng; g += 4) {
            uint4 c = ld16(E + zz_qoff(T, row, g));
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (t < nt) {
                    const int8_t *x = xq[t] + g * 64;
                    uint4 x0 = ld16(x), x1 = ld16(x + 16), x2 = ld16(x + 32), x3 = ld16(x + 48);
                    int d0 = zz_dot_tq2(c, 0, x0, x1), d1 = zz_dot_tq2(c, 1, x2, x3);
                    acc[t] = fmaf(xs[t][2 * g], (float)d0, acc[t]);
                    acc[t] = fmaf(xs[t][2 * g + 1], (float)d1, acc[t]);
                }
            }
        }
        return;
    }
    const int nb = T.I / ZZ_BLK;
    const bool q8 = T.fmt == ZZ_FMT_Q80;
    for (int b = sub; b < nb; b += 4) {
        const uint8_t *qs = E + zz_qoff(T, row, b);
        float dw = zz_h2f(*(const uint16_t *)(E + zz_soff(T, row, b)));
        uint4 w0 = ld16(qs), w1 = make_uint4(0, 0, 0, 0);
        if (q8) w1 = ld16(qs + 16);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < nt) {
                const int8_t *x = xq[t] + b * ZZ_BLK;
                uint4 x0 = ld16(x), x1 = ld16(x + 16);
                int d = q8 ? zz_dot_q80(w0, w1, x0, x1) : zz_dot_q40(w0, x0, x1) - 8 * xsum[t][b];
                acc[t] = fmaf(dw * xs[t][b], (float)d, acc[t]);
            }
        }
    }
}

// ------------------------------------------------------------------ repack
// Reference record [gate | up | down] (18/34-byte blocks, tq2 alpha+codes) into
// the slot-table layout. One thread per (row, block); grid.y selects the tensor.
__global__ void zz_repack_kernel(ZzRepackArgs a) {
    const ZzTensor &T = blockIdx.y == 0 ? a.lay.gate : (blockIdx.y == 1 ? a.lay.up : a.lay.down);
    const int64_t so = blockIdx.y == 0 ? a.src_gate : (blockIdx.y == 1 ? a.src_up : a.src_down);
    const uint8_t *src = a.src + so;
    uint8_t *dst = a.dst;
    const int nb = zz_nblk(T);
    const int64_t n = (int64_t)T.O * nb;
    if (T.fmt == ZZ_FMT_TQ2) {
        const uint8_t *codes = src + (int64_t)T.O * 4;
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
             i += (int64_t)gridDim.x * blockDim.x) {
            const int row = (int)(i / nb), g = (int)(i % nb);
            const uint8_t *s = codes + (int64_t)row * (T.I / 4) + (int64_t)g * 16;
            uint8_t *q = dst + zz_qoff(T, row, g);
            for (int k = 0; k < 16; k++) q[k] = s[k];
            if (g == 0)
                for (int k = 0; k < 4; k++) dst[T.off_s + (int64_t)row * 4 + k] = src[(int64_t)row * 4 + k];
        }
        return;
    }
    const int pb = zz_pbytes(T), bb = pb + 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int row = (int)(i / nb), b = (int)(i % nb);
        const uint8_t *s = src + i * bb;
        uint8_t *q = dst + zz_qoff(T, row, b);
        for (int k = 0; k < pb; k++) q[k] = s[2 + k];
        uint8_t *sc = dst + zz_soff(T, row, b);
        sc[0] = s[0];
        sc[1] = s[1];
    }
}

// ------------------------------------------------------------------ gate / up
// grid (MI/32, items). Waves 0,1 compute gate rows rb*32 + 0..31, waves 2,3 the
// same up rows; 4 lanes per row. Then one lane per (token, row) forms
// h = act(g, u) and the 32 lanes of a token quantise the 32-block of h
// (gemma4.c:642-645, lfm25.c:712-723, maple.c:665-684).
__global__ __launch_bounds__(256) void zz_ffn_up_kernel(ZzFfnArgs a) {
    const int it = blockIdx.y;
    if (it >= a.meta[1]) return;
    const ZzItem item = a.items[it];
    const int rb = blockIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63, sub = l & 3;
    const ZzTensor &T = w < 2 ? a.lay.gate : a.lay.up;
    const int rloc = (w & 1) * 16 + (l >> 2), row = rb * 32 + rloc;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    const int D = a.D, nb = D / ZZ_BLK;
    const int8_t *xq[ZZ_TCH];
    const float *xs[ZZ_TCH];
    const int *xsum[ZZ_TCH];
    int tok[ZZ_TCH];
#pragma unroll
    for (int t = 0; t < ZZ_TCH; t++) {
        tok[t] = t < item.n ? a.ptok[item.p0 + t] : 0;
        xq[t] = a.xq + (size_t)tok[t] * D;
        xs[t] = a.xs + (size_t)tok[t] * nb;
        xsum[t] = a.xsum + (size_t)tok[t] * nb;
    }
    float acc[ZZ_TCH];
    zz_row_partial<ZZ_TCH>(E, T, row, sub, item.n, xq, xs, xsum, acc);
    __shared__ float gu[ZZ_TCH][64];
#pragma unroll
    for (int t = 0; t < ZZ_TCH; t++) {
        float v = acc[t];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        if (T.fmt == ZZ_FMT_TQ2) {
            const float alpha = ((const float *)(E + T.off_s))[row];
            v = alpha * (v - a.xt[tok[t]]);                   // tq2.h:154
        }
        if (sub == 0) gu[t][w * 16 + (l >> 2)] = v;
    }
    __syncthreads();
    __shared__ float hb[ZZ_TCH][ZZ_BLK + 1];
    {
        const int t = threadIdx.x >> 5, r = threadIdx.x & 31;
        if (t < item.n) hb[t][r] = zz_act(a.act, gu[t][r], gu[t][32 + r], a.clamp);
    }
    __syncthreads();
    if (threadIdx.x < item.n) {                       // one thread quantises a token's block
        float v[ZZ_BLK];
#pragma unroll
        for (int r = 0; r < ZZ_BLK; r++) v[r] = hb[threadIdx.x][r];
        const size_t p = (size_t)item.p0 + threadIdx.x;
        int qs;
        const float d = zz_quant_block(v, a.hq + p * a.MI + rb * 32, &qs);
        a.hs[p * (a.MI / ZZ_BLK) + rb] = d;
        a.hsum[p * (a.MI / ZZ_BLK) + rb] = qs;
    }
}

// ------------------------------------------------------------------ down
// grid (D/64, items): 64 output rows per workgroup, 4 lanes per row. Writes the
// unweighted expert output y[pair][row]; the combine applies the gate weights.
__global__ __launch_bounds__(256) void zz_ffn_down_kernel(ZzFfnArgs a) {
    const int it = blockIdx.y;
    if (it >= a.meta[1]) return;
    const ZzItem item = a.items[it];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, sub = l & 3;
    const int row = blockIdx.x * 64 + w * 16 + (l >> 2);
    const ZzTensor &T = a.lay.down;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    const int MI = a.MI, nb = MI / ZZ_BLK;
    __shared__ float htot[ZZ_TCH];
    if (T.fmt == ZZ_FMT_TQ2 && threadIdx.x < item.n) {
        const size_t p = (size_t)item.p0 + threadIdx.x;   // tq2.h:101-106, serial
        double tot = 0.0;
        for (int b = 0; b < nb; b++)
            tot += (double)a.hs[p * nb + b] * (double)a.hsum[p * nb + b];
        htot[threadIdx.x] = (float)tot;
    }
    __syncthreads();
    if (row >= a.D) return;
    const int8_t *xq[ZZ_TCH];
    const float *xs[ZZ_TCH];
    const int *xsum[ZZ_TCH];
#pragma unroll
    for (int t = 0; t < ZZ_TCH; t++) {
        const size_t p = (size_t)item.p0 + (t < item.n ? t : 0);
        xq[t] = a.hq + p * MI;
        xs[t] = a.hs + p * nb;
        xsum[t] = a.hsum + p * nb;
    }
    float acc[ZZ_TCH];
    zz_row_partial<ZZ_TCH>(E, T, row, sub, item.n, xq, xs, xsum, acc);
#pragma unroll
    for (int t = 0; t < ZZ_TCH; t++) {
        float v = acc[t];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        if (T.fmt == ZZ_FMT_TQ2) {
            const float alpha = ((const float *)(E + T.off_s))[row];
            v = alpha * (v - htot[t]);
        }
        if (sub == 0 && t < item.n) a.y[((size_t)item.p0 + t) * a.D + row] = v;
    }
}

// ------------------------------------------------------------------ combine
// out[s] = sum_j w[s,j] * y[pair(s,j)] in slot order, fused multiply-add as the
// reference's `out[o] += ww * dot` (gemma4.c:652); gemma then applies
// rmsnorm(out, post_ffn_ln2) (gemma4.c:807-808). One workgroup per token.
__global__ __launch_bounds__(256) void zz_combine_kernel(ZzCombineArgs a) {
    const int s = blockIdx.x, D = a.D, K = a.K;
    __shared__ float row[ZZ_MAXD];
    __shared__ double red[4];
    __shared__ int pos[ZZ_MAXK];
    __shared__ float wt[ZZ_MAXK];
    if (threadIdx.x < K) {
        pos[threadIdx.x] = a.ppos[(size_t)s * K + threadIdx.x];
        wt[threadIdx.x] = a.ewt[(size_t)s * K + threadIdx.x];
    }
    __syncthreads();
    double ss = 0.0;
    for (int o = 4 * threadIdx.x; o < D; o += 1024) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
        for (int j = 0; j < K; j++) {
            const float4 y = *(const float4 *)(a.y + (size_t)pos[j] * D + o);
            const float w = wt[j];
            v.x = fmaf(w, y.x, v.x);
            v.y = fmaf(w, y.y, v.y);
            v.z = fmaf(w, y.z, v.z);
            v.w = fmaf(w, y.w, v.w);
        }
        *(float4 *)&row[o] = v;
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    float r = 1.0f;
    if (a.gemma) {
        ss = zz_wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        double tot = red[0] + red[1] + red[2] + red[3];
        r = 1.0f / sqrtf((float)(tot / D) + a.eps);
    }
    for (int o = 4 * threadIdx.x; o < D; o += 1024) {
        float4 v = *(const float4 *)&row[o];
        if (a.gemma) {
            const float4 w = *(const float4 *)(a.post_ln + o);
            v = make_float4((v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w);
        }
        *(float4 *)(a.out + (size_t)s * D + o) = v;
    }
}

// ------------------------------------------------------------------ debug dots
__global__ void zz_blockdots_kernel(const uint8_t *E, ZzTensor T, int row0, int nrows,
                                    const int8_t *xq, int32_t *out) {
    const int nb = T.I / ZZ_BLK;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * nb) return;
    const int r = row0 + i / nb, b = i % nb;
    const int8_t *x = xq + b * ZZ_BLK;
    uint4 x0 = ld16(x), x1 = ld16(x + 16);
    int xs = 0;
    for (int j = 0; j < ZZ_BLK; j++) xs += x[j];
    int d;
    if (T.fmt == ZZ_FMT_Q40) {
        d = zz_dot_q40(ld16(E + zz_qoff(T, r, b)), x0, x1) - 8 * xs;
    } else if (T.fmt == ZZ_FMT_Q80) {
        const uint8_t *q = E + zz_qoff(T, r, b);
        d = zz_dot_q80(ld16(q), ld16(q + 16), x0, x1);
    } else {
        d = zz_dot_tq2(ld16(E + zz_qoff(T, r, b / 2)), b & 1, x0, x1) - xs;
    }
    out[i] = d;
}

// ------------------------------------------------------------------ launchers
int zz_launch_repack(const ZzRepackArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(zz_repack_kernel, dim3(256, 3), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_ffn_up(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    hipLaunchKernelGGL(zz_ffn_up_kernel, dim3(a.MI / 32, max_items), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_ffn_down(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    hipLaunchKernelGGL(zz_ffn_down_kernel, dim3((a.D + 63) / 64, max_items), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_combine(const ZzCombineArgs &a, int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_combine_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_blockdots(const uint8_t *expert, ZzTensor t, int row0, int nrows,
                        const int8_t *xq, int32_t *out, hipStream_t st) {
    int n = nrows * (t.I / ZZ_BLK);
    hipLaunchKernelGGL(zz_blockdots_kernel, dim3((n + 255) / 256), dim3(256), 0, st, expert, t,
                       row0, nrows, xq, out);
    return hipGetLastError() == hipSuccess;
}
