// zz_ffn.hip -- slot-table repack of uploaded expert records, the gate-weighted
// combine of the batched path (+ gemma's post-norm), and the debug block dots.
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_dot_dev.h"

// ------------------------------------------------------------------ repack
// Reference record [gate | up | down] (18/34-byte blocks, tq2 alpha + codes) into
// the slot-table layout (zz_common.h). One thread per (row, block); grid.y selects
// the tensor.
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
            uint8_t *q = dst + zz_tq2off(T, row, g);
            for (int k = 0; k < 16; k++) q[k] = s[k];
            if (g == 0)
                for (int k = 0; k < 4; k++) dst[T.off_s + (int64_t)row * 4 + k] = src[(int64_t)row * 4 + k];
        }
        return;
    }
    const bool q8 = T.fmt == ZZ_FMT_Q80;
    const int bb = zz_pbytes(T) + 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int row = (int)(i / nb), b = (int)(i % nb), g = row >> 4, r = row & 15;
        const uint8_t *s = src + i * bb;              // [d fp16][qs]
        const uint8_t *qs = s + 2;
        for (int qq = 0; qq < 4; qq++) {
            uint8_t *q = dst + zz_qlane(T, g, b, 16 * qq + r);
            if (q8) {
                for (int m = 0; m < 8; m++) q[m] = qs[8 * qq + m];
            } else {
                for (int m = 0; m < 4; m++) {       // q40.h:16-17: qs[j] = w_j | w_{j+16} << 4
                    const int k0 = 8 * qq + m, k1 = k0 + 4;
                    const int n0 = k0 < 16 ? qs[k0] & 15 : qs[k0 - 16] >> 4;
                    const int n1 = k1 < 16 ? qs[k1] & 15 : qs[k1 - 16] >> 4;
                    q[m] = (uint8_t)((n0 ^ 8) | ((n1 ^ 8) << 4));   // q - 8 as 4-bit two's complement
                }
            }
        }
        uint8_t *sc = dst + zz_sidx(T, g, b, r);
        sc[0] = s[0];
        sc[1] = s[1];
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
        pos[threadIdx.x] = s * K + threadIdx.x;       // y rows are by flat pair
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

// The same combine for K <= 8 and D <= 1024 * NO with every load issued first: the
// token's weights, its 8 rows' values for all NO column slots of the
// thread, the post-norm weights. The loop above waits out one memory round trip per
// column slot; this one waits once (same sums, same order).
template <int NO>
__global__ __launch_bounds__(256) void zz_combine_fast_kernel(ZzCombineArgs a) {
    const int s = blockIdx.x, D = a.D, K = a.K, t = threadIdx.x;
    __shared__ double red[4];
    int pos[8];
    float wt[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {                // slots past K repeat the last (unused)
        const int jj = min(j, K - 1);
        pos[j] = s * K + jj;                     // y rows are by flat pair
        wt[j] = a.ewt[(size_t)s * K + jj];
    }
    float4 y[NO][8], pl[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) {
        const int o = min(4 * t + 1024 * i, D - 4);
#pragma unroll
        for (int j = 0; j < 8; j++) y[i][j] = *(const float4 *)(a.y + (size_t)pos[j] * D + o);
        if (a.gemma) pl[i] = *(const float4 *)(a.post_ln + o);
    }
    float4 v[NO];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < NO; i++) {
        v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j < K) {
                v[i].x = fmaf(wt[j], y[i][j].x, v[i].x);
                v[i].y = fmaf(wt[j], y[i][j].y, v[i].y);
                v[i].z = fmaf(wt[j], y[i][j].z, v[i].z);
                v[i].w = fmaf(wt[j], y[i][j].w, v[i].w);
            }
        }
        if (4 * t + 1024 * i < D)
            ss += (double)v[i].x * v[i].x + (double)v[i].y * v[i].y + (double)v[i].z * v[i].z +
                  (double)v[i].w * v[i].w;
    }
    float r = 1.0f;
    if (a.gemma) {
        ss = zz_wave_sum(ss);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        const double tot = red[0] + red[1] + red[2] + red[3];
        r = 1.0f / sqrtf((float)(tot / D) + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NO; i++) {
        const int o = 4 * t + 1024 * i;
        if (o < D) {
            float4 u = v[i];
            if (a.gemma)
                u = make_float4((u.x * r) * pl[i].x, (u.y * r) * pl[i].y, (u.z * r) * pl[i].z, (u.w * r) * pl[i].w);
            *(float4 *)(a.out + (size_t)s * D + o) = u;
        }
    }
}

// ------------------------------------------------------------------ debug dots
// Exact int32 dot of one (row, block) against xq: q4_0 sum (q-8)*x, q8_0 sum q*x,
// tq2 sum (c-1)*x, read from the slot table in its lane order.
__global__ void zz_blockdots_kernel(const uint8_t *E, ZzTensor T, int row0, int nrows,
                                    const int8_t *xq, int32_t *out) {
    const int nb = T.I / ZZ_BLK;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * nb) return;
    const int row = row0 + i / nb, b = i % nb, g = row >> 4, r = row & 15;
    const int8_t *x = xq + b * ZZ_BLK;
    int d = 0;
    if (T.fmt == ZZ_FMT_TQ2) {
        const uint4 x0 = ld16(x), x1 = ld16(x + 16);
        int xs = 0;
        for (int j = 0; j < ZZ_BLK; j++) xs += x[j];
        d = zz_dot_tq2(ld16(E + zz_tq2off(T, row, b / 2)), b & 1, x0, x1) - xs;
    } else {
        for (int qq = 0; qq < 4; qq++) {
            const uint8_t *q = E + zz_qlane(T, g, b, 16 * qq + r);
            const uint2 xv = *(const uint2 *)(x + 8 * qq);
            uint2 w;
            if (T.fmt == ZZ_FMT_Q80) w = *(const uint2 *)q;
            else w = zz_q4_unpack16(*(const unsigned *)q);
            d = zz_dot4(w.x, xv.x, d);
            d = zz_dot4(w.y, xv.y, d);
        }
        if (T.fmt == ZZ_FMT_Q40) d >>= 4;          // the 16*(q - 8) weights: exact
    }
    out[i] = d;
}

// ------------------------------------------------------------------ launchers
int zz_launch_repack(const ZzRepackArgs &a, hipStream_t st) { return zz_launch_repack_n(a, 3, st); }

int zz_launch_repack_n(const ZzRepackArgs &a, int n, hipStream_t st) {
    hipLaunchKernelGGL(zz_repack_kernel, dim3(256, n), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_combine(const ZzCombineArgs &a, int S, hipStream_t st) {
    const int no = (a.D + 1023) / 1024;
    if (a.K <= 8 && no <= 1) hipLaunchKernelGGL(zz_combine_fast_kernel<1>, dim3(S), dim3(256), 0, st, a);
    else if (a.K <= 8 && no <= 2) hipLaunchKernelGGL(zz_combine_fast_kernel<2>, dim3(S), dim3(256), 0, st, a);
    else if (a.K <= 8 && no <= 3) hipLaunchKernelGGL(zz_combine_fast_kernel<3>, dim3(S), dim3(256), 0, st, a);
    else if (a.K <= 8 && no <= 4) hipLaunchKernelGGL(zz_combine_fast_kernel<4>, dim3(S), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(zz_combine_kernel, dim3(S), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess;
}

int zz_launch_blockdots(const uint8_t *expert, ZzTensor t, int row0, int nrows,
                        const int8_t *xq, int32_t *out, hipStream_t st) {
    int n = nrows * (t.I / ZZ_BLK);
    hipLaunchKernelGGL(zz_blockdots_kernel, dim3((n + 255) / 256), dim3(256), 0, st, expert, t,
                       row0, nrows, xq, out);
    return hipGetLastError() == hipSuccess;
}
