// zz_flash.hip -- FlashHead, gemma4's approximate tied lm_head (flash_logits and
// flash_partition, gemma4.c:1055-1131; the tensors tools/flashhead.py writes): score
// every cluster's q4_0 centroid against the q8_0 row of rmsnorm(H, final_norm), take
// the n_probes best clusters, and compute logits only for their member tokens and the
// forced ids; every other logit is -inf.
//
// Which clusters are probed decides which tokens can be chosen, so the scores are the
// reference's own floats: each centroid dot is q40_dot in the AVX2 build's order
// (zz_q40_dot_avx), and the n_probes best are taken by a radix select whose result is
// checked for a tie straddling the boundary. Only then does the set depend on the
// reference quickselect's steps, and the select kernel replays them serially.
//
// Kernels, per decode step and row:
//   zz_flash_sim_kernel     NC/8 workgroups: 32 threads per centroid row (and the
//                           -inf fill of the logits)
//   zz_flash_select_kernel  one workgroup per row: radix select, tie check, replay
//   zz_flash_probe_kernel   one 32-thread group per candidate id: its logit, softcap,
//                           and per-workgroup (logit, -id) keys for the argmax finish
// The probed rows are read from a reference-layout copy of the table (one contiguous
// 18-byte block after another), which zz_flash_unpack_kernel writes once from the
// slot-table lane order the full head streams.
#include "zz_common.h"
#include "zz_kernels.h"

#include <math.h>

#define FL_ROWS 8               // rows per 256-thread workgroup, 32 threads each

__device__ __forceinline__ unsigned zz_fl_ord(float f) {   // order-preserving float bits
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// q40_dot (q40.h:162-207) of one reference-layout q4_0 row against S q8_0 rows (in
// LDS), exactly as the AVX2 build computes it. Thread t of a 32-thread group plays
// float lane l = t & 7 of accumulator a = t >> 3. Lane l of a block is elements
// 4l..4l+3: the low nibbles of bytes 4l..4l+3 for l < 4, the high nibbles of bytes
// 4(l-4).. for l >= 4 (the two 128-bit halves of the unpacked block). Block b = 4i + a
// of the main loop (while b + 3 < nb) is fma(d_w * d_x, <q, x> - 8 * sum(x), acc_a);
// the tail blocks go to accumulator 0 after it. The reduction is the reference's:
// per lane (a0 + a1) + (a2 + a3), then lo + hi halves, movehl, shuffle, that is
// ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)). Each xor partner computes the
// same sum (float addition commutes), so every thread of the group returns the dot.
template <int S>
__device__ __forceinline__ void zz_q40_dot_avx(const uint8_t *row, int nb, const int8_t *xq, const float *xs, int D,
                                               int t, float (&out)[S]) {
    const int l = t & 7, a = t >> 3, nfull = nb >> 2;
    float acc[S];
#pragma unroll
    for (int s = 0; s < S; s++) acc[s] = 0.0f;
    auto step = [&](int b) {
        const uint8_t *bp = row + (size_t)18 * b;
        const float dw = zz_h2f(*(const uint16_t *)bp);
        const unsigned lo = *(const uint16_t *)(bp + 2 + 4 * (l & 3));
        const unsigned hi = *(const uint16_t *)(bp + 4 + 4 * (l & 3));
        const unsigned w = lo | (hi << 16);
        const int q = (int)((l < 4 ? w : w >> 4) & 0x0F0F0F0Fu);     // 4 nibbles, 0..15
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int x4 = *(const int *)(xq + (size_t)s * D + 32 * b + 4 * l);
            const int p = zz_dot4(q, x4, 0) - 8 * zz_dot4(0x01010101, x4, 0);
            acc[s] = fmaf(dw * xs[s * nb + b], (float)p, acc[s]);
        }
    };
#pragma unroll 4
    for (int i = 0; i < nfull; i++) step(4 * i + a);
    if (a == 0)
        for (int b = 4 * nfull; b < nb; b++) step(b);
#pragma unroll
    for (int s = 0; s < S; s++) {
        float v = acc[s];
        v = v + __shfl_xor(v, 8, 64);            // a0 + a1, a2 + a3
        v = v + __shfl_xor(v, 16, 64);           // (a0 + a1) + (a2 + a3)
        v = v + __shfl_xor(v, 4, 64);            // lanes l and l + 4
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 1, 64);
        out[s] = v;
    }
}

// the q8_0 rows of xn into LDS: S*D codes, then S*nb scales
__device__ __forceinline__ void zz_fl_stage(const ZzFlashArgs &a, int s0, int S, int8_t *xq, float *xs) {
    const int D = a.D, nb = D / ZZ_BLK;
    for (int i = threadIdx.x; i < S * D / 4; i += blockDim.x)
        ((int *)xq)[i] = ((const int *)(a.xq + (size_t)s0 * D))[i];
    for (int i = threadIdx.x; i < S * nb; i += blockDim.x) xs[i] = a.xs[(size_t)s0 * nb + i];
    __syncthreads();
}

// fsim[s][c] = centroid c . xq[s] (times cluster_scale[c] when not folded in),
// gemma4.c:1062-1071
// The workgroup's 8 centroid rows are contiguous: copied into LDS with 16-byte loads
// first. The same launch fills logits[S][V] with -inf when they are wanted (the probe
// kernel, which follows, writes the candidates').
template <int S>
__global__ __launch_bounds__(256) void zz_flash_sim_kernel(ZzFlashArgs a, int S_rows) {
    extern __shared__ __attribute__((aligned(16))) char fl_lds[];
    const int D = a.D, nb = D / ZZ_BLK, rb = 18 * nb, tid = threadIdx.x;
    if (a.logits) {
        const size_t n = (size_t)S_rows * a.V;
        for (size_t i = (size_t)blockIdx.x * 256 + tid; i < n; i += (size_t)gridDim.x * 256) a.logits[i] = -INFINITY;
    }
    int8_t *xq = (int8_t *)fl_lds;
    float *xs = (float *)(fl_lds + S * D);
    uint8_t *rows = (uint8_t *)(fl_lds + S * D + 4 * S * nb);
    const int c0 = blockIdx.x * FL_ROWS, nr = min(FL_ROWS, a.NC - c0);
    const uint4 *src = (const uint4 *)(a.cent + (size_t)c0 * rb);
    for (int k = tid; k < nr * rb / 16; k += 256) ((uint4 *)rows)[k] = src[k];
    zz_fl_stage(a, 0, S, xq, xs);                // its barrier also completes the rows
    const int t = tid & 31, g = tid >> 5, c = c0 + g;
    if (c >= a.NC) return;                       // whole 32-thread groups
    float d[S];
    zz_q40_dot_avx<S>(rows + (size_t)g * rb, nb, xq, xs, D, t, d);
    if (t == 0) {
        const float sc = a.scaled ? 1.0f : a.cscale[c];
#pragma unroll
        for (int s = 0; s < S; s++) a.fsim[(size_t)s * a.NC + c] = a.scaled ? d[s] : d[s] * sc;
    }
}

// exclusive prefix sum over the 1024 threads of a workgroup
__device__ __forceinline__ int zz_fl_scan1024(int v, int *wsum) {
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int n = __shfl_up(x, off, 64);
        if (l >= off) x += n;
    }
    if (l == 63) wsum[w] = x;
    __syncthreads();
    int base = 0;
    for (int q = 0; q < w; q++) base += wsum[q];
    __syncthreads();
    return base + x - v;
}

// The n_probes best clusters of row s into sel[s] (gemma4.c:1073-1074, 1112-1131).
// A radix select over the order-preserving bits of the scores (-0 folded into +0, so
// equal keys are equal floats) finds the boundary value T and how many scores equal
// it. If every score equal to T is needed, the set is fixed: the scores above T and
// those at T, written in cluster order. Otherwise the set depends on how the
// reference's quickselect breaks the tie, and thread 0 replays it: the same seeded
// LCG, pivot positions, partition and narrowing, over the index array in LDS. The
// replay is counted in diag[4].
__global__ __launch_bounds__(1024) void zz_flash_select_kernel(ZzFlashArgs a) {
    __shared__ float v[ZZ_FLASH_MAXNC];
    __shared__ int idx[ZZ_FLASH_MAXNC];
    __shared__ unsigned hist[16][256];           // one per wave: fewer colliding atomics
    __shared__ int wsum[16];
    __shared__ unsigned sh_prefix, sh_need, sh_eq;
    const int s = blockIdx.x, NC = a.NC, NP = a.NP, t = threadIdx.x;
    for (int i = t; i < NC; i += 1024) v[i] = a.fsim[(size_t)s * NC + i];
    unsigned prefix = 0u, mask = 0u, need = (unsigned)NP;
    for (int p = 3; p >= 0; p--) {
        const int sh = 8 * p;
        for (int i = t; i < 16 * 256; i += 1024) (&hist[0][0])[i] = 0u;
        __syncthreads();
        for (int i = t; i < NC; i += 1024) {
            const unsigned key = zz_fl_ord(v[i] + 0.0f);
            if ((key & mask) == prefix) atomicAdd(&hist[t >> 6][(key >> sh) & 255u], 1u);
        }
        __syncthreads();
        if (t < 64) {                            // the bin holding the need-th largest:
            unsigned h[4], loc = 0u;             // lane j has bins 255-4j .. 252-4j
#pragma unroll
            for (int r = 0; r < 4; r++) {
                h[r] = 0u;
                for (int w = 0; w < 16; w++) h[r] += hist[w][255 - 4 * t - r];
                loc += h[r];
            }
            unsigned x = loc;                    // scores in the bins above and in mine
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned n = __shfl_up(x, off, 64);
                if (t >= off) x += n;
            }
            unsigned above = x - loc;
            if (above < need && x >= need) {     // exactly one lane
                int r = 0;
                while (r < 3 && above + h[r] < need) above += h[r++];
                sh_prefix = prefix | ((unsigned)(255 - 4 * t - r) << sh);
                sh_need = need - above;
                sh_eq = h[r];
            }
        }
        __syncthreads();
        prefix = sh_prefix;
        mask |= 255u << sh;
        need = sh_need;
    }
    int *sel = a.sel + (size_t)s * NP;
    if (need == sh_eq) {                         // all scores equal to T are in
        const int per = (NC + 1023) / 1024, i0 = t * per, i1 = min(i0 + per, NC);
        int n = 0;
        for (int i = i0; i < i1; i++) n += zz_fl_ord(v[i] + 0.0f) >= prefix;
        int o = zz_fl_scan1024(n, wsum);
        for (int i = i0; i < i1; i++)
            if (zz_fl_ord(v[i] + 0.0f) >= prefix) idx[o++] = i;
        __syncthreads();
    } else {
        for (int i = t; i < NC; i += 1024) idx[i] = i;
        __syncthreads();
        if (t == 0) {
            unsigned long long g = 0x9e3779b97f4a7c15ULL;
            int lo = 0, hi = NC - 1, x;
            while (lo < hi) {
                g = g * 6364136223846793005ULL + 1442695040888963407ULL;
                const int pp = lo + (int)((g >> 33) % (unsigned long long)(hi - lo + 1));
                const float pv = v[idx[pp]];
                x = idx[pp]; idx[pp] = idx[hi]; idx[hi] = x;
                int st = lo;
                for (int i = lo; i < hi; i++)
                    if (v[idx[i]] > pv) { x = idx[i]; idx[i] = idx[st]; idx[st] = x; st++; }
                x = idx[st]; idx[st] = idx[hi]; idx[hi] = x;
                if (st == NP) break;
                if (st < NP) lo = st + 1;
                else hi = st - 1;
            }
            if (a.diag) atomicAdd(&a.diag[4], 1u);
        }
        __syncthreads();
    }
    for (int i = t; i < NP; i += 1024) sel[i] = idx[i];
}

// Candidate i of row s (blockIdx.y): member i % CS of the (i / CS)-th chosen cluster,
// then the forced ids (gemma4.c:1076-1085); padding (-1) and ids outside the
// vocabulary are skipped (gemma4.c:1094). Its logit,
// softcapped (gemma4.c:1103-1105), into logits[s][id] when logits is not null; the
// workgroup's best (logit, -id) key into part[s][blockIdx.x]. The workgroup's 8 rows
// are first copied into LDS with 16-byte loads (a q4_0 row of D % 64 == 0 is a whole
// number of 16-byte pieces), all of them in flight at once.
__global__ __launch_bounds__(256) void zz_flash_probe_kernel(ZzFlashArgs a) {
    extern __shared__ __attribute__((aligned(16))) char fl_lds[];
    __shared__ unsigned long long wkey[4];
    __shared__ int ids[FL_ROWS];
    const int D = a.D, nb = D / ZZ_BLK, s = blockIdx.y, tid = threadIdx.x, t = tid & 31;
    const int rb = 18 * nb, r16 = rb / 16;
    int8_t *xq = (int8_t *)fl_lds;
    float *xs = (float *)(fl_lds + D);
    uint8_t *rows = (uint8_t *)(fl_lds + D + 4 * nb);
    if (tid < FL_ROWS) {
        const int i = blockIdx.x * FL_ROWS + tid, nc = a.NP * a.CS;
        int id = -1;
        if (i < nc) {
            const int c = a.sel[(size_t)s * a.NP + i / a.CS];
            if (c >= 0 && c < a.NC) id = a.tmap[(size_t)c * a.CS + i % a.CS];
        } else if (i < nc + a.nforce) {
            id = a.force[i - nc];
        }
        ids[tid] = id >= 0 && id < a.V ? id : -1;    // padding and out-of-range ids: none
    }
    __syncthreads();
    for (int k = tid; k < FL_ROWS * r16; k += 256) {
        const int g = k / r16, id = ids[g];
        if (id >= 0) ((uint4 *)rows)[k] = ((const uint4 *)(a.rtab + (size_t)id * rb))[k - g * r16];
    }
    zz_fl_stage(a, s, 1, xq, xs);                // its barrier also completes the rows
    const int g = tid >> 5, id = ids[g];
    unsigned long long key = 0ull;
    if (id >= 0) {                               // the same id across the 32-thread group
        float d[1];
        zz_q40_dot_avx<1>(rows + (size_t)g * rb, nb, xq, xs, D, t, d);
        const float lg = a.cap > 0.0f ? tanhf(d[0] / a.cap) * a.cap : d[0];
        if (t == 0 && a.logits) a.logits[(size_t)s * a.V + id] = lg;
        key = ((unsigned long long)zz_fl_ord(lg) << 32) | (0xffffffffu - (unsigned)id);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long k2 = __shfl_xor(key, m, 64);
        key = k2 > key ? k2 : key;
    }
    if ((tid & 63) == 0) wkey[tid >> 6] = key;
    __syncthreads();
    if (tid == 0) {
        for (int q = 1; q < 4; q++) key = wkey[q] > key ? wkey[q] : key;
        a.part[(size_t)s * gridDim.x + blockIdx.x] = key;
    }
}

// The slot-table lane order (zz_common.h) of a q4_0 [V, D] table back to the
// reference layout (q40.h:9-18): one thread per (row, block) gathers the row's four
// lane words and its scale. Nibble k of the row sits in lane word k / 8, byte k % 4,
// low half for k % 8 < 4, stored as q ^ 8.
__global__ __launch_bounds__(256) void zz_flash_unpack_kernel(const uint8_t *src, ZzTensor T, uint8_t *dst) {
    const int nb = T.I / ZZ_BLK;
    const long long n = (long long)T.O * nb;
    for (long long j = (long long)blockIdx.x * 256 + threadIdx.x; j < n; j += (long long)gridDim.x * 256) {
        const int row = (int)(j / nb), b = (int)(j % nb), g = row >> 4, r = row & 15;
        unsigned wq[4];
#pragma unroll
        for (int qq = 0; qq < 4; qq++) wq[qq] = *(const unsigned *)(src + zz_qlane(T, g, b, 16 * qq + r));
        uint8_t *o = dst + (size_t)row * 18 * nb + (size_t)18 * b;
        const uint16_t sc = *(const uint16_t *)(src + zz_sidx(T, g, b, r));
        o[0] = (uint8_t)(sc & 0xff);
        o[1] = (uint8_t)(sc >> 8);
#pragma unroll
        for (int m = 0; m < 16; m++) {           // byte m: nibble m | nibble m + 16 << 4
            unsigned nib[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int k = m + 16 * h, word = k >> 3, kk = k & 7;
                const unsigned by = (wq[word] >> (8 * (kk & 3))) & 0xffu;
                nib[h] = ((kk < 4 ? by : by >> 4) & 15u) ^ 8u;
            }
            o[2 + m] = (uint8_t)(nib[0] | (nib[1] << 4));
        }
    }
}

// ------------------------------------------------------------------ launchers
int zz_launch_flash_unpack(const uint8_t *src, const ZzTensor &T, uint8_t *dst, hipStream_t st) {
    const long long n = (long long)T.O * (T.I / ZZ_BLK);
    const unsigned g = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    hipLaunchKernelGGL(zz_flash_unpack_kernel, dim3(g), dim3(256), 0, st, src, T, dst);
    return hipGetLastError() == hipSuccess;
}

int zz_flash_probe_groups(const ZzFlashArgs &a) {
    return (a.NP * a.CS + a.nforce + FL_ROWS - 1) / FL_ROWS;
}

int zz_launch_flash(const ZzFlashArgs &a, int S, hipStream_t st) {
    const int nb = a.D / ZZ_BLK;
    const dim3 gs((a.NC + FL_ROWS - 1) / FL_ROWS);
    const size_t lds = (size_t)S * a.D + sizeof(float) * (size_t)S * nb + (size_t)FL_ROWS * 18 * nb;
    switch (S) {
    case 1: hipLaunchKernelGGL(zz_flash_sim_kernel<1>, gs, dim3(256), lds, st, a, S); break;
    case 2: hipLaunchKernelGGL(zz_flash_sim_kernel<2>, gs, dim3(256), lds, st, a, S); break;
    case 3: hipLaunchKernelGGL(zz_flash_sim_kernel<3>, gs, dim3(256), lds, st, a, S); break;
    default: hipLaunchKernelGGL(zz_flash_sim_kernel<4>, gs, dim3(256), lds, st, a, S); break;
    }
    hipLaunchKernelGGL(zz_flash_select_kernel, dim3(S), dim3(1024), 0, st, a);
    hipLaunchKernelGGL(zz_flash_probe_kernel, dim3(zz_flash_probe_groups(a), S), dim3(256),
                       (size_t)a.D + sizeof(float) * nb + (size_t)FL_ROWS * 18 * nb, st, a);
    return hipGetLastError() == hipSuccess;
}
