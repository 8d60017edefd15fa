// zz_mma_up.hip -- the gate/up half of the grouped expert FFN on the int8 matrix
// cores: gate and up rows x the item's tokens, the activation, and the q8_0
// quantisation of the hidden (zz_mma.h holds the shared K loops).
#include "zz_mma.h"

// ------------------------------------------------------------------ up
union MmUpShared {
    MmStage st[2];
    Mm4Shared t4;
    struct {
        float u[32][MM_TN + 1];              // up values, [hidden row][token]
        float amax[2][MM_TN];
        int qsum[2][MM_TN];
    } e;
};

// GF, UF: the gate and up formats (gate and up are both tq2 or neither)
template <int GF, int UF, int NT, bool DBG>
__device__ __forceinline__ void mm_up_body(const ZzFfnArgs &a, const ZzItem &item, int rb, MmUpShared &sm,
                                           int *tok) {
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, qq = l >> 4;
    const ZzTensor &T = w < 2 ? a.lay.gate : a.lay.up;
    const int g = 2 * rb + (w & 1), n = item.n, D = a.D, nb = D / ZZ_BLK;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    if (tid < MM_TN) tok[tid] = a.ptok[item.p0 + min(tid, n - 1)];
    __syncthreads();
    MmSrc src;
    src.xb = (const uint8_t *)a.xq;
    src.sb = (const uint8_t *)a.xs;
#pragma unroll
    for (int k = 0; k < MM_XP; k++) {
        const int i = tid + 256 * k, t = i >> 3;
        src.row[k] = (uint32_t)tok[t] * (uint32_t)D;     // tok[t >= n]: token n - 1
        src.seg[k] = i & 7;
    }
#pragma unroll
    for (int k = 0; k < MM_SP; k++) {
        const int i = tid + 256 * k, t = i % MM_TN;
        src.srow[k] = (uint32_t)tok[t] * (uint32_t)(4 * nb);
        src.kb[k] = i / MM_TN;
    }

    // gate and up may differ in format (q4_0 / q8_0); each wave runs its tensor's loop
    // (the same number of chunks and barriers either way)
    // lane l, tile t, VGPR i: row 16g + 4qq + i of the wave's tensor, token 16t + l%16
    auto dbgc = [&](int c, int j, const zz_v4i (&rr)[NT]) {
        if constexpr (DBG) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (16 * t + (l & 15) < n)
                        mm_dbg_up(a, item.p0 + 16 * t + (l & 15), w < 2 ? 0 : 1, 16 * g + 4 * qq + i, 4 * c + j, rr[t][i]);
        }
    };
    float acc[NT][4];
    float alr[4] = {1.0f, 1.0f, 1.0f, 1.0f};     // tq2.h:154, alpha of the row: read now,
    if (GF == ZZ_FMT_TQ2)                        // used after the K loop
#pragma unroll
        for (int i = 0; i < 4; i++) alr[i] = ((const float *)(E + T.off_s))[16 * g + 4 * qq + i];
    if (GF == UF || w < 2) mm_kloop<GF, NT, MM_RING(NT)>(E, T, g, src, sm.st, acc, dbgc);
    else mm_kloop<UF, NT, MM_RING(NT)>(E, T, g, src, sm.st, acc, dbgc);
    if ((w < 2 ? GF : UF) == ZZ_FMT_Q40)         // the 16*(q - 8) weights
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] *= 0.0625f;
    if (GF == ZZ_FMT_TQ2) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t][i] *= alr[i];
    }
    __syncthreads();                             // the stages are done with
    if (w >= 2) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) sm.e.u[16 * (w & 1) + 4 * qq + i][16 * t + (l & 15)] = acc[t][i];
    }
    __syncthreads();
    // waves 0, 1: h = act(g, u) for hidden rows 16w + 4qq + i, then the q8_0
    // quantisation of each token's 32-row block (q40.h:124-138)
    float amx[NT];
    if (w < 2) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float h = zz_act(a.act, acc[t][i], sm.e.u[16 * w + 4 * qq + i][16 * t + (l & 15)], a.clamp);
                acc[t][i] = h;
                m = fmaxf(m, fabsf(h));
            }
            m = zz_rows_max(m);
            amx[t] = m;
            if (qq == 0) sm.e.amax[w][16 * t + l] = m;
        }
    }
    __syncthreads();
    if (w < 2) {
        const int nbM = a.MI / ZZ_BLK;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int tk = 16 * t + (l & 15);
            const float amax = fmaxf(amx[t], sm.e.amax[w ^ 1][tk]);
            const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            unsigned pk = 0;
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float f = rintf(acc[t][i] * id);
                f = fminf(fmaxf(f, -127.0f), 127.0f);
                const int qi = (int)f;
                s += qi;
                pk |= (unsigned)(qi & 0xff) << (8 * i);
            }
            s = zz_rows_sum(s);
            if (qq == 0) sm.e.qsum[w][tk] = s;
            if (tk < n) {
                const size_t p = (size_t)item.p0 + tk;
                *(unsigned *)(a.hq + p * a.MI + rb * ZZ_BLK + 16 * w + 4 * qq) = pk;
                if (w == 0 && qq == 0) a.hs[p * nbM + rb] = d;
            }
        }
    }
    __syncthreads();
    if (tid < n) a.hsum[((size_t)item.p0 + tid) * (a.MI / ZZ_BLK) + rb] = sm.e.qsum[0][tid] + sm.e.qsum[1][tid];
}

// Tiny items (<= 4 NS tokens): lanes 0..31 own gate rows 32rb.., lanes 32..63 the up
// rows (gate and up in one format); then h = act(g, u) and its q8_0 quantisation per
// token.
template <int FMT, int NS, bool DBG>
__device__ __forceinline__ void mm4_up_body(const ZzFfnArgs &a, const ZzItem &item, int rb, Mm4Shared &sm) {
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, n = item.n, D = a.D, nb = D / ZZ_BLK;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    const int *ptok = a.ptok + item.p0;
    const ZzTensor &T = l < 32 ? a.lay.gate : a.lay.up;
    Mm4Ring<FMT> R;
    mm4_first<FMT>(R, E, T, 2 * rb + ((l >> 4) & 1), l, w);       // weights first
    mm4_stage<NS>(sm.st, [&](int t) { return a.xq + (size_t)ptok[min(t, n - 1)] * D; },
                  [&](int t) { return a.xs + (size_t)ptok[min(t, n - 1)] * nb; }, D);
    // lane l, set s, VGPR v: weight row R = 4(l/4) + v of the 64 (lane R's row: gate
    // rows 32rb.. for R < 32, up rows 32rb.. for R >= 32), token 4s + l%4
    auto dbg = [&](int c, int j, const zz_v4i (&d)[NS]) {
        if constexpr (DBG) {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int R = 4 * (l >> 2) + v, t = 4 * s + (l & 3);
                    if (t < n) mm_dbg_up(a, item.p0 + t, R < 32 ? 0 : 1, 32 * rb + (R & 31), 4 * c + j, d[s][v]);
                }
        }
    };
    float acc[NS][4];
    mm4_kloop<FMT, NS>(R, E, l, w, sm.st, D, acc, dbg);
    __syncthreads();                             // the stage is done with
#pragma unroll
    for (int s = 0; s < NS; s++) mm4_reduce(sm.rd, acc[s], s);
    if (tid < 4 * NS * ZZ_BLK) {                 // token t, hidden row 32rb + r
        const int t = tid >> 5, r = tid & 31;
        sm.hb[t][r] = zz_act(a.act, sm.rd.res[r][t], sm.rd.res[32 + r][t], a.clamp);
    }
    __syncthreads();
    if (tid < 32 * NS) {                         // q8_0 of each token's block (q40.h:124-138)
        const int t = tid >> 3, m = tid & 7;
        float d;
        int qs;
        const unsigned pk = zz_quant8(*(const float4 *)&sm.hb[t][4 * m], &d, &qs);
        if (t < n) {
            const size_t p = (size_t)item.p0 + t;
            const int nbM = a.MI / ZZ_BLK;
            *(unsigned *)(a.hq + p * a.MI + rb * ZZ_BLK + 4 * m) = pk;
            if (m == 0) {
                a.hs[p * nbM + rb] = d;
                a.hsum[p * nbM + rb] = qs;
            }
        }
    }
}

template <int GF, int UF, bool DBG>
__global__ __launch_bounds__(256, 4) void zz_up_mma_kernel(ZzFfnArgs a) {
    int it, rb;
    zz_xcd_tile(a.MI / 32, &it, &rb);
    if (it >= a.meta[1]) return;
    const ZzItem item = a.items[it];
    if (item.n <= 0) return;
    __shared__ MmUpShared sm;
    __shared__ int tok[MM_TN];
    const int nt = (item.n + 15) / 16;
    if (GF == UF && GF != ZZ_FMT_TQ2 && item.n <= 4 && a.D <= MM4_K1) mm4_up_body<GF, 1, DBG>(a, item, rb, sm.t4);
    else if (GF == UF && GF == ZZ_FMT_Q40 && item.n <= 8 && a.D <= MM4_K2) mm4_up_body<GF, 2, DBG>(a, item, rb, sm.t4);
    else if (nt <= 1) mm_up_body<GF, UF, 1, DBG>(a, item, rb, sm, tok);
    else if (nt <= 2) mm_up_body<GF, UF, 2, DBG>(a, item, rb, sm, tok);
    else if (nt <= 3) mm_up_body<GF, UF, 3, DBG>(a, item, rb, sm, tok);
    else mm_up_body<GF, UF, 4, DBG>(a, item, rb, sm, tok);
}

template <bool DBG>
static void zz_up_mfma(const ZzFfnArgs &a, dim3 g, hipStream_t st) {
    const int gf = a.lay.gate.fmt, uf = a.lay.up.fmt;
    if (gf == ZZ_FMT_TQ2) hipLaunchKernelGGL((zz_up_mma_kernel<ZZ_FMT_TQ2, ZZ_FMT_TQ2, DBG>), g, dim3(256), 0, st, a);
    else if (gf == ZZ_FMT_Q40 && uf == ZZ_FMT_Q40) hipLaunchKernelGGL((zz_up_mma_kernel<ZZ_FMT_Q40, ZZ_FMT_Q40, DBG>), g, dim3(256), 0, st, a);
    else if (gf == ZZ_FMT_Q80 && uf == ZZ_FMT_Q80) hipLaunchKernelGGL((zz_up_mma_kernel<ZZ_FMT_Q80, ZZ_FMT_Q80, DBG>), g, dim3(256), 0, st, a);
    else if (gf == ZZ_FMT_Q40) hipLaunchKernelGGL((zz_up_mma_kernel<ZZ_FMT_Q40, ZZ_FMT_Q80, DBG>), g, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((zz_up_mma_kernel<ZZ_FMT_Q80, ZZ_FMT_Q40, DBG>), g, dim3(256), 0, st, a);
}

int zz_launch_up_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    const dim3 g(zz_xcd_grid(max_items, a.MI / 32));
    if (a.dbg_up) zz_up_mfma<true>(a, g, st);
    else zz_up_mfma<false>(a, g, st);
    return hipGetLastError() == hipSuccess;
}
