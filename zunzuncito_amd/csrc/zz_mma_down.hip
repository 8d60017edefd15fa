// zz_mma_down.hip -- the down half of the grouped expert FFN on the int8 matrix
// cores: the unweighted expert outputs y of each pair, stored at its flat index
// token*K + slot so that the combine reads a token's K rows without a lookup
// (zz_mma.h holds the shared K loops).
#include "zz_mma.h"

// ------------------------------------------------------------------ down
union MmDownShared {
    MmStage st[2];
    Mm4Shared t4;
};

// yrow[t]: the flat pair (token*K + slot) of the item's token t, the row of y that the
// combine reads for that token and slot
template <int FMT, int NT, bool DBG>
__device__ __forceinline__ void mm_down_body(const ZzFfnArgs &a, const ZzItem &item, int rt, MmDownShared &sm,
                                             const int *yrow) {
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, qq = l >> 4;
    const ZzTensor &T = a.lay.down;
    const int g = 4 * rt + w, n = item.n, MI = a.MI, nb = MI / ZZ_BLK;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    MmSrc src;
    src.xb = (const uint8_t *)a.hq;
    src.sb = (const uint8_t *)a.hs;
#pragma unroll
    for (int k = 0; k < MM_XP; k++) {
        const int i = tid + 256 * k, t = i >> 3;
        src.row[k] = (uint32_t)(item.p0 + min(t, n - 1)) * (uint32_t)MI;
        src.seg[k] = i & 7;
    }
#pragma unroll
    for (int k = 0; k < MM_SP; k++) {
        const int i = tid + 256 * k, t = i % MM_TN;
        src.srow[k] = (uint32_t)(item.p0 + min(t, n - 1)) * (uint32_t)(4 * nb);
        src.kb[k] = i / MM_TN;
    }

    auto dbgc = [&](int c, int j, const zz_v4i (&rr)[NT]) {
        if constexpr (DBG) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (16 * t + (l & 15) < n)
                        mm_dbg_dn(a, item.p0 + 16 * t + (l & 15), 16 * g + 4 * qq + i, 4 * c + j, rr[t][i]);
        }
    };
    float acc[NT][4];
    const int row0 = 16 * g + 4 * qq;
    float al[4] = {1.0f, 1.0f, 1.0f, 1.0f};     // tq2's row alpha: read now, used at the end
    if (FMT == ZZ_FMT_TQ2)
#pragma unroll
        for (int i = 0; i < 4; i++) al[i] = ((const float *)(E + T.off_s))[row0 + i];
    mm_kloop<FMT, NT, MM_RING(NT)>(E, T, g, src, sm.st, acc, dbgc);
    if (FMT == ZZ_FMT_Q40)                       // the 16*(q - 8) weights
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] *= 0.0625f;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tk = 16 * t + (l & 15);
        if (tk < n)
            *(float4 *)(a.y + (size_t)yrow[tk] * a.D + row0) =
                make_float4(acc[t][0] * al[0], acc[t][1] * al[1], acc[t][2] * al[2], acc[t][3] * al[3]);
    }
}

// Tiny items (<= 4 NS tokens), down: rows 64rt + l, the unweighted y of each token.
template <int FMT, int NS, bool DBG>
__device__ __forceinline__ void mm4_down_body(const ZzFfnArgs &a, const ZzItem &item, int rt, Mm4Shared &sm,
                                              const int *yrow) {
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63, n = item.n, MI = a.MI, nb = MI / ZZ_BLK;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    Mm4Ring<FMT> R;
    mm4_first<FMT>(R, E, a.lay.down, 4 * rt + (l >> 4), l, w);     // weights first
    mm4_stage<NS>(sm.st, [&](int t) { return a.hq + ((size_t)item.p0 + min(t, n - 1)) * MI; },
                  [&](int t) { return a.hs + ((size_t)item.p0 + min(t, n - 1)) * nb; }, MI);
    auto dbg = [&](int c, int j, const zz_v4i (&d)[NS]) {
        if constexpr (DBG) {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int t = 4 * s + (l & 3);
                    if (t < n) mm_dbg_dn(a, item.p0 + t, 64 * rt + 4 * (l >> 2) + v, 4 * c + j, d[s][v]);
                }
        }
    };
    float acc[NS][4];
    mm4_kloop<FMT, NS>(R, E, l, w, sm.st, MI, acc, dbg);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NS; s++) mm4_reduce(sm.rd, acc[s], s);
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int t = 4 * s + (tid >> 6), r = tid & 63;
        if (t < n) a.y[(size_t)yrow[t] * a.D + 64 * rt + r] = sm.rd.res[r][t];
    }
}

template <int FMT, bool DBG>
__global__ __launch_bounds__(256, 4) void zz_down_mma_kernel(ZzFfnArgs a) {
    int it, rt;
    zz_xcd_tile(a.D / 64, &it, &rt);
    if (it >= a.meta[1]) return;
    const ZzItem item = a.items[it];
    if (item.n <= 0) return;
    __shared__ MmDownShared sm;
    __shared__ int yrow[MM_TN];
    // read before the bodies' first barrier (the staging's), used after it
    if ((int)threadIdx.x < item.n) {
        const int p = item.p0 + (int)threadIdx.x;
        yrow[threadIdx.x] = a.ptok[p] * a.K + a.pslot[p];
    }
    const int nt = (item.n + 15) / 16;
    if (FMT != ZZ_FMT_TQ2 && item.n <= 4 && a.MI <= MM4_K1) mm4_down_body<FMT, 1, DBG>(a, item, rt, sm.t4, yrow);
    else if (FMT == ZZ_FMT_Q40 && item.n <= 8 && a.MI <= MM4_K2) mm4_down_body<FMT, 2, DBG>(a, item, rt, sm.t4, yrow);
    else if (nt <= 1) mm_down_body<FMT, 1, DBG>(a, item, rt, sm, yrow);
    else if (nt <= 2) mm_down_body<FMT, 2, DBG>(a, item, rt, sm, yrow);
    else if (nt <= 3) mm_down_body<FMT, 3, DBG>(a, item, rt, sm, yrow);
    else mm_down_body<FMT, 4, DBG>(a, item, rt, sm, yrow);
}

template <bool DBG>
static void zz_down_mfma(const ZzFfnArgs &a, dim3 g, hipStream_t st) {
    switch (a.lay.down.fmt) {
    case ZZ_FMT_Q40: hipLaunchKernelGGL((zz_down_mma_kernel<ZZ_FMT_Q40, DBG>), g, dim3(256), 0, st, a); break;
    case ZZ_FMT_Q80: hipLaunchKernelGGL((zz_down_mma_kernel<ZZ_FMT_Q80, DBG>), g, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((zz_down_mma_kernel<ZZ_FMT_TQ2, DBG>), g, dim3(256), 0, st, a); break;
    }
}

int zz_launch_down_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    const dim3 g(zz_xcd_grid(max_items, a.D / 64));
    if (a.dbg_dn) zz_down_mfma<true>(a, g, st);
    else zz_down_mfma<false>(a, g, st);
    return hipGetLastError() == hipSuccess;
}
