// zz_prefill.hip -- grouped expert FFN for many tokens per expert, on the int8
// matrix cores of gfx950 (v_mfma_i32_16x16x32_i8).
//
// One MFMA covers exactly one 32-weight block (K = 32), so its int32 results are
// the reference's per-block integer dots (q40.h:27 <q_w - 8, q_x>, q8_0's
// <q_w, q_x>, tq2's <c - 1, x>) and each is scaled by d_w[row,b] * d_x[token,b]
// into an fp32 accumulator, as the reference's per-block FMA does (q40.h:186).
//
// Work unit: (expert, up to 64 of its tokens) from the dispatch work list x a tile
// of weight rows. 4 waves; wave w owns 16 rows and all 64 tokens (4 MFMA tiles).
// The token activations of a K-chunk are staged in LDS; weight fragments come
// straight from the slot table, whose 16-row chunks are already in MFMA lane
// order (one 256/512-byte coalesced read per wave per block).
//   up:   rows rb*32..+31 of gate (waves 0,1) and of up (waves 2,3); then
//         h = act(g, u) and its per-token q8_0 quantisation, fused.
//   down: rows rt*64..+63 of down; unweighted y[pair][row] for the combine.
#include "zz_common.h"
#include "zz_kernels.h"

typedef int zz_v4i __attribute__((ext_vector_type(4)));

#define PF_TN 64       // tokens per work item
#define PF_KB 4        // 32-blocks per LDS stage
// LDS row stride of a staged token: 256 data bytes + 8, so the 16 tokens a
// quarter-wave reads (8 bytes each) fall on 16 distinct bank pairs
#define PF_XS (PF_KB * 32 + 8)

// Per-lane cursor over one weight row-group of a tensor: the A operand of
// v_mfma_i32_16x16x32_i8 (lane l: row l%16, k = 8*(l/16)..+7, signed int8) and the
// fp16 scales of the lane's 4 output rows (4*(l/16)..+3), one 32-block at a time.
template <int FMT>
struct ZzACursor {
    const uint8_t *q;          // payload of (row l%16, block 0)
    const uint8_t *s;          // scales of rows 4(l/16).., block 0
    __device__ __forceinline__ void init(const uint8_t *E, const ZzTensor &T, int g16, int l) {
        const int r = l & 15, qq = l >> 4;
        if (FMT == ZZ_FMT_Q80) q = E + zz_qoff(T, g16 * 16 + r, 0) + qq * 8;
        else q = E + zz_qoff(T, g16 * 16 + r, 0) + (qq & 1) * 8;
        s = FMT == ZZ_FMT_TQ2 ? nullptr : E + zz_soff(T, g16 * 16 + 4 * qq, 0);
    }
    // chunk stride in bytes between consecutive blocks (or tq2 groups)
    static constexpr int QSTEP = 16 * (FMT == ZZ_FMT_Q80 ? 32 : 16);
    __device__ __forceinline__ long frag(int b, int l) const {
        const int qq = l >> 4;
        if (FMT == ZZ_FMT_Q80) {
            const uint2 v = *(const uint2 *)(q + (size_t)b * QSTEP);
            return (long)((unsigned long)v.x | ((unsigned long)v.y << 32));
        }
        if (FMT == ZZ_FMT_Q40) {
            // k 0..15 are the low nibbles of bytes 0..15, k 16..31 the high ones
            const uint2 v = *(const uint2 *)(q + (size_t)b * QSTEP);
            const unsigned sh = (qq >> 1) * 4;
            unsigned x = (v.x >> sh) & 0x0F0F0F0Fu, y = (v.y >> sh) & 0x0F0F0F0Fu;
            x = (x + 0x78787878u) ^ 0x80808080u;      // bytewise q - 8, no carries
            y = (y + 0x78787878u) ^ 0x80808080u;
            return (long)((unsigned long)x | ((unsigned long)y << 32));
        }
        // tq2: block b is half b&1 of group b/2; k 0..15 of a half are bit plane
        // 2*(b&1), k 16..31 plane 2*(b&1)+1, byte k%16 (tq2.h:46-51)
        const uint2 v = *(const uint2 *)(q + (size_t)(b >> 1) * QSTEP);
        const unsigned sh = 2 * (2 * (b & 1) + (qq >> 1));
        unsigned x = (v.x >> sh) & 0x03030303u, y = (v.y >> sh) & 0x03030303u;
        x = (x + 0x7F7F7F7Fu) ^ 0x80808080u;          // bytewise c - 1
        y = (y + 0x7F7F7F7Fu) ^ 0x80808080u;
        return (long)((unsigned long)x | ((unsigned long)y << 32));
    }
    __device__ __forceinline__ uint2 scale(int b) const {
        if (FMT == ZZ_FMT_TQ2) return make_uint2(0x3c003c00u, 0x3c003c00u);   // 1.0
        return *(const uint2 *)(s + (size_t)b * 32);
    }
};

struct ZzStage {
    int8_t x[PF_TN][PF_XS];
    float s[PF_KB][PF_TN];
};

// Token activations of one K-chunk held in registers before they go to LDS.
// Thread tid always moves the same (token, 8-byte piece) slots, so its source
// offsets are computed once per work item.
#define PF_PIECES (PF_TN * PF_KB * 4 / 256)    // 8-byte pieces per thread
#define PF_SCALES (PF_TN * PF_KB / 256)
struct ZzBChunk {
    uint2 v[PF_PIECES];
    float s[PF_SCALES];
};

struct ZzBSrc {
    const int8_t *xq;           // int8 rows of the item's tokens live here
    const float *xs;            // and their block scales here
    int off[PF_PIECES];         // byte offset of the slot's row, or -1 (padding)
    int soff[PF_SCALES];        // scale offset of the slot's row, or -1
};

template <typename RowF>
__device__ __forceinline__ void zz_bsrc_init(ZzBSrc &b, const int8_t *xq, const float *xs, int n,
                                             int row_bytes, int row_scales, RowF row) {
    const int tid = threadIdx.x;
    b.xq = xq;
    b.xs = xs;
#pragma unroll
    for (int k = 0; k < PF_PIECES; k++) {
        const int i = tid + 256 * k, t = i / (PF_KB * 4), piece = i % (PF_KB * 4);
        b.off[k] = t < n ? row(t) * row_bytes + piece * 8 : -1;
    }
#pragma unroll
    for (int k = 0; k < PF_SCALES; k++) {
        const int i = tid + 256 * k, t = i / PF_KB, kb = i % PF_KB;
        b.soff[k] = t < n ? row(t) * row_scales + kb : -1;
    }
}

__device__ __forceinline__ void zz_load_bchunk(const ZzBSrc &b, int b0, int kn, ZzBChunk &c) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < PF_PIECES; k++) {
        const int piece = (tid + 256 * k) % (PF_KB * 4);
        uint2 v = make_uint2(0, 0);
        if (b.off[k] >= 0 && piece < kn * 4) v = *(const uint2 *)(b.xq + b.off[k] + b0 * 32);
        c.v[k] = v;
    }
#pragma unroll
    for (int k = 0; k < PF_SCALES; k++) {
        const int kb = (tid + 256 * k) % PF_KB;
        c.s[k] = (b.soff[k] >= 0 && kb < kn) ? b.xs[b.soff[k] + b0] : 0.0f;
    }
}

__device__ __forceinline__ void zz_store_bchunk(const ZzBChunk &c, ZzStage &st) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < PF_PIECES; k++) {
        const int i = tid + 256 * k, t = i / (PF_KB * 4), piece = i % (PF_KB * 4);
        *(uint2 *)&st.x[t][piece * 8] = c.v[k];
    }
#pragma unroll
    for (int k = 0; k < PF_SCALES; k++) {
        const int i = tid + 256 * k;
        st.s[i % PF_KB][i / PF_KB] = c.s[k];
    }
}

// One 32-block on the matrix cores for NJ 16-token tiles: NJ MFMAs, then the
// per-block scaling acc += d_w * d_x * int32 (q40.h:186).
template <int NJ>
__device__ __forceinline__ void zz_mfma_block(const ZzStage &S, int kb, long fa, uint2 sa, int l,
                                              float (&acc)[4][4]) {
    const zz_v4i zero = {0, 0, 0, 0};
    long B[NJ];
    float sx[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        B[j] = *(const long *)&S.x[16 * j + (l & 15)][kb * 32 + 8 * (l >> 4)];
        sx[j] = S.s[kb][16 * j + (l & 15)];
    }
    zz_v4i r[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) r[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa, B[j], zero, 0, 0, 0);
    float dw[4];
    dw[0] = zz_h2f((uint16_t)(sa.x & 0xffff));
    dw[1] = zz_h2f((uint16_t)(sa.x >> 16));
    dw[2] = zz_h2f((uint16_t)(sa.y & 0xffff));
    dw[3] = zz_h2f((uint16_t)(sa.y >> 16));
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = fmaf(dw[i] * sx[j], (float)r[j][i], acc[j][i]);
}

// acc[j][i] = sum over blocks of d_w * d_x * int32 for (row 4(l/16)+i of the
// cursor's row-group, token 16j + l%16), activations from `src`. The next
// K-chunk's weight fragments and activations are fetched into registers while
// the current chunk runs (two LDS stages). NJ = number of 16-token tiles in use.
template <int FMT, int NJ>
__device__ __forceinline__ void zz_mfma_kloop(const ZzACursor<FMT> &A, int nb, int n,
                                              ZzStage (&st)[2], const ZzBSrc &src,
                                              float (&acc)[4][4]) {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = 0.0f;
    long fa[PF_KB], fn[PF_KB];
    uint2 sa[PF_KB], sn[PF_KB];
    ZzBChunk bn;
    int kn = min(PF_KB, nb);
#pragma unroll
    for (int kb = 0; kb < PF_KB; kb++)
        if (kb < kn) { fa[kb] = A.frag(kb, l); sa[kb] = A.scale(kb); }
    zz_load_bchunk(src, 0, kn, bn);
    zz_store_bchunk(bn, st[0]);
    __syncthreads();
    int buf = 0;
    for (int b0 = 0; b0 < nb; b0 += PF_KB) {
        const int b1 = b0 + PF_KB, kn1 = min(PF_KB, nb - b1);
        if (b1 < nb) {                            // prefetch the next chunk
            if (kn1 == PF_KB) {
#pragma unroll
                for (int kb = 0; kb < PF_KB; kb++) { fn[kb] = A.frag(b1 + kb, l); sn[kb] = A.scale(b1 + kb); }
            } else {
#pragma unroll
                for (int kb = 0; kb < PF_KB; kb++)
                    if (kb < kn1) { fn[kb] = A.frag(b1 + kb, l); sn[kb] = A.scale(b1 + kb); }
            }
            zz_load_bchunk(src, b1, kn1, bn);
        }
        const ZzStage &S = st[buf];
        if (kn == PF_KB) {                        // full chunk: straight-line code
#pragma unroll
            for (int kb = 0; kb < PF_KB; kb++) zz_mfma_block<NJ>(S, kb, fa[kb], sa[kb], l, acc);
        } else {
#pragma unroll
            for (int kb = 0; kb < PF_KB; kb++)
                if (kb < kn) zz_mfma_block<NJ>(S, kb, fa[kb], sa[kb], l, acc);
        }
        if (b1 < nb) {
            zz_store_bchunk(bn, st[buf ^ 1]);      // the other stage is free: read last round
#pragma unroll
            for (int kb = 0; kb < PF_KB; kb++) { fa[kb] = fn[kb]; sa[kb] = sn[kb]; }
            kn = kn1;
        }
        __syncthreads();
        buf ^= 1;
    }
}

template <int FMT>
__device__ __forceinline__ void zz_mfma_kloop_n(const ZzACursor<FMT> &A, int nb, int n,
                                                ZzStage (&st)[2], const ZzBSrc &src,
                                                float (&acc)[4][4]) {
    switch ((n + 15) / 16) {
    case 1: zz_mfma_kloop<FMT, 1>(A, nb, n, st, src, acc); break;
    case 2: zz_mfma_kloop<FMT, 2>(A, nb, n, st, src, acc); break;
    case 3: zz_mfma_kloop<FMT, 3>(A, nb, n, st, src, acc); break;
    default: zz_mfma_kloop<FMT, 4>(A, nb, n, st, src, acc); break;
    }
}

template <int FMT>
__device__ __forceinline__ void zz_up_body(const ZzFfnArgs &a, const ZzItem &item, int rb) {
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const ZzTensor &T = w < 2 ? a.lay.gate : a.lay.up;
    const int g16 = rb * 2 + (w & 1);
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    const int D = a.D, nb = D / ZZ_BLK, n = item.n;
    __shared__ union {
        ZzStage st[2];
        struct {
            float gu[64][PF_TN + 1];
            float h[PF_TN][ZZ_BLK + 1];
        } e;
    } sm;
    __shared__ int tok[PF_TN];
    if (tid < PF_TN) tok[tid] = tid < n ? a.ptok[item.p0 + tid] : 0;
    __syncthreads();
    ZzACursor<FMT> A;
    A.init(E, T, g16, l);
    float acc[4][4];
    ZzBSrc bs;
    zz_bsrc_init(bs, a.xq, a.xs, n, D, nb, [&](int t) { return tok[t]; });
    zz_mfma_kloop_n<FMT>(A, nb, n, sm.st, bs, acc);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rt = g16 * 16 + 4 * (l >> 4) + i;           // row of T
        const float alpha = FMT == ZZ_FMT_TQ2 ? ((const float *)(E + T.off_s))[rt] : 1.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) sm.e.gu[w * 16 + 4 * (l >> 4) + i][16 * j + (l & 15)] = acc[j][i] * alpha;
    }
    __syncthreads();
    // h = act(gate, up) for 32 rows x n tokens (gemma4.c:644, lfm25.c:714,
    // maple.c:672-675), then one thread per token quantises its 32-block
    for (int i = tid; i < n * ZZ_BLK; i += 256) {
        const int t = i / ZZ_BLK, r = i % ZZ_BLK;
        sm.e.h[t][r] = zz_act(a.act, sm.e.gu[r][t], sm.e.gu[32 + r][t], a.clamp);
    }
    __syncthreads();
    if (tid < n) {
        float v[ZZ_BLK];
#pragma unroll
        for (int r = 0; r < ZZ_BLK; r++) v[r] = sm.e.h[tid][r];
        const size_t p = (size_t)item.p0 + tid;
        const int nbM = a.MI / ZZ_BLK;
        int qs;
        const float d = zz_quant_block(v, a.hq + p * a.MI + rb * 32, &qs);
        a.hs[p * nbM + rb] = d;
        a.hsum[p * nbM + rb] = qs;
    }
}

template <int FMT>
__device__ __forceinline__ void zz_down_body(const ZzFfnArgs &a, const ZzItem &item, int rt) {
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const ZzTensor &T = a.lay.down;
    const int g16 = rt * 4 + w;
    const uint8_t *E = a.experts + (size_t)item.e * a.estride;
    const int MI = a.MI, nb = MI / ZZ_BLK, n = item.n;
    __shared__ ZzStage st[2];
    ZzACursor<FMT> A;
    A.init(E, T, g16, l);
    float acc[4][4];
    ZzBSrc bs;
    zz_bsrc_init(bs, a.hq + (size_t)item.p0 * MI, a.hs + (size_t)item.p0 * nb, n, MI, nb,
                 [&](int t) { return t; });
    zz_mfma_kloop_n<FMT>(A, nb, n, st, bs, acc);
    const int row0 = g16 * 16 + 4 * (l >> 4);
    float al[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (FMT == ZZ_FMT_TQ2)
        for (int i = 0; i < 4; i++) al[i] = ((const float *)(E + T.off_s))[row0 + i];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = 16 * j + (l & 15);
        if (t < n) {
            float4 v = make_float4(acc[j][0] * al[0], acc[j][1] * al[1], acc[j][2] * al[2], acc[j][3] * al[3]);
            *(float4 *)(a.y + ((size_t)item.p0 + t) * a.D + row0) = v;
        }
    }
}

// XCD-aware work order. Workgroup g of a launch runs on XCD g % 8 (round-robin
// dispatch), and each XCD has its own L2. All row tiles of one work item read the
// same activations, so they are given workgroup ids of one residue mod 8: the item
// stays in one L2 and its row tiles run back to back. Item i goes to XCD i % 8 as
// that XCD's (i / 8)-th item; ids past the last item exit.
#define ZZ_XCDS 8
__device__ __forceinline__ void zz_xcd_tile(int ntiles, int *item, int *tile) {
    const int g = blockIdx.x, x = g % ZZ_XCDS, k = g / ZZ_XCDS;
    *item = (k / ntiles) * ZZ_XCDS + x;
    *tile = k % ntiles;
}
__host__ __device__ inline unsigned zz_xcd_grid(int max_items, int ntiles) {
    return (unsigned)((max_items + ZZ_XCDS - 1) / ZZ_XCDS * ZZ_XCDS * ntiles);
}

// gate and up share one format in these instantiations (the host checks)
template <int FMT>
__global__ __launch_bounds__(256) void zz_up_mfma_kernel(ZzFfnArgs a) {
    int it, rb;
    zz_xcd_tile(a.MI / 32, &it, &rb);
    if (it >= a.meta[1]) return;
    zz_up_body<FMT>(a, a.items[it], rb);
}

template <int FMT>
__global__ __launch_bounds__(256) void zz_down_mfma_kernel(ZzFfnArgs a) {
    int it, rt;
    zz_xcd_tile(a.D / 64, &it, &rt);
    if (it >= a.meta[1]) return;
    zz_down_body<FMT>(a, a.items[it], rt);
}

int zz_launch_up_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    if (a.lay.gate.fmt != a.lay.up.fmt) return 0;
    dim3 g(zz_xcd_grid(max_items, a.MI / 32));
    switch (a.lay.gate.fmt) {
    case ZZ_FMT_Q40: hipLaunchKernelGGL(zz_up_mfma_kernel<ZZ_FMT_Q40>, g, dim3(256), 0, st, a); break;
    case ZZ_FMT_Q80: hipLaunchKernelGGL(zz_up_mfma_kernel<ZZ_FMT_Q80>, g, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(zz_up_mfma_kernel<ZZ_FMT_TQ2>, g, dim3(256), 0, st, a); break;
    }
    return hipGetLastError() == hipSuccess;
}

int zz_launch_down_mfma(const ZzFfnArgs &a, int max_items, hipStream_t st) {
    dim3 g(zz_xcd_grid(max_items, a.D / 64));
    switch (a.lay.down.fmt) {
    case ZZ_FMT_Q40: hipLaunchKernelGGL(zz_down_mfma_kernel<ZZ_FMT_Q40>, g, dim3(256), 0, st, a); break;
    case ZZ_FMT_Q80: hipLaunchKernelGGL(zz_down_mfma_kernel<ZZ_FMT_Q80>, g, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(zz_down_mfma_kernel<ZZ_FMT_TQ2>, g, dim3(256), 0, st, a); break;
    }
    return hipGetLastError() == hipSuccess;
}
