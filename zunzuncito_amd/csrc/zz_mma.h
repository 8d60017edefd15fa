// zz_mma.h -- the grouped expert FFN for batches (S >= 5) on the int8 matrix cores
// of gfx950 (v_mfma_i32_16x16x32_i8, v_mfma_i32_4x4x4_16b_i8): the K loops and
// fragment code shared by the gate/up kernel (zz_mma_up.hip) and the down kernel
// (zz_mma_down.hip).
//
// One MFMA step covers exactly one 32-weight block (K = 32), so its int32 results are
// the reference's per-block integer dots (q40.h:27 <q_w - 8, q_x>, q8_0's <q_w, q_x>,
// tq2's <c - 1, x>). Each is scaled by d_w[row,b] * d_x[token,b] into an fp32
// accumulator, as the reference's per-block FMA does (q40.h:186).
//
// Work unit: (item, tile). An item is one expert with up to 64 of its tokens (the
// dispatch work list); a tile is 64 weight rows: 4 waves x one 16-row group each.
// Every wave multiplies its rows by all of the item's tokens (up to 8 MFMA tiles of
// 16 tokens), so each weight fragment is loaded and unpacked once per item.
//   up:   hidden rows 32*rb..+31: waves 0, 1 the gate groups, waves 2, 3 the up
//         groups; then h = act(g, u) and its per-token q8_0 quantisation
//         (gemma4.c:642-645, lfm25.c:712-723, maple.c:665-684) in registers;
//   down: rows 64*rt..+63 of down; the unweighted y[token*K + slot][row] for the combine.
// The K loop walks the slot table's chunks of 4 blocks. Weights go straight to
// registers, two chunks ahead: the slot table holds each lane's bytes for a chunk
// contiguously (zz_common.h). Activations are staged through LDS, one chunk ahead.
#pragma once
#include "zz_common.h"
#include "zz_kernels.h"
#include "zz_dot_dev.h"
#include <type_traits>

typedef int zz_v4i __attribute__((ext_vector_type(4)));

#define MM_TN ZZ_MMA_TOKENS            // tokens per work item: 4 tiles of 16
#define MM_XP (8 * MM_TN / 256)        // 16-byte activation pieces per thread and chunk
#define MM_SP (4 * MM_TN / 256)        // activation scales per thread and chunk
// LDS row stride of a staged token: one 4-block chunk (128 bytes) + 8, so the 16
// tokens a quarter-wave reads fall on distinct banks
#define MM_XS (4 * ZZ_BLK + 8)

struct MmStage {
    __attribute__((aligned(16))) int8_t x[MM_TN][MM_XS];
    float s[4][MM_TN];               // block scales d_x, [block][token]
};

// One wave's weight operand for one chunk (4 blocks, or 2 in a short last chunk).
//   q4_0: q = the lane's 4 words (k 8qq..8qq+7 of each block, zz_common.h)
//   q8_0: q, q2 = the lane's 32 bytes
//   tq2:  q.xy, q.zw = 8 bytes of row r's 64-groups 2c, 2c+1 (bit planes)
// s0, s1: fp16 scales of rows 4qq..4qq+3, [row][block] (q4_0, q8_0).
struct MmA {
    uint4 q, q2, s0, s1;
};

template <int FMT>
__device__ __forceinline__ MmA mm_load_a(const uint8_t *E, const ZzTensor &T, const ZzWalk &W, int g, int c,
                                         int l) {
    const int r = l & 15, qq = l >> 4;
    const uint4 z = make_uint4(0, 0, 0, 0);
    MmA A = {z, z, z, z};
    if (FMT == ZZ_FMT_TQ2) {
        const int ng = T.I / 64, row = 16 * g + r;
        const uint2 v0 = *(const uint2 *)(E + zz_tq2off(T, row, 2 * c) + (qq & 1) * 8);
        const uint2 v1 = *(const uint2 *)(E + zz_tq2off(T, row, min(2 * c + 1, ng - 1)) + (qq & 1) * 8);
        A.q = make_uint4(v0.x, v0.y, v1.x, v1.y);
        return A;
    }
    // Branch-free: the same loads on every path (only addresses are selected), so
    // the compiler's load counters stay exact across the pipelined loops. A short
    // last chunk (2 blocks) has 8 (q4_0) or 16 (q8_0) bytes per lane and 4 scale
    // words per lane group; the extra bytes read stay inside the slot (the q plane
    // is followed by the scale plane) and belong to blocks the loop skips.
    const bool full = c < W.nfull;
    const uint32_t qo = zz_walk_qo(W, c), so = zz_walk_so(W, c);    // so: 16-byte aligned
    A.q = ld16(E + qo);
    if (FMT == ZZ_FMT_Q80) A.q2 = ld16(E + (qo + (full ? 16u : 0u)));
    A.s0 = ld16(E + so);
    A.s1 = ld16(E + (so + (full ? 16u : 0u)));
    return A;
}

// A fragment of block j (8 signed int8, k = 8qq..8qq+7 of the lane's row)
template <int FMT>
__device__ __forceinline__ long mm_frag(const MmA &A, int j, int l) {
    if (FMT == ZZ_FMT_Q80) {
        const uint4 v = j < 2 ? A.q : A.q2;
        const uint2 w = (j & 1) ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y);
        return (long)((unsigned long)w.x | ((unsigned long)w.y << 32));
    }
    if (FMT == ZZ_FMT_Q40) {
        // byte m of the word = nibble(8qq + m) | nibble(8qq + m + 4) << 4
        const unsigned w = j == 0 ? A.q.x : (j == 1 ? A.q.y : (j == 2 ? A.q.z : A.q.w));
        const uint2 u = zz_q4_unpack16(w);             // 16 * (q - 8)
        return (long)((unsigned long)u.x | ((unsigned long)u.y << 32));
    }
    // tq2: block j is half j&1 of group j/2; k 0..15 of a half are bit plane
    // 2*(j&1), k 16..31 plane 2*(j&1)+1, byte k%16 (tq2.h:46-51)
    const uint2 v = j < 2 ? make_uint2(A.q.x, A.q.y) : make_uint2(A.q.z, A.q.w);
    const unsigned sh = 2 * (2 * (j & 1) + ((l >> 4) >> 1));
    unsigned x = (v.x >> sh) & 0x03030303u, y = (v.y >> sh) & 0x03030303u;
    x = (x + 0x7F7F7F7Fu) ^ 0x80808080u;          // bytewise c - 1
    y = (y + 0x7F7F7F7Fu) ^ 0x80808080u;
    return (long)((unsigned long)x | ((unsigned long)y << 32));
}

// d_w of row 4qq+i, block j of the chunk, as fp16: halfword i*cbs + j of s0|s1
// (i, j and the chunk size compile-time, so this is a register and a half select).
template <bool FULL>
__device__ __forceinline__ _Float16 mm_dwh(const uint4 &s0, const uint4 &s1, int j, int i) {
    const int h = FULL ? 4 * i + j : 2 * i + j, w = h >> 1;
    const unsigned u = w == 0 ? s0.x : w == 1 ? s0.y : w == 2 ? s0.z : w == 3 ? s0.w
                     : w == 4 ? s1.x : w == 5 ? s1.y : w == 6 ? s1.z : s1.w;
    return __builtin_bit_cast(_Float16, (unsigned short)((h & 1) ? u >> 16 : u & 0xffff));
}

// One chunk: acc[t][i] += d_w * d_x * <w, x> for row 4qq+i of the wave's row group
// and token 16t + l%16, over the chunk's 4 (FULL) or 2 blocks. X(t, j) is the 8-byte
// B operand of token tile t, block j; SX(t, j) that token's d_x.
// Per product: d_w * d_x (a multiply by the block's d_w, converted once per block),
// the int32 conversion, the accumulating FMA.
// DF(j, r): called with block j's int32 results before their scaling (diagnostics
// builds store them; the timed build passes a hook that does nothing).
template <int FMT, int NT, bool FULL, typename XF, typename SF, typename DF>
__device__ __forceinline__ void mm_chunk(const MmA &A, int l, float (&acc)[NT][4], XF X, SF SX, DF dbg) {
    const zz_v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < (FULL ? 4 : 2); j++) {
        const long fa = mm_frag<FMT>(A, j, l);
        long B[NT];
        float sx[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            B[t] = X(t, j);
            sx[t] = SX(t, j);
        }
        // all tiles' products first, into distinct registers, so that each epilogue
        // finds its matrix-core result ready instead of waiting on it
        zz_v4i r[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) r[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa, B[t], zero, 0, 0, 0);
        dbg(j, r);
        // the 4 rows' d_w as f32 once per block, for every tile: the product d_w * d_x
        // is then a v_mul_f32, which ran the up kernel 3 % faster than the fused
        // mixed-precision form (v_fma_mix_f32) the compiler otherwise picks; the empty
        // asm keeps it from folding them back together. tq2 has no block scale (its
        // alpha is per row), and no asm: pinned, the constant 1 cost four moves a block.
        float dwf[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (FMT != ZZ_FMT_TQ2) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                dwf[i] = (float)mm_dwh<FULL>(A.s0, A.s1, j, i);
                asm volatile("" : "+v"(dwf[i]));
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float s = FMT == ZZ_FMT_TQ2 ? sx[t] : dwf[i] * sx[t];
                acc[t][i] = fmaf(s, (float)r[t][i], acc[t][i]);
            }
        }
        // three or four tiles: one block at a time (the next block's LDS reads hoisted
        // over this one would hold NT more operand registers); one or two tiles leave
        // the scheduler free to overlap them (0.5 us off each FFN kernel at S = 512)
        if (NT >= 3) __builtin_amdgcn_sched_barrier(0);
    }
}

// Activations of one chunk: a thread moves 4 16-byte pieces (token, segment) and
// two (token, block) scales per chunk, always the same slots.
struct MmX {
    uint4 v[MM_XP];
    float s[MM_SP];
};

// Rows are 32-bit byte offsets from uniform bases (the activation planes are far
// below 4 GB), so each load is a scalar base plus one lane offset.
struct MmSrc {
    const uint8_t *xb, *sb;          // the int8 activations and their f32 block scales
    uint32_t row[MM_XP];             // byte offset of each piece's token row
    uint32_t srow[MM_SP];            // byte offset of each scale slot's d_x row
    int seg[MM_XP], kb[MM_SP];
};

// No masks: padding tokens of an item read a real token's row (so their columns hold
// finite values that the epilogues never store), and the segments and scales of a
// short chunk's missing blocks are clamped into the row and never read back.
// KP pieces per thread cover tokens 0 .. 32KP-1 (16 NT <= 32 KP).
template <int KP>
__device__ __forceinline__ void mm_load_x(const MmSrc &src, int c, int cbs, MmX &x) {
#pragma unroll
    for (int k = 0; k < KP; k++)
        x.v[k] = ld16(src.xb + (src.row[k] + (uint32_t)(c * 4 * ZZ_BLK + 16 * min(src.seg[k], 2 * cbs - 1))));
#pragma unroll
    for (int k = 0; k < MM_SP; k++)
        x.s[k] = *(const float *)(src.sb + (src.srow[k] + (uint32_t)(4 * (4 * c + min(src.kb[k], cbs - 1)))));
}

template <int KP>
__device__ __forceinline__ void mm_store_x(const MmX &x, MmStage &st) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < KP; k++) {
        const int i = tid + 256 * k, t = i >> 3, seg = i & 7;
        uint2 *d = (uint2 *)&st.x[t][16 * seg];
        d[0] = make_uint2(x.v[k].x, x.v[k].y);
        d[1] = make_uint2(x.v[k].z, x.v[k].w);
    }
#pragma unroll
    for (int k = 0; k < MM_SP; k++) {
        const int i = tid + 256 * k;
        st.s[i / MM_TN][i % MM_TN] = x.s[k];
    }
}

// Weight chunks live in a ring of RING register sets with static indices (the loop
// body is unrolled RING times, so no register copies): chunk c + RING - 1 is
// requested at step c, RING - 1 steps before its use. The main loop runs whole
// rings of full chunks with every load unconditional (clamped past the end); the
// remaining chunks (fewer than RING + 1, the short one last) run in a tail.
//
// Large items: activations one chunk ahead through the two LDS stages, one
// workgroup barrier per chunk.
template <int FMT, int NT, int RING, typename DF>
__device__ __forceinline__ void mm_kloop(const uint8_t *E, const ZzTensor &T, int g, const MmSrc &src,
                                         MmStage (&st)[2], float (&acc)[NT][4], DF dbgc) {
    const int l = threadIdx.x & 63, nb = T.I / ZZ_BLK, nch = (nb + 3) / 4, nfull = nb / 4;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;
    constexpr int KP = (NT + 1) / 2 < MM_XP ? (NT + 1) / 2 : MM_XP;
    const ZzWalk W = zz_walk(T, g, l, 4 * (l >> 4));
    MmA r[RING];
#pragma unroll
    for (int i = 0; i < RING - 1; i++) r[i] = mm_load_a<FMT>(E, T, W, g, min(i, nch - 1), l);
    MmX xr;
    mm_load_x<KP>(src, 0, min(4, nb), xr);
    mm_store_x<KP>(xr, st[0]);
    // x of chunk c + 1 is requested before the weight prefetch: the wait for it at
    // the end of the step (loads complete in order) then leaves the prefetch in flight
    auto load_x = [&](int c) {
        const int c1 = min(c + 1, nch - 1);
        mm_load_x<KP>(src, c1, min(4, nb - 4 * c1), xr);
    };
    auto step = [&](int c, const MmA &A, auto full) {
        __syncthreads();                         // stage c%2 complete; stage (c+1)%2 free
        const MmStage &S = st[c & 1];
        mm_chunk<FMT, NT, decltype(full)::value>(
            A, l, acc, [&](int t, int j) { return *(const long *)&S.x[16 * t + (l & 15)][j * ZZ_BLK + 8 * (l >> 4)]; },
            [&](int t, int j) { return S.s[j][16 * t + (l & 15)]; },
            [&](int j, const zz_v4i (&rr)[NT]) { dbgc(c, j, rr); });
        mm_store_x<KP>(xr, st[(c + 1) & 1]);     // the last step refills the free stage: harmless
    };
    int c0 = 0;
    for (; c0 + RING <= nfull; c0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; u++) {
            load_x(c0 + u);
            r[(u + RING - 1) % RING] = mm_load_a<FMT>(E, T, W, g, min(c0 + u + RING - 1, nch - 1), l);
            step(c0 + u, r[u], std::true_type());
        }
    }
#pragma unroll
    for (int u = 0; u < RING; u++) {
        const int c = c0 + u;
        if (c < nch) {
            load_x(c);
            if (u == RING - 1) r[u] = mm_load_a<FMT>(E, T, W, g, c, l);
            if (c < nfull) step(c, r[u], std::true_type());
            else step(c, r[u], std::false_type());
        }
    }
}

#define MM_RING(NT) ((NT) <= 2 ? 4 : 3)

// ------------------------------------------------------------------ tiny items
// Items of <= 4 tokens (the long tail of experts under skewed routing) would fill a
// 16-token tile with padding. They run on v_mfma_i32_4x4x4_16b_i8 instead: its 16
// blocks are 16 row quads of the workgroup's 64 weight rows, its 4 columns the 4
// tokens. Lane l owns weight row l (the row's four lane-order pieces of a chunk) and,
// after the 8 steps of a 32-weight block, the block's int32 dots of rows 4(l/4)..+3
// with token l%4 (layout checked on the device: A lane 4b+i = row i of block b,
// B lane 4b+j = column j, D lane 4b+j, VGPR v = row v). The 4 waves split the K range
// by chunks (c = w, w+4, ...) and their partial sums meet in LDS. Per 32-weight block
// a lane spends 12 unpack and 12 epilogue operations for 64 rows x 4 tokens, where
// the 16x16x32 path spends 4 x 15 for 64 rows x 16 padded tokens. Items of 5-8 tokens
// take two token sets (NS = 2, q4_0; q8_0's twice-as-large weight registers would spill):
// the same weight operand feeds both sets' MFMAs, so a block costs 12 unpack and 24
// epilogue operations for 64 rows x 8 tokens.
// Staged rows are K + 16 bytes apart and scale rows K/32 + 1 words apart: at the
// unpadded strides (K a multiple of 128 bytes) every token's 16-byte read of block b
// would fall on the same LDS banks, a 4- or 8-way conflict per read.
#define MM4_K1 6144                      // K limit of one token set (4 rows)
#define MM4_K2 3072                      // K limit of two token sets (8 rows)
#define MM4_XB (8 * (MM4_K2 + 16))       // staged activation bytes (also >= 4 * (MM4_K1 + 16))
#define MM4_XS(K) ((K) + 16)
#define MM4_SS(K) ((K) / ZZ_BLK + 1)
struct Mm4Stage {
    __attribute__((aligned(16))) int8_t x[MM4_XB];      // token t's row at t * MM4_XS(K)
    float s[8 * MM4_SS(MM4_K2)];                       // token t's block scales at t * MM4_SS(K)
};
static_assert(4 * MM4_XS(MM4_K1) <= MM4_XB && 4 * MM4_SS(MM4_K1) <= 8 * MM4_SS(MM4_K2), "stage sizes");
struct Mm4Red {
    float part[4][64][4];                // [wave][lane][row of the quad]
    float res[64][9];                    // [row][token]
};

// The item's (up to) 4 * NS token rows and block scales, whole. row(t) / srow(t) for
// t < 4 * NS (callers clamp t to the item's last token).
template <int NS, typename RF, typename SF>
__device__ __forceinline__ void mm4_stage(Mm4Stage &st, RF row, SF srow, int K) {
    const int tid = threadIdx.x, nseg = K / 16, nb = K / ZZ_BLK;
    for (int i = tid; i < 4 * NS * nseg; i += 256) {
        const int t = i / nseg, sg = i - t * nseg;
        *(uint4 *)&st.x[t * MM4_XS(K) + 16 * sg] = ld16(row(t) + 16 * sg);
    }
    for (int i = tid; i < 4 * NS * nb; i += 256) {
        const int t = i / nb, b = i - t * nb;
        st.s[t * MM4_SS(K) + b] = srow(t)[b];
    }
    __syncthreads();
}

// A lane's chunk: its row's four pieces (q4_0 16 bytes each, q8_0 32) and the fp16
// scales of its row quad, rows 4((l>>2)&3)..+3 of its group.
struct Mm4A {
    uint4 q[4], q2[4], s0, s1;
};

template <int FMT>
__device__ __forceinline__ Mm4A mm4_load(const uint8_t *E, const ZzWalk &W, int c) {
    Mm4A A;
    const bool full = c < W.nfull;
    const uint8_t *q = zz_walk_q(E, W, c), *s = zz_walk_s(E, W, c);
    // piece qq of row r is lane 16qq + r of the chunk: 16 lanes of 4 (full) or 2
    // blocks' bytes further
    const int ps = 16 * (full ? 4 : 2) * (FMT == ZZ_FMT_Q80 ? 8 : 4);
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
        A.q[qq] = ld16(q + qq * ps);
        A.q2[qq] = FMT == ZZ_FMT_Q80 ? ld16(q + qq * ps + (full ? 16 : 0)) : make_uint4(0, 0, 0, 0);
    }
    A.s0 = ld16(s);
    A.s1 = ld16(s + (full ? 16 : 0));
    return A;
}

// the int8 operand of step m (k = 4m..4m+3) of block j: piece m/2, low (m even) or
// high half of its 8 weights
template <int FMT>
__device__ __forceinline__ int mm4_frag(const Mm4A &A, int j, int m) {
    const int qq = m >> 1;
    if (FMT == ZZ_FMT_Q80) {
        const uint4 v = j < 2 ? A.q[qq] : A.q2[qq];
        const unsigned w0 = (j & 1) ? v.z : v.x, w1 = (j & 1) ? v.w : v.y;
        return (int)((m & 1) ? w1 : w0);
    }
    const uint4 v = A.q[qq];
    const unsigned w = j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
    const uint2 u = zz_q4_unpack16(w);                 // 16 * (q - 8)
    return (int)((m & 1) ? u.y : u.x);
}

// acc[s][v]: row 4(l/4)+v of the 64, token 4s + l%4, over this wave's chunks c = w,
// w+4, ... (K: the row length; the staged rows are MM4_XS(K) apart)
template <int FMT, bool FULLC, int NS, typename DF>
__device__ __forceinline__ void mm4_chunk(const Mm4A &A, const Mm4Stage &st, int c, int l, int K,
                                          float (&acc)[NS][4], DF dbg) {
#pragma unroll
    for (int j = 0; j < (FULLC ? 4 : 2); j++) {
        const int b = 4 * c + j;
        zz_v4i d[NS];
        float sx[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int t = 4 * s + (l & 3);
            const int8_t *xr = &st.x[t * MM4_XS(K) + b * ZZ_BLK];
            const uint4 xa = *(const uint4 *)xr, xb = *(const uint4 *)(xr + 16);
            const unsigned xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            d[s] = (zz_v4i){0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 8; m++) d[s] = __builtin_amdgcn_mfma_i32_4x4x4i8(mm4_frag<FMT>(A, j, m), (int)xw[m], d[s], 0, 0, 0);
            sx[s] = st.s[t * MM4_SS(K) + b];
        }
        dbg(c, j, d);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float dw = (float)mm_dwh<FULLC>(A.s0, A.s1, j, v);
#pragma unroll
            for (int s = 0; s < NS; s++) acc[s][v] = fmaf(fmaf(dw, sx[s], 0.0f), (float)d[s][v], acc[s][v]);
        }
    }
}

// This wave's chunks c = w, w+4, ... of the tensor, in a ring of three register sets
// (two chunks in flight while one is multiplied; q8_0: two sets): the work per chunk
// is far shorter than a memory latency, so the depth of the ring sets the pace. The caller issues
// the first two chunks (mm4_first) before it stages the activations, so those loads
// overlap the staging.
template <int FMT>
struct Mm4Ring {
    ZzWalk W;
    int nch;
    Mm4A r0, r1, r2;
};

template <int FMT>
__device__ __forceinline__ void mm4_first(Mm4Ring<FMT> &R, const uint8_t *E, const ZzTensor &T, int g, int l, int w) {
    R.nch = (T.I / ZZ_BLK + 3) / 4;
    R.W = zz_walk(T, g, l & 15, 4 * ((l >> 2) & 3));    // piece 0 of row l%16
    R.r0 = mm4_load<FMT>(E, R.W, min(w, R.nch - 1));
    R.r1 = mm4_load<FMT>(E, R.W, min(w + 4, R.nch - 1));
}

// acc[v]: row 4(l/4)+v of the 64, token l%4, over this wave's chunks. Every load is
// unconditional (clamped past the end) so the compiler's load counters stay exact.
template <int FMT, int NS, typename DF>
__device__ __forceinline__ void mm4_kloop(Mm4Ring<FMT> &R, const uint8_t *E, int l, int w, const Mm4Stage &st,
                                          int K, float (&acc)[NS][4], DF dbg) {
    const int nch = R.nch;
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[s][v] = 0.0f;
    auto chunk = [&](const Mm4A &A, int c) {
        if (c < R.W.nfull) mm4_chunk<FMT, true, NS>(A, st, c, l, K, acc, dbg);
        else if (c < nch) mm4_chunk<FMT, false, NS>(A, st, c, l, K, acc, dbg);
    };
    if (FMT == ZZ_FMT_Q80 || NS == 2) {
        // q8_0 chunks are twice the registers, and two token sets twice the work per
        // chunk: two sets, one chunk in flight
        for (int c = w; c < nch; c += 8) {
            chunk(R.r0, c);
            R.r0 = mm4_load<FMT>(E, R.W, min(c + 8, nch - 1));
            chunk(R.r1, c + 4);
            R.r1 = mm4_load<FMT>(E, R.W, min(c + 12, nch - 1));
        }
    } else {
        for (int c = w; c < nch; c += 12) {
            R.r2 = mm4_load<FMT>(E, R.W, min(c + 8, nch - 1));
            chunk(R.r0, c);
            R.r0 = mm4_load<FMT>(E, R.W, min(c + 12, nch - 1));
            chunk(R.r1, c + 4);
            R.r1 = mm4_load<FMT>(E, R.W, min(c + 16, nch - 1));
            chunk(R.r2, c + 8);
        }
    }
    if (FMT == ZZ_FMT_Q40)                       // the 16*(q - 8) weights
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[s][v] *= 0.0625f;
}

// the four waves' partial sums of token set s into res[row][4s + token] (fixed order)
__device__ __forceinline__ void mm4_reduce(Mm4Red &rd, const float (&acc)[4], int s) {
    const int tid = threadIdx.x, w = zz_wave_id(), l = tid & 63;
#pragma unroll
    for (int v = 0; v < 4; v++) rd.part[w][l][v] = acc[v];
    __syncthreads();
    const int L = tid >> 2, v = tid & 3;
    rd.res[4 * (L >> 2) + v][4 * s + (L & 3)] =
        ((rd.part[0][L][v] + rd.part[1][L][v]) + rd.part[2][L][v]) + rd.part[3][L][v];
    __syncthreads();
}

struct Mm4Shared {
    Mm4Stage st;
    Mm4Red rd;
    float hb[8][ZZ_BLK];
};

// Diagnostics store of one int32 block dot at flat pair (token*K + slot) of sorted
// pair pos: up [P][gate/up][MI][D/32], down [P][D][MI/32].
__device__ __forceinline__ void mm_dbg_up(const ZzFfnArgs &a, int pos, int tensor, int row, int b, int v) {
    const int fl = a.ptok[pos] * a.K + a.pslot[pos];
    a.dbg_up[(((size_t)fl * 2 + tensor) * a.MI + row) * (a.D / ZZ_BLK) + b] = v;
}
__device__ __forceinline__ void mm_dbg_dn(const ZzFfnArgs &a, int pos, int row, int b, int v) {
    const int fl = a.ptok[pos] * a.K + a.pslot[pos];
    a.dbg_dn[((size_t)fl * a.D + row) * (a.MI / ZZ_BLK) + b] = v;
}

// XCD-aware work order. Workgroup g of a launch runs on XCD g % 8 (round-robin
// dispatch), and each XCD has its own L2. All tiles of one item read the same
// activations, so they get workgroup ids of one residue mod 8: item slot i runs on
// XCD i % 8 as that XCD's (i / 8)-th item, its tiles back to back. The dispatch
// kernel fills the slots so that all items of one expert share an XCD (its weights
// then come from HBM once) with the XCDs' loads balanced; empty slots (n = 0) and
// ids past the last slot exit.
#define ZZ_XCDS 8
__device__ __forceinline__ void zz_xcd_tile(int ntiles, int *item, int *tile) {
    const int g = blockIdx.x, x = g % ZZ_XCDS, k = g / ZZ_XCDS;
    *item = (k / ntiles) * ZZ_XCDS + x;
    *tile = k % ntiles;
}
static inline unsigned zz_xcd_grid(int max_items, int ntiles) {
    return (unsigned)((max_items + ZZ_XCDS - 1) / ZZ_XCDS * ZZ_XCDS * ntiles);
}
