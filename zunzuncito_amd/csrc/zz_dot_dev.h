// zz_dot_dev.h -- exact int32 block dots of one 32-weight block (q4_0, q8_0) or
// one half of a 64-weight tq2 group against int8 activations, v_dot4_i32_i8.
#pragma once
#include "zz_common.h"

__device__ __forceinline__ int zz_dot_q40(uint4 w, uint4 x0, uint4 x1) {
    const unsigned m = 0x0F0F0F0Fu;
    int s = zz_dot4(w.x & m, x0.x, 0);
    s = zz_dot4(w.y & m, x0.y, s);
    s = zz_dot4(w.z & m, x0.z, s);
    s = zz_dot4(w.w & m, x0.w, s);
    s = zz_dot4((w.x >> 4) & m, x1.x, s);
    s = zz_dot4((w.y >> 4) & m, x1.y, s);
    s = zz_dot4((w.z >> 4) & m, x1.z, s);
    s = zz_dot4((w.w >> 4) & m, x1.w, s);
    return s;                      // sum q*x with q in 0..15
}

__device__ __forceinline__ int zz_dot_q80(uint4 w0, uint4 w1, uint4 x0, uint4 x1) {
    int s = zz_dot4(w0.x, x0.x, 0);
    s = zz_dot4(w0.y, x0.y, s);
    s = zz_dot4(w0.z, x0.z, s);
    s = zz_dot4(w0.w, x0.w, s);
    s = zz_dot4(w1.x, x1.x, s);
    s = zz_dot4(w1.y, x1.y, s);
    s = zz_dot4(w1.z, x1.z, s);
    s = zz_dot4(w1.w, x1.w, s);
    return s;
}

// half h of a tq2 group: weights 32h..32h+31 are bit planes 2h (weights 32h+k) and
// 2h+1 (weights 32h+16+k) of the 16 code bytes (tq2.h:46-51)
__device__ __forceinline__ int zz_dot_tq2(uint4 c, int h, uint4 xa, uint4 xb) {
    const unsigned m = 0x03030303u;
    const int sa = 4 * h, sb = 4 * h + 2;
    int s = zz_dot4((c.x >> sa) & m, xa.x, 0);
    s = zz_dot4((c.y >> sa) & m, xa.y, s);
    s = zz_dot4((c.z >> sa) & m, xa.z, s);
    s = zz_dot4((c.w >> sa) & m, xa.w, s);
    s = zz_dot4((c.x >> sb) & m, xb.x, s);
    s = zz_dot4((c.y >> sb) & m, xb.y, s);
    s = zz_dot4((c.z >> sb) & m, xb.z, s);
    s = zz_dot4((c.w >> sb) & m, xb.w, s);
    return s;                      // sum c*x with c in {0,1,2}
}

__device__ __forceinline__ uint4 ld16(const void *p) { return *(const uint4 *)p; }

// One lane-order q4_0 word of the slot table (weights k = 8qq..8qq+7 of one block).
// The slot table stores each nibble as q ^ 8, the 4-bit two's complement of q - 8,
// so moving a nibble to the high half of its byte gives the int8 16*(q - 8) with one
// shift and mask: .x holds k 0..3, .y k 4..7 of the quarter, both scaled by 16. Dots
// of these are exactly 16 times the reference's integer dots; the kernels scale
// their fp32 sums by 1/16 (exact) at the end.
__device__ __forceinline__ uint2 zz_q4_unpack16(unsigned w) {
    return make_uint2((w << 4) & 0xF0F0F0F0u, w & 0xF0F0F0F0u);
}

// One lane-order chunk of a q4_0 / q8_0 row group: the lane's weight bytes (q4_0 in
// .a, q8_0 in .a and .b) and its row's fp16 scales, for the chunk's 4 or 2 blocks.
struct ZzChunk {
    uint4 a, b;
    uint2 s;
};

// Branch-free (only addresses are selected), so the load counters stay exact. A
// short last chunk (2 blocks) has 8 (q4_0) or 16 (q8_0) bytes per lane and 2 scales
// per row: the extra bytes read stay inside the slot (the q plane is followed by
// the scale plane, which is preceded by the q plane) and are not used.
template <int FMT>
__device__ __forceinline__ ZzChunk zz_load_chunk(const uint8_t *E, const ZzWalk &W, int c) {
    ZzChunk k;
    const bool full = c < W.nfull;
    const uint8_t *q = zz_walk_q(E, W, c);
    const uint8_t *sp = zz_walk_s(E, W, c);
    k.a = ld16(q);
    k.b = FMT == ZZ_FMT_Q80 ? ld16(q + (full ? 16 : 0)) : make_uint4(0, 0, 0, 0);
    k.s = *(const uint2 *)(sp - (full ? 0 : 4));   // short: the 2 scales in .y
    return k;
}

// signed int8 weights k = 8qq..8qq+7 of block j of a chunk, and its scale
template <int FMT>
__device__ __forceinline__ uint2 zz_chunk_w(const ZzChunk &k, int j) {
    if (FMT == ZZ_FMT_Q80) {
        const uint4 v = j < 2 ? k.a : k.b;
        return (j & 1) ? make_uint2(v.z, v.w) : make_uint2(v.x, v.y);
    }
    const unsigned w = j == 0 ? k.a.x : (j == 1 ? k.a.y : (j == 2 ? k.a.z : k.a.w));
    return zz_q4_unpack16(w);                       // 16 * (q - 8): sums scaled by 1/16
}
__device__ __forceinline__ float zz_chunk_dw(const ZzChunk &k, int j, bool full) {
    const unsigned v = j < 2 && full ? k.s.x : k.s.y;
    return zz_h2f((uint16_t)((j & 1) ? v >> 16 : v & 0xffff));
}
