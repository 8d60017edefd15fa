// zz_common.h -- shared device/host definitions for the MI355X MoE library.
//
// Everything here is gfx950-only HIP. Files are compiled with -ffp-contract=off:
// every fused multiply-add is written as fmaf(), so bit-level behaviour is
// explicit wherever it matters (activation quantisation, router logits).
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#define ZZ_BLK 32              // q4_0 / q8_0 / activation block (q40.h:41)
#define ZZ_MAXK 16             // top-k limit (gemma4.c:53 MAXTOPK)
#define ZZ_MAXE 512            // experts per layer (maple.c:67 MAXEXPERTS)
#define ZZ_MAXD 8192           // hidden / intermediate limit of one call

// formats: gpu.h:49-52
#define ZZ_FMT_Q40 1
#define ZZ_FMT_Q80 2
#define ZZ_FMT_TQ2 3
#define ZZ_FMT_Q4A 4           // gpu_matmul only: maple's lm_head / centroid format

// gating and activation kinds, mirrored in include/zz_moe.h
#define ZZ_GATE_SOFTMAX_PES 0   // gemma4.c:581-613
#define ZZ_GATE_SIGMOID_BIAS 1  // lfm25.c:636-668
#define ZZ_GATE_SOFTMAX_TOPK 2  // maple.c:582-601
#define ZZ_GATE_DENSE 3         // gemma4.c:1012-1020: the dense MLP branch, no router
#define ZZ_GATE_GROUPED 4       // ling.c:705-789: grouped sigmoid top-k
#define ZZ_MAXGROUP 64          // expert groups of a grouped router

#define ZZ_ACT_GEGLU_TANH 0     // gemma4.c:432-434
#define ZZ_ACT_SWIGLU 1         // lfm25.c:456-458
#define ZZ_ACT_SWIGLU_CLAMP 2   // maple.c:607-611

#define ZZ_CHECK(x)                                                            \
    do {                                                                       \
        hipError_t e_ = (x);                                                   \
        if (e_ != hipSuccess) {                                                \
            zz_set_error("%s:%d %s: %s", __FILE__, __LINE__, #x,                 \
                         hipGetErrorString(e_));                               \
            return 0;                                                          \
        }                                                                      \
    } while (0)

void zz_set_error(const char *fmt, ...);

// Device view of one expert tensor inside the HBM slot table. Rows are stored in
// groups of 16: for each (16-row group, block) the 16 rows' payloads are one
// contiguous chunk, so a wave reading one block of 16 rows reads 256 (q4_0, tq2)
// or 512 (q8_0) contiguous bytes, in the order the 16x16x32 int8 MFMA wants them.
//   q4_0: payload [O/16][I/32][16][16 B nibbles], scales [O/16][I/32][16] fp16
//   q8_0: payload [O/16][I/32][16][32 B int8],    scales as q4_0
//   tq2:  codes   [O/16][I/64][16][16 B],         alpha [O] f32 (row order)
// The block contents are the reference's bytes unchanged (q40.h:12-17, 320-329;
// tq2.h:46-51); only their placement differs.
struct ZzTensor {
    int fmt, O, I;
    int64_t off_q;       // byte offset of the payload plane inside the expert
    int64_t off_s;       // byte offset of the scale plane (alpha for tq2)
};

// blocks per row: 32-weight blocks (q4_0, q8_0) or 64-weight groups (tq2)
__host__ __device__ __forceinline__ int zz_nblk(const ZzTensor &T) {
    return T.fmt == ZZ_FMT_TQ2 ? T.I / 64 : T.I / ZZ_BLK;
}

// q4_0 / q8_0 payload, matrix-core lane order. Rows are grouped by 16 (g = row/16)
// and the 32-weight blocks of a row by 4 (chunk = b/4; the last chunk of a row holds
// 2 when I/32 % 4 == 2). Lane l = 16*qq + r of a chunk holds, for row 16g + r, the
// weights k = 8qq..8qq+7 of every block of the chunk, ZZ_LB bytes per block:
//   q8_0: those 8 int8 in order;
//   q4_0: 4 bytes, byte m = nibble(8qq+m) | nibble(8qq+m+4) << 4.
// A lane's bytes for the blocks of one chunk are contiguous (one 16/32-byte load),
// and a chunk is 64 lanes x its blocks x ZZ_LB bytes. This is the A operand layout of
// v_mfma_i32_16x16x32_i8 (lane l: row l%16, k = 8*(l/16)..+7). The fp16 block
// scales of a chunk are ordered [row][block]: one row's scales of a chunk are
// contiguous, and so are 4 consecutive rows'. The plane sizes equal the reference
// tensor's payload and scale bytes.
__host__ __device__ __forceinline__ int zz_lb(const ZzTensor &T) { return T.fmt == ZZ_FMT_Q80 ? 8 : 4; }
// blocks in the chunk holding block b (4, or 2 for a short last chunk)
__host__ __device__ __forceinline__ int zz_cbs(const ZzTensor &T, int b) {
    const int left = T.I / ZZ_BLK - (b & ~3);
    return left < 4 ? left : 4;
}
// byte offset of lane `lane`'s ZZ_LB bytes of block b in row group g
__host__ __device__ __forceinline__ int64_t zz_qlane(const ZzTensor &T, int g, int b, int lane) {
    const int nb = T.I / ZZ_BLK, lb = zz_lb(T);
    return T.off_q + ((int64_t)g * nb + (b & ~3)) * 64 * lb + (int64_t)lane * zz_cbs(T, b) * lb + (b & 3) * lb;
}
// byte offset of the fp16 scale of row 16g + r, block b
__host__ __device__ __forceinline__ int64_t zz_sidx(const ZzTensor &T, int g, int b, int r) {
    const int nb = T.I / ZZ_BLK;
    return T.off_s + ((int64_t)g * nb + (b & ~3)) * 32 + (r * zz_cbs(T, b) + (b & 3)) * 2;
}
// tq2 codes: 16-row groups, each a run of the 16 rows' 16-byte 64-weight groups in
// the reference byte order (byte k: weights k, k+16, k+32, k+48 at bits 0, 2, 4, 6)
// A lane's walk over the chunks of one 16-row group of a q4_0 / q8_0 tensor, with
// the offsets of zz_qlane / zz_sidx strength-reduced: a full chunk is chunk 0 plus c
// strides, the short last chunk (if any) has its own offset. rr is the row of the
// scale pointer within the group. Offsets are from the expert's base and fit 32
// bits (an expert of the largest accepted shape, D = MI = 8192 in q8_0, is 214 MB),
// so a load is the uniform base plus one 32-bit lane offset.
struct ZzWalk {
    uint32_t qb, qs, sb, ss, qstep;
    int nfull;
};
__device__ __forceinline__ ZzWalk zz_walk(const ZzTensor &T, int g, int lane, int rr) {
    ZzWalk w;
    const int nb = T.I / ZZ_BLK, lb = zz_lb(T);
    w.nfull = nb / 4;
    w.qstep = 256 * lb;
    w.qb = (uint32_t)zz_qlane(T, g, 0, lane);
    w.sb = (uint32_t)zz_sidx(T, g, 0, rr);
    const int bl = 4 * (w.nfull < (nb + 3) / 4 ? w.nfull : 0);     // the short chunk's first block
    w.qs = (uint32_t)zz_qlane(T, g, bl, lane);
    w.ss = (uint32_t)zz_sidx(T, g, bl, rr);
    return w;
}
__device__ __forceinline__ uint32_t zz_walk_qo(const ZzWalk &w, int c) {
    return c < w.nfull ? w.qb + (uint32_t)c * w.qstep : w.qs;
}
__device__ __forceinline__ uint32_t zz_walk_so(const ZzWalk &w, int c) {
    return c < w.nfull ? w.sb + (uint32_t)c * 128u : w.ss;
}
__device__ __forceinline__ const uint8_t *zz_walk_q(const uint8_t *E, const ZzWalk &w, int c) {
    return E + zz_walk_qo(w, c);
}
__device__ __forceinline__ const uint8_t *zz_walk_s(const uint8_t *E, const ZzWalk &w, int c) {
    return E + zz_walk_so(w, c);
}
// The wave's index in its workgroup, as a uniform value: what is derived from it
// (the tensor a wave walks, its chunk counts) then stays in scalar registers.
__device__ __forceinline__ int zz_wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__host__ __device__ __forceinline__ int64_t zz_tq2off(const ZzTensor &T, int row, int gp) {
    return T.off_q + (((int64_t)(row >> 4) * (T.I / 64) + gp) * 16 + (row & 15)) * 16;
}
// payload bytes per row and 32-weight block (q4_0 16, q8_0 32)
__host__ __device__ __forceinline__ int zz_pbytes(const ZzTensor &T) {
    return T.fmt == ZZ_FMT_Q80 ? 32 : 16;
}

struct ZzLayout {        // byte layout of one repacked expert, all 256-aligned
    ZzTensor gate, up, down;
    int64_t bytes;       // stride between experts in the slot table
};

// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ float zz_h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;     // v_cvt_f32_f16: exact for every binary16 value
}

// distance from |x| to the next float away from zero
__device__ __forceinline__ float ulp_of(float x) {
    float a = fabsf(x);
    return __uint_as_float(__float_as_uint(a) + 1u) - a;
}

__device__ __forceinline__ int zz_dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);   // v_dot4_i32_i8
}

// Cross-lane reductions without the LDS crossbar (a shuffle is a ds_bpermute, one
// LDS round trip per step). Within a row of 16 lanes, DPP: quad_perm [1,0,3,2] and
// [2,3,0,1] pair lane i with i ^ 1 and i ^ 2, row_half_mirror lane i of each 8 with
// 7 - i, row_mirror lane i of the row with 15 - i. Across rows, gfx950's permlane
// swaps with both operands v: lanes i and i ^ 16 (W = 16) or i ^ 32 (W = 32) both
// receive (v of the lower lane, v of the upper lane).
template <int CTRL>
__device__ __forceinline__ unsigned zz_dpp_b32(unsigned v) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL, typename T>
__device__ __forceinline__ T zz_dpp_x(T v) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        return __builtin_bit_cast(T, ((unsigned long long)zz_dpp_b32<CTRL>((unsigned)(u >> 32)) << 32) |
                                         zz_dpp_b32<CTRL>((unsigned)u));
    } else {
        return __builtin_bit_cast(T, zz_dpp_b32<CTRL>(__builtin_bit_cast(unsigned, v)));
    }
}
template <int W>
__device__ __forceinline__ void zz_swap_b32(unsigned v, unsigned &lo, unsigned &hi) {
    if constexpr (W == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        lo = r[0];
        hi = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        lo = r[0];
        hi = r[1];
    }
}
template <int W, typename T>
__device__ __forceinline__ void zz_swap_x(T v, T &lo, T &hi) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        unsigned l0, h0, l1, h1;
        zz_swap_b32<W>((unsigned)u, l0, h0);
        zz_swap_b32<W>((unsigned)(u >> 32), l1, h1);
        lo = __builtin_bit_cast(T, ((unsigned long long)l1 << 32) | l0);
        hi = __builtin_bit_cast(T, ((unsigned long long)h1 << 32) | h0);
    } else {
        unsigned l, h;
        zz_swap_b32<W>(__builtin_bit_cast(unsigned, v), l, h);
        lo = __builtin_bit_cast(T, l);
        hi = __builtin_bit_cast(T, h);
    }
}
// v combined by op over aligned groups of N lanes (N a power of 2, 2..64); every lane
// of a group gets the same result (each step combines two values, a op b == b op a
// for the commutative ops used: IEEE add, fmaxf, integer add). Every lane of the
// wave must take part.
template <int N, typename T, typename OP>
__device__ __forceinline__ T zz_group_reduce(T v, OP op) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group of 2..64 lanes");
    if constexpr (N >= 2) v = op(v, zz_dpp_x<0xB1>(v));
    if constexpr (N >= 4) v = op(v, zz_dpp_x<0x4E>(v));
    if constexpr (N >= 8) v = op(v, zz_dpp_x<0x141>(v));
    if constexpr (N >= 16) v = op(v, zz_dpp_x<0x140>(v));
    if constexpr (N >= 32) {
        T a, b;
        zz_swap_x<16>(v, a, b);
        v = op(a, b);
    }
    if constexpr (N >= 64) {
        T a, b;
        zz_swap_x<32>(v, a, b);
        v = op(a, b);
    }
    return v;
}
template <int N, typename T>
__device__ __forceinline__ T zz_group_sum(T v) {
    return zz_group_reduce<N>(v, [](T x, T y) { return x + y; });
}
template <int N>
__device__ __forceinline__ float zz_group_max(float v) {
    return zz_group_reduce<N>(v, [](float x, float y) { return fmaxf(x, y); });
}

// v combined over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the same position in the
// wave's four rows); every one of the four gets the result
template <typename T, typename OP>
__device__ __forceinline__ T zz_rows_reduce(T v, OP op) {
    T a, b;
    zz_swap_x<16>(v, a, b);
    v = op(a, b);
    zz_swap_x<32>(v, a, b);
    return op(a, b);
}
template <typename T>
__device__ __forceinline__ T zz_rows_sum(T v) {
    return zz_rows_reduce(v, [](T x, T y) { return x + y; });
}
__device__ __forceinline__ float zz_rows_max(float v) {
    return zz_rows_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}

// inclusive prefix sum over a wave: DPP shifts within each 16-lane row by 1, 2, 4,
// 8 (lanes shifted in from outside the row add zero), then row_bcast:15 adds row 0's
// total to row 1 and row 2's to row 3, row_bcast:31 the total of rows 0-1 to rows 2
// and 3. Six levels of adds, as a shuffle scan. Every lane must take part.
template <typename T>
__device__ __forceinline__ T zz_wave_incl_scan_add(T x) {
    auto sh = [](T v, auto ctrl, auto rows) {
        constexpr int C = decltype(ctrl)::value, RW = decltype(rows)::value;
        if constexpr (sizeof(T) == 8) {
            const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
            const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, C, RW, 0xF, false);
            const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), C, RW, 0xF, false);
            return __builtin_bit_cast(T, ((unsigned long long)hi << 32) | lo);
        } else {
            return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), C, RW, 0xF, false));
        }
    };
    using F = std::integral_constant<int, 0xF>;
    x += sh(x, std::integral_constant<int, 0x111>(), F());
    x += sh(x, std::integral_constant<int, 0x112>(), F());
    x += sh(x, std::integral_constant<int, 0x114>(), F());
    x += sh(x, std::integral_constant<int, 0x118>(), F());
    x += sh(x, std::integral_constant<int, 0x142>(), std::integral_constant<int, 0xA>());
    x += sh(x, std::integral_constant<int, 0x143>(), std::integral_constant<int, 0xC>());
    return x;
}

// the value of lane q (q wave-uniform)
__device__ __forceinline__ double zz_lane_f64(double v, int q) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, q);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), q);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T zz_wave_sum(T v) {
    return zz_group_sum<64>(v);
}

__device__ __forceinline__ float zz_wave_max(float v) { return zz_group_max<64>(v); }

// q40.h:124-138 activation quantisation of one 32-value block held one value per
// lane of a 32-lane group (lanes 0..31 or 32..63 of a wave). d = amax/127 (IEEE
// division), q = rint(v * (1/d)) clamped to +-127. Bit-exact with the reference.
__device__ __forceinline__ int zz_quant_lane(float v, float *d_out) {
    const float a = zz_group_max<32>(fabsf(v));
    float d = a / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    float q = rintf(v * id);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    *d_out = d;
    return (int)q;
}

// q40.h:124-138 for one whole 32-block held by a single thread: no cross-lane
// traffic. Writes 32 int8 to q (16-byte aligned), returns d; *sum = sum of q.
__device__ __forceinline__ float zz_quant_block(const float (&v)[ZZ_BLK], int8_t *q, int *sum) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < ZZ_BLK; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    unsigned w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int s = 0;
#pragma unroll
    for (int j = 0; j < ZZ_BLK; j++) {
        float f = rintf(v[j] * id);
        f = fminf(fmaxf(f, -127.0f), 127.0f);
        const int qi = (int)f;
        s += qi;
        w[j >> 2] |= (unsigned)(qi & 0xff) << (8 * (j & 3));
    }
    ((uint4 *)q)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    ((uint4 *)q)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *sum = s;
    return d;
}

// zz_quant_block of a 32-block held by 8 consecutive lanes of a wave, 4 values each
// (lane 8i + m holds values 4m..4m+3): the same amax, scale and rounding. Returns the
// lane's 4 codes packed; d and the block's code sum go to every lane of the 8.
// Every lane of the wave must call it.
__device__ __forceinline__ unsigned zz_quant8(float4 v, float *d_out, int *sum_out) {
    const float m = zz_group_max<8>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float d = m / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q0 = (int)fminf(fmaxf(rintf(v.x * id), -127.0f), 127.0f);
    const int q1 = (int)fminf(fmaxf(rintf(v.y * id), -127.0f), 127.0f);
    const int q2 = (int)fminf(fmaxf(rintf(v.z * id), -127.0f), 127.0f);
    const int q3 = (int)fminf(fmaxf(rintf(v.w * id), -127.0f), 127.0f);
    const int qs = zz_group_sum<8>(q0 + q1 + q2 + q3);
    *d_out = d;
    *sum_out = qs;
    return (unsigned)(q0 & 0xff) | (unsigned)(q1 & 0xff) << 8 | (unsigned)(q2 & 0xff) << 16 |
           (unsigned)(q3 & 0xff) << 24;
}

// The activations (gemma4.c:432-437, lfm25.c:456-458, maple.c:607-611) in forms of one
// hardware exp (v_exp_f32, 2^x) and one reciprocal (v_rcp_f32) per element, without
// branches. gelu_tanh: 0.5 x (1 + tanh(y)) equals x / (1 + e^(-2y)) exactly in real
// arithmetic, with y = sqrt(2/pi) (x + 0.044715 x^3); silu: x / (1 + e^(-x)). Each
// result is within a few ulp of the reference's glibc tanhf / expf forms, except where
// the reference's 1 + tanhf(y) cancels (y << 0), whose outputs are below any block's
// q8_0 step. These feed the q8_0 hidden, which the reference quantises the same way.
#define ZZ_LOG2E 1.4426950408889634f
__device__ __forceinline__ float zz_gelu_tanh(float x) {
    const float inner = fmaf((0.044715f * x) * x, x, x);
    const float e = __builtin_amdgcn_exp2f(inner * (-2.0f * 0.7978845608028654f * ZZ_LOG2E));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float zz_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -ZZ_LOG2E));
}

__device__ __forceinline__ float zz_act(int act, float g, float u, float clamp) {
    if (act == ZZ_ACT_GEGLU_TANH) return zz_gelu_tanh(g) * u;
    if (act == ZZ_ACT_SWIGLU_CLAMP) {           // maple.c:672-675
        if (g > clamp) g = clamp;
        u = u < -clamp ? -clamp : (u > clamp ? clamp : u);
    }
    return zz_silu(g) * u;
}
