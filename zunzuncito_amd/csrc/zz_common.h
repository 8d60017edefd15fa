// zz_common.h -- shared device/host definitions for the MI355X MoE library.
//
// Everything here is gfx950-only HIP. Files are compiled with -ffp-contract=off:
// every fused multiply-add is written as fmaf(), so bit-level behaviour is
// explicit wherever it matters (activation quantisation, router logits).
#pragma once
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

// gating and activation kinds, mirrored in include/zz_moe.h
#define ZZ_GATE_SOFTMAX_PES 0   // gemma4.c:581-613
#define ZZ_GATE_SIGMOID_BIAS 1  // lfm25.c:636-668
#define ZZ_GATE_SOFTMAX_TOPK 2  // maple.c:582-601

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
__host__ __device__ __forceinline__ int zz_pbytes(const ZzTensor &T) {
    return T.fmt == ZZ_FMT_Q80 ? 32 : 16;
}
// byte offset of row `row`, block `b` payload; of its fp16 scale (q4_0/q8_0)
__host__ __device__ __forceinline__ int64_t zz_qoff(const ZzTensor &T, int row, int b) {
    return T.off_q + (((int64_t)(row >> 4) * zz_nblk(T) + b) * 16 + (row & 15)) * zz_pbytes(T);
}
__host__ __device__ __forceinline__ int64_t zz_soff(const ZzTensor &T, int row, int b) {
    return T.off_s + (((int64_t)(row >> 4) * zz_nblk(T) + b) * 16 + (row & 15)) * 2;
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

template <typename T>
__device__ __forceinline__ T zz_wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float zz_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// q40.h:124-138 activation quantisation of one 32-value block held one value per
// lane of a 32-lane group (lanes 0..31 or 32..63 of a wave). d = amax/127 (IEEE
// division), q = rint(v * (1/d)) clamped to +-127. Bit-exact with the reference.
__device__ __forceinline__ int zz_quant_lane(float v, float *d_out) {
    float a = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
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

__device__ __forceinline__ float zz_gelu_tanh(float x) {
    float inner = fmaf((0.044715f * x) * x, x, x);
    return (0.5f * x) * (1.0f + tanhf(0.7978845608028654f * inner));
}

__device__ __forceinline__ float zz_silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float zz_act(int act, float g, float u, float clamp) {
    if (act == ZZ_ACT_GEGLU_TANH) return zz_gelu_tanh(g) * u;
    if (act == ZZ_ACT_SWIGLU_CLAMP) {           // maple.c:672-675
        if (g > clamp) g = clamp;
        u = u < -clamp ? -clamp : (u > clamp ? clamp : u);
    }
    return zz_silu(g) * u;
}
