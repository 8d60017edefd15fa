/* zz_oracle.c -- CPU restatement of the zunzuncito MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see zz_oracle.h): the checker for the HIP library,
 * never linked into it. Built with -ffp-contract=off so that every fused
 * multiply-add below is one the reference build (gcc -O3 -march=x86-64-v3) also
 * makes, written out with fmaf().
 */
#include "zz_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define BLK 32

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* The host libm's expf on n values: glibc's, the function the reference's sigmoid
 * routers call (lfm25.c:654, ling.c:731), for checking the device's expf. */
void orc_expf(const float *x, float *y, long long n) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ------------------------------------------------------------------ A1 ----
 * IEEE binary16 <-> binary32, round half to even, subnormals kept.
 * Follows q40.h:46-80, including its NaN encoding (quiet, payload dropped).
 * Pinned by numpy.float16 on all 65536 halves and on random floats. */
float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (ex == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (ex == 0) {
        float v = (float)man * 0x1p-24f;        /* exact: man < 2^10 */
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f2h(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t ex = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)ex - 112;                      /* binary16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t full = man | 0x800000u;
        int sh = 14 - e;                        /* 14..24 */
        uint32_t q = full >> sh, r = full & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (r > half || (r == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = man >> 13, r = man & 0x1fffu;
    uint32_t v = ((uint32_t)e << 10) | q;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) v++;   /* carries into exponent */
    if (v >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | v);
}

static inline float blk_scale(const uint8_t *blk) {
    uint16_t h;
    memcpy(&h, blk, 2);
    return orc_h2f(h);
}

/* ------------------------------------------------------------- A3 / A7 ----
 * q40.h:83-110: d = fp16(mx / -8) with mx the first max-|x| element, then
 * q = trunc(x*id + 8.5) clamped to 0..15 (the multiply-add is fused in the
 * reference build). Pinned bit-exact against oracle/_ref. */
void orc_q40_quant_row(const float *w, uint8_t *dst, int I) {
    for (int b = 0; b < I / BLK; b++) {
        const float *x = w + (size_t)b * BLK;
        uint8_t *blk = dst + (size_t)b * 18;
        float amax = 0.f, mx = 0.f;
        for (int j = 0; j < BLK; j++) {
            float a = fabsf(x[j]);
            if (a > amax) { amax = a; mx = x[j]; }
        }
        uint16_t hd = orc_f2h(mx / -8.0f);
        memcpy(blk, &hd, 2);
        float d = orc_h2f(hd);
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int j = 0; j < 16; j++) {
            int lo = (int)fmaf(x[j], id, 8.5f);
            int hi = (int)fmaf(x[j + 16], id, 8.5f);
            lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
            hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
            blk[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* q40.h:332-348: d = fp16(amax/127), q = rint(x/d) clamped to +-127 */
void orc_q80_quant_row(const float *w, uint8_t *dst, int I) {
    for (int b = 0; b < I / BLK; b++) {
        const float *x = w + (size_t)b * BLK;
        uint8_t *blk = dst + (size_t)b * 34;
        float amax = 0.f;
        for (int j = 0; j < BLK; j++) {
            float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        uint16_t hd = orc_f2h(amax / 127.0f);
        memcpy(blk, &hd, 2);
        float d = orc_h2f(hd), id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int j = 0; j < BLK; j++) {
            long q = lrintf(x[j] * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            blk[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

void orc_q40_dequant_row(const uint8_t *src, float *w, int I) {
    for (int b = 0; b < I / BLK; b++) {
        const uint8_t *blk = src + (size_t)b * 18;
        float d = blk_scale(blk);
        for (int j = 0; j < 16; j++) {
            w[b * BLK + j] = d * (float)((blk[2 + j] & 15) - 8);
            w[b * BLK + j + 16] = d * (float)((blk[2 + j] >> 4) - 8);
        }
    }
}

/* Test-only planted mistakes (zz_oracle.h lists them); 0 everywhere else. */
static int g_plant = 0;
void orc_set_plant(int plant) { g_plant = plant; }

/* q40.h:349-356: w = d * q per block. Pinned against the compiled reference's
 * q80_dequant_row and against numpy's float16 decode of the scale times the codes. */
void orc_q80_dequant_row(const uint8_t *src, float *w, int I) {
    for (int b = 0; b < I / BLK; b++) {
        const uint8_t *blk = src + (size_t)b * 34;
        float d = blk_scale(g_plant == 5 && b > 0 ? blk - 34 : blk);
        for (int j = 0; j < BLK; j++) w[b * BLK + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* tq2.h:46-51: in each 64-weight group, byte k holds weights k, k+16, k+32, k+48
 * at bit offsets 0, 2, 4, 6. */
void orc_tq2_pack_row(const int8_t *code, uint8_t *dst, int I) {
    for (int g = 0; g < I / 64; g++)
        for (int k = 0; k < 16; k++) {
            const int8_t *c = code + (size_t)g * 64;
            dst[(size_t)g * 16 + k] = (uint8_t)((c[k] & 3) | ((c[k + 16] & 3) << 2) |
                                                ((c[k + 32] & 3) << 4) | ((c[k + 48] & 3) << 6));
        }
}

static inline int tq2_code(const uint8_t *codes, int j) {
    return (codes[(size_t)(j / 64) * 16 + (j % 16)] >> (2 * ((j / 16) % 4))) & 3;
}

void orc_tq2_dequant_row(const uint8_t *codes, float alpha, float *w, int I) {
    for (int j = 0; j < I; j++) w[j] = alpha * (float)(tq2_code(codes, j) - 1);
}

/* ------------------------------------------------------------- A4 / A8 ----
 * q40.h:124-138: per block d = amax/127 (f32), q = lrint(v * (1/d)) clamped. */
void orc_quant_act(const float *x, int8_t *xq, float *sx, int I) {
    for (int b = 0; b < I / BLK; b++) {
        const float *v = x + (size_t)b * BLK;
        float amax = 0.f;
        for (int j = 0; j < BLK; j++) {
            float a = fabsf(v[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        sx[b] = d;
        for (int j = 0; j < BLK; j++) {
            long q = lrintf(v[j] * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            xq[(size_t)b * BLK + j] = (int8_t)q;
        }
    }
}

/* tq2.h:98-108: the above plus Sx = sum_b sx[b]*sum_j xq (serial, double) */
float orc_tq2_quant_act(const float *x, int8_t *xq, float *sx, int I) {
    orc_quant_act(x, xq, sx, I);
    double tot = 0.0;
    for (int b = 0; b < I / BLK; b++) {
        int32_t s = 0;
        for (int j = 0; j < BLK; j++) s += xq[(size_t)b * BLK + j];
        tot += (double)sx[b] * (double)s;
    }
    return (float)tot;
}

/* --------------------------------------------------------- A5 / A7 / A8 ----
 * The AVX2 dots keep 4 accumulators x 8 lanes; lane l of a 32-weight block holds
 * the exact integer partial over weights 4l..4l+3 and is folded in with one FMA
 * (q40.h:162-207, 359-391; tq2.h:116-155). Blocks b go to accumulator b%4 while
 * four remain, the tail to accumulator 0; the final reduction is
 * ((a0+a1)+(a2+a3)) per lane, then lanes (l, l+4), then (0,2),(1,3), then the pair. */
typedef struct { float a[4][8]; } acc8;

static inline void acc_zero(acc8 *A) { memset(A, 0, sizeof *A); }

static inline float acc_reduce(const acc8 *A) {
    float v[8];
    for (int l = 0; l < 8; l++) v[l] = (A->a[0][l] + A->a[1][l]) + (A->a[2][l] + A->a[3][l]);
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s2) + (s1 + s3);
}

static inline int acc_slot(int b, int nb) { return b < (nb & ~3) ? (b & 3) : 0; }

/* lane partials of one q4_0 block: sum over j in lane of (q_j - 8) * x_j */
static inline void q40_lanes(const uint8_t *blk, const int8_t *x, int32_t p[8]) {
    for (int l = 0; l < 8; l++) {
        int32_t s = 0;
        for (int j = 4 * l; j < 4 * l + 4; j++) {
            int q = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
            s += (q - 8) * (int32_t)x[j];
        }
        p[l] = s;
    }
}

float orc_q40_dot(const uint8_t *w, const int8_t *xq, const float *sx, int I) {
    acc8 A;
    acc_zero(&A);
    int nb = I / BLK;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = w + (size_t)b * 18;
        float d = blk_scale(blk) * sx[b];
        int32_t p[8];
        q40_lanes(blk, xq + (size_t)b * BLK, p);
        int a = acc_slot(b, nb);
        for (int l = 0; l < 8; l++) A.a[a][l] = fmaf(d, (float)p[l], A.a[a][l]);
    }
    return acc_reduce(&A);
}

float orc_q80_dot(const uint8_t *w, const int8_t *xq, const float *sx, int I) {
    acc8 A;
    acc_zero(&A);
    int nb = I / BLK;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = w + (size_t)b * 34;
        const int8_t *q = (const int8_t *)(blk + 2), *x = xq + (size_t)b * BLK;
        float d = blk_scale(blk) * sx[b];
        int a = acc_slot(b, nb);
        for (int l = 0; l < 8; l++) {
            int32_t s = 0;
            for (int j = 4 * l; j < 4 * l + 4; j++) s += (int32_t)q[j] * x[j];
            A.a[a][l] = fmaf(d, (float)s, A.a[a][l]);
        }
    }
    return acc_reduce(&A);
}

float orc_tq2_dot(const uint8_t *codes, float alpha, const int8_t *xq,
                  const float *sx, float sxtot, int I) {
    acc8 A;
    acc_zero(&A);
    int ng = I / 64;
    for (int g = 0; g < ng; g++) {
        const uint8_t *c = codes + (size_t)g * 16;
        const int8_t *x = xq + (size_t)g * 64;
        int a = acc_slot(g, ng);
        for (int half = 0; half < 2; half++) {
            float d = sx[2 * g + half];
            for (int l = 0; l < 8; l++) {
                int32_t s = 0;
                for (int j = 4 * l; j < 4 * l + 4; j++) {
                    int jj = 32 * half + j;          /* weight index inside the group */
                    s += ((c[jj % 16] >> (2 * (jj / 16))) & 3) * (int32_t)x[jj];
                }
                A.a[a][l] = fmaf(d, (float)s, A.a[a][l]);
            }
        }
    }
    return alpha * (acc_reduce(&A) - sxtot);
}

void orc_blockdots(int fmt, const uint8_t *row, const int8_t *xq, int I, int32_t *out) {
    for (int b = 0; b < I / BLK; b++) {
        const int8_t *x = xq + (size_t)b * BLK;
        int32_t s = 0;
        for (int j = 0; j < BLK; j++) {
            int w;
            if (fmt == ORC_FMT_Q40) {
                const uint8_t *blk = row + (size_t)b * 18;
                w = (j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4)) - 8;
            } else if (fmt == ORC_FMT_Q80) {
                w = (int8_t)row[(size_t)b * 34 + 2 + j];
            } else {
                w = tq2_code(row, b * BLK + j) - 1;
            }
            s += w * (int32_t)x[j];
        }
        out[b] = s;
    }
}

/* ------------------------------------------------------------- A6 / A9 ---- */
float orc_q40_dot_f32(const uint8_t *w, const float *x, int I) {
    double acc = 0.0;
    for (int b = 0; b < I / BLK; b++) {
        const uint8_t *blk = w + (size_t)b * 18;
        double s = 0.0;
        for (int j = 0; j < 16; j++) {
            s += (double)((blk[2 + j] & 15) - 8) * x[b * BLK + j];
            s += (double)((blk[2 + j] >> 4) - 8) * x[b * BLK + j + 16];
        }
        acc += (double)blk_scale(blk) * s;
    }
    return (float)acc;
}

float orc_q80_dot_f32(const uint8_t *w, const float *x, int I) {
    double acc = 0.0;
    for (int b = 0; b < I / BLK; b++) {
        const uint8_t *blk = w + (size_t)b * 34;
        double s = 0.0;
        for (int j = 0; j < BLK; j++) s += (double)(int8_t)blk[2 + j] * x[b * BLK + j];
        acc += (double)blk_scale(blk) * s;
    }
    return (float)acc;
}

float orc_tq2_dot_f32(const uint8_t *codes, float alpha, const float *x, int I) {
    double acc = 0.0;
    for (int g = 0; g < I / 64; g++) {
        double s = 0.0;
        for (int k = 0; k < 16; k++)
            for (int q = 0; q < 4; q++)
                s += (double)(((codes[(size_t)g * 16 + k] >> (2 * q)) & 3) - 1) *
                     x[(size_t)g * 64 + k + 16 * q];
        acc += s;
    }
    return (float)((double)alpha * acc);
}

/* tq2.h:405-427: a Q4A group is 64 weights in 36 bytes -- fp16 d, fp16 m, then two
 * 16-byte halves, byte j of half h holding q[32h + j] (low nibble) and q[32h + j + 16]
 * (high); w = d q + m. Per half, sum q u and sum u in double, then add d s + m t. */
float orc_q4a_dot_f32(const uint8_t *w, const float *x, int I) {
    double acc = 0.0;
    for (int g = 0; g < I / 64; g++) {
        const uint8_t *grp = w + (size_t)g * 36;
        const double d = orc_h2f((uint16_t)(grp[0] | grp[1] << 8));
        const double m = orc_h2f((uint16_t)(grp[2] | grp[3] << 8));
        for (int h = 0; h < 2; h++) {
            const uint8_t *nib = grp + 4 + 16 * h;
            const float *u = x + (size_t)g * 64 + 32 * h;
            double s = 0.0, t = 0.0;
            for (int j = 0; j < 16; j++) {
                s += (double)(nib[j] & 15) * u[j];
                s += (double)(nib[j] >> 4) * u[j + 16];
                t += (double)u[j] + (double)u[j + 16];
            }
            acc += d * s + m * t;
        }
    }
    return (float)acc;
}

int64_t orc_tensor_bytes(int fmt, int O, int I) {
    if (fmt == ORC_FMT_Q40) return (int64_t)O * (I / BLK) * 18;
    if (fmt == ORC_FMT_Q80) return (int64_t)O * (I / BLK) * 34;
    if (fmt == ORC_FMT_TQ2) return (int64_t)O * 4 + (int64_t)O * (I / 4);
    if (fmt == ORC_FMT_Q4A) return (int64_t)O * (I / 64) * 36;      /* tq2.h:287-292 */
    return -1;
}

static inline int64_t row_bytes(int fmt, int I) {
    return fmt == ORC_FMT_Q40 ? (int64_t)(I / BLK) * 18
         : fmt == ORC_FMT_Q80 ? (int64_t)(I / BLK) * 34
         : fmt == ORC_FMT_Q4A ? (int64_t)(I / 64) * 36 : (int64_t)I / 4;
}

void orc_matmul_f32(int fmt, float *y, const uint8_t *W, const float *x, int O, int I, int S) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++) {
            const float *xs = x + (size_t)s * I;
            float v;
            if (fmt == ORC_FMT_TQ2) {
                const float *alpha = (const float *)W;
                const uint8_t *codes = W + (size_t)O * 4;
                v = orc_tq2_dot_f32(codes + (size_t)o * (I / 4), alpha[o], xs, I);
            } else if (fmt == ORC_FMT_Q80) {
                v = orc_q80_dot_f32(W + (size_t)o * row_bytes(fmt, I), xs, I);
            } else if (fmt == ORC_FMT_Q4A) {
                v = orc_q4a_dot_f32(W + (size_t)o * row_bytes(fmt, I), xs, I);
            } else {
                v = orc_q40_dot_f32(W + (size_t)o * row_bytes(fmt, I), xs, I);
            }
            y[(size_t)s * O + o] = v;
        }
}

/* ----------------------------------------------------------------- A18 ----
 * gemma4.c:425-437: sum of squares in double, r = 1/sqrtf(float(s/D) + eps),
 * o = (x*r)*w. Aliasing o == x is allowed (the reference post-norm does it). */
void orc_rmsnorm(float *o, const float *x, const float *w, int D, float eps) {
    double s = 0.0;
    for (int i = 0; i < D; i++) s += (double)x[i] * x[i];
    float r = 1.0f / sqrtf((float)(s / D) + eps);
    for (int i = 0; i < D; i++) o[i] = w ? (x[i] * r) * w[i] : x[i] * r;
}

static inline float gelu_tanh(float x) {
    /* gemma4.c:432-434; the cubic term is fused into the add by the reference build */
    float inner = fmaf((0.044715f * x) * x, x, x);
    return (0.5f * x) * (1.0f + tanhf(0.7978845608028654f * inner));
}

static inline float silu(float x) { return x / (1.0f + expf(-x)); }

float orc_act(int act, float g, float u, float clamp) {
    if (act == ORC_ACT_GEGLU_TANH) return gelu_tanh(g) * u;
    if (act == ORC_ACT_SWIGLU_CL) {                 /* maple.c:607-611, 672-675 */
        if (g > clamp) g = clamp;
        u = u < -clamp ? -clamp : (u > clamp ? clamp : u);
    }
    return silu(g) * u;
}

/* ------------------------------------------------------------ A10-A12 ----
 * Insertion top-K with strict '>' so ties keep the lower expert index; result in
 * descending score order (gemma4.c:596-608, lfm25.c:650-659, maple.c:586-594). */
static void topk_insert(float v, int e, int K, float *topv, int *idx) {
    int j = K;
    while (j > 0 && v > topv[j - 1]) j--;
    if (j == K) return;
    for (int t = K - 1; t > j; t--) { topv[t] = topv[t - 1]; idx[t] = idx[t - 1]; }
    topv[j] = v;
    idx[j] = e;
}

void orc_route(const orc_cfg *c, const orc_weights *w, const float *x,
               int *idx, float *wts, float *logits_out) {
    int D = c->D, E = c->E, K = c->K;
    float topv[64];
    for (int j = 0; j < K; j++) { idx[j] = -1; topv[j] = -INFINITY; }
    if (c->gating == ORC_GATE_GEMMA) {
        /* gemma4.c:581-613 */
        float *xn = (float *)malloc(sizeof(float) * (size_t)D);
        orc_rmsnorm(xn, x, NULL, D, c->eps);
        float rs = 1.0f / sqrtf((float)D);
        for (int i = 0; i < D; i++) xn[i] *= w->router_scale[i] * rs;
        /* The harness's Zipf offset is one float add after the in-order
         * chain, v = fl(chain + bias[e]); selection and softmax both see v. The
         * reference router has no offset (gemma4.c:600-601). sel/soft differ only
         * under a planted mistake. */
        const int zb = c->use_bias && w->bias;
        float *soft = (float *)malloc(sizeof(float) * (size_t)E);
        for (int e = 0; e < E; e++) {
            const float *r = w->router + (size_t)e * D;
            const float b = zb ? w->bias[e] : 0.0f;
            float v = (zb && g_plant == 1) ? b : 0.0f;
            for (int i = 0; i < D; i++) {
                if (zb && g_plant == 2 && i == D - 1) v += b;
                v += r[i] * xn[i];                           /* in order, unfused */
            }
            float sel = v, sv = v;
            if (zb && g_plant == 0) sel = sv = v + b;
            if (zb && g_plant == 3) sv = v + b;
            if (zb && g_plant == 4) sel = v + b;
            soft[e] = sv;
            if (logits_out) logits_out[e] = sel;
            topk_insert(sel, e, K, topv, idx);
        }
        free(xn);
        float sum = 0.0f, mx = soft[idx[0]];
        for (int j = 0; j < K; j++) { wts[j] = expf(soft[idx[j]] - mx); sum += wts[j]; }
        for (int j = 0; j < K; j++) wts[j] = (wts[j] / sum) * w->pes[idx[j]];
        free(soft);
    } else if (c->gating == ORC_GATE_LFM) {
        /* lfm25.c:636-668 */
        float *sg = (float *)malloc(sizeof(float) * (size_t)E);
        for (int e = 0; e < E; e++) {
            const float *r = w->router + (size_t)e * D;
            double v = 0.0;
            for (int i = 0; i < D; i++) v += (double)r[i] * x[i];
            float s = 1.0f / (1.0f + expf(-(float)v));
            sg[e] = s;
            if (logits_out) logits_out[e] = (float)v;
            float sel = (c->use_bias && w->bias) ? s + w->bias[e] : s;
            topk_insert(sel, e, K, topv, idx);
        }
        float sum = 0.0f;
        for (int j = 0; j < K; j++) { wts[j] = sg[idx[j]]; sum += wts[j]; }
        if (c->norm_topk)
            for (int j = 0; j < K; j++) wts[j] /= (sum + 1e-6f);
        for (int j = 0; j < K; j++) wts[j] *= c->routed_scaling;
        free(sg);
    } else if (c->gating == ORC_GATE_LING) {
        /* ling.c:705-789: eight double accumulators (exact products), sigmoid, the bias
         * for selection only; groups ranked by the sum of their two best biased scores,
         * the best topk_group kept (strict '>', lower group on ties); top-K among their
         * experts in ascending expert order; weights the unbiased sigmoid */
        int NG = c->n_group, TG = c->topk_group, EG = E / NG;
        float *rwt = (float *)malloc(sizeof(float) * (size_t)E);
        float *rsel = (float *)malloc(sizeof(float) * (size_t)E);
        for (int e = 0; e < E; e++) {
            const float *r = w->router + (size_t)e * D;
            double s8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int i = 0;
            for (; i + 8 <= D; i += 8)
                for (int k = 0; k < 8; k++) s8[k] += (double)r[i + k] * x[i + k];
            for (; i < D; i++) s8[0] += (double)r[i] * x[i];
            double v = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
            rwt[e] = 1.0f / (1.0f + expf(-(float)v));
            rsel[e] = rwt[e] + ((c->use_bias && w->bias) ? w->bias[e] : 0.0f);
            if (logits_out) logits_out[e] = (float)v;
        }
        float gs[64], topg[64];
        int keep[64];
        unsigned char live[64] = {0};
        for (int g = 0; g < NG; g++) {
            float a = -INFINITY, bb = -INFINITY;
            const float *sg = rsel + (size_t)g * EG;
            for (int i = 0; i < EG; i++) {
                if (sg[i] > a) { bb = a; a = sg[i]; }
                else if (sg[i] > bb) bb = sg[i];
            }
            gs[g] = EG > 1 ? a + bb : a;
        }
        for (int j = 0; j < TG; j++) { keep[j] = -1; topg[j] = -INFINITY; }
        for (int g = 0; g < NG; g++) topk_insert(gs[g], g, TG, topg, keep);
        for (int j = 0; j < TG; j++) if (keep[j] >= 0) live[keep[j]] = 1;
        for (int e = 0; e < E; e++)
            if (live[e / EG]) topk_insert(rsel[e], e, K, topv, idx);
        float sum = 0.0f;
        for (int j = 0; j < K; j++) { wts[j] = rwt[idx[j]]; sum += wts[j]; }
        if (c->norm_topk && K > 1)
            for (int j = 0; j < K; j++) wts[j] /= (sum + 1e-20f);
        for (int j = 0; j < K; j++) wts[j] *= c->routed_scaling;
        free(rwt);
        free(rsel);
    } else {
        /* maple.c:744 (w_dot_f32 logits, 400-410) + route_row 582-601 */
        for (int e = 0; e < E; e++) {
            const float *r = w->router + (size_t)e * D;
            double v = 0.0;
            for (int i = 0; i < D; i++) v += (double)r[i] * x[i];
            float lv = (float)v;
            if (logits_out) logits_out[e] = lv;
            topk_insert(lv, e, K, topv, idx);
        }
        float mx = topv[0], sum = 0.0f;
        for (int j = 0; j < K; j++) { wts[j] = expf(topv[j] - mx); sum += wts[j]; }
        if (c->norm_topk)
            for (int j = 0; j < K; j++) wts[j] /= (sum + 1e-20f);
    }
}

/* ------------------------------------------------------------ A14-A17 ---- */
void orc_dispatch(const int *eidx, const float *ewt, int S, int K, const int *uniq, int nu,
                  int *offs, int *rows, float *wts, int *slots) {
    int n = 0;
    for (int u = 0; u < nu; u++) {
        offs[u] = n;
        for (int s = 0; s < S; s++)
            for (int j = 0; j < K; j++)
                if (eidx[s * K + j] == uniq[u]) {
                    rows[n] = s;
                    if (wts) wts[n] = ewt[s * K + j];
                    if (slots) slots[n] = j;
                    n++;
                }
    }
    offs[nu] = n;
}

static float wdot(int fmt, const uint8_t *T, int O, int o, int I,
                  const int8_t *xq, const float *sx, float tot) {
    if (fmt == ORC_FMT_TQ2) {
        const float *alpha = (const float *)T;
        return orc_tq2_dot(T + (size_t)O * 4 + (size_t)o * (I / 4), alpha[o], xq, sx, tot, I);
    }
    const uint8_t *row = T + (size_t)o * row_bytes(fmt, I);
    return fmt == ORC_FMT_Q80 ? orc_q80_dot(row, xq, sx, I) : orc_q40_dot(row, xq, sx, I);
}

int orc_moe_layer(const orc_cfg *c, const orc_weights *w, const float *in, int S,
                  float *out, int *eidx, float *ewt, int *uniq, int *nu_out, orc_dump *dump) {
    int D = c->D, MI = c->MI, E = c->E, K = c->K;
    if (D % 64 || MI % 64 || K < 1 || K > 64 || K > E || S < 0) return -1;
    if (c->gating == ORC_GATE_LING && (c->n_group < 1 || c->n_group > 64 || E % c->n_group ||
                                       c->topk_group < 1 || c->topk_group > c->n_group))
        return -1;
    int64_t gb = orc_tensor_bytes(c->fmt_gate, MI, D), ub = orc_tensor_bytes(c->fmt_up, MI, D);
    int64_t db = orc_tensor_bytes(c->fmt_down, D, MI);
    if (gb < 0 || ub < 0 || db < 0 || gb + ub + db > w->esz) return -1;

    /* moe_start: route every row, then the first-seen union (gemma4.c:750-765) */
    #pragma omp parallel for schedule(static)
    for (int s = 0; s < S; s++)
        orc_route(c, w, in + (size_t)s * D, eidx + (size_t)s * K, ewt + (size_t)s * K,
                  dump && dump->logits ? dump->logits + (size_t)s * E : NULL);
    int nu = 0;
    for (int s = 0; s < S; s++)
        for (int j = 0; j < K; j++) {
            int e = eidx[s * K + j], seen = 0;
            for (int u = 0; u < nu; u++) if (uniq[u] == e) { seen = 1; break; }
            if (!seen) uniq[nu++] = e;
        }
    *nu_out = nu;

    float *X = (float *)malloc(sizeof(float) * (size_t)S * D + 4);
    if (c->gating == ORC_GATE_GEMMA) {
        for (int s = 0; s < S; s++)
            orc_rmsnorm(X + (size_t)s * D, in + (size_t)s * D, w->pre_ln, D, c->eps);
    } else {
        memcpy(X, in, sizeof(float) * (size_t)S * D);
    }
    memset(out, 0, sizeof(float) * (size_t)S * D);

    /* per-token input quantisation: identical for every expert the token visits */
    int8_t *xq = (int8_t *)malloc((size_t)S * D + 4);
    float *xs = (float *)malloc(sizeof(float) * (size_t)S * (D / BLK) + 4);
    float *xt = (float *)malloc(sizeof(float) * (size_t)S + 4);
    int tq = c->fmt_gate == ORC_FMT_TQ2 || c->fmt_up == ORC_FMT_TQ2;
    for (int s = 0; s < S; s++) {
        if (tq) xt[s] = orc_tq2_quant_act(X + (size_t)s * D, xq + (size_t)s * D, xs + (size_t)s * (D / BLK), D);
        else { orc_quant_act(X + (size_t)s * D, xq + (size_t)s * D, xs + (size_t)s * (D / BLK), D); xt[s] = 0.f; }
    }

    int *offs = (int *)malloc(sizeof(int) * (size_t)(nu + 1));
    int *rows = (int *)malloc(sizeof(int) * (size_t)S * K + 4);
    float *rw = (float *)malloc(sizeof(float) * (size_t)S * K + 4);
    int *slot = (int *)malloc(sizeof(int) * (size_t)S * K + 4);
    orc_dispatch(eidx, ewt, S, K, uniq, nu, offs, rows, rw, slot);
    int tqd = c->fmt_down == ORC_FMT_TQ2;

    /* moe_finish: experts in union order; within an expert the rows are independent */
    for (int u = 0; u < nu; u++) {
        const uint8_t *rec = w->experts + (size_t)uniq[u] * (size_t)w->esz;
        const uint8_t *G = rec, *U = rec + gb, *Dn = rec + gb + ub;
        int n0 = offs[u], n1 = offs[u + 1];
        #pragma omp parallel for schedule(dynamic, 1)
        for (int r = n0; r < n1; r++) {
            int s = rows[r];
            const int8_t *q = xq + (size_t)s * D;
            const float *qs = xs + (size_t)s * (D / BLK);
            float *h = (float *)malloc(sizeof(float) * (size_t)MI);
            int8_t *hq = (int8_t *)malloc((size_t)MI);
            float *hs = (float *)malloc(sizeof(float) * (size_t)(MI / BLK));
            for (int o = 0; o < MI; o++) {
                float g = wdot(c->fmt_gate, G, MI, o, D, q, qs, xt[s]);
                float v = wdot(c->fmt_up, U, MI, o, D, q, qs, xt[s]);
                h[o] = orc_act(c->act, g, v, c->clamp);
            }
            float ht = 0.f;
            if (tqd) ht = orc_tq2_quant_act(h, hq, hs, MI);
            else orc_quant_act(h, hq, hs, MI);
            float ww = rw[r], *os = out + (size_t)s * D;
            for (int o = 0; o < D; o++) os[o] = fmaf(ww, wdot(c->fmt_down, Dn, D, o, MI, hq, hs, ht), os[o]);
            if (dump) {
                size_t p = (size_t)s * K + slot[r];
                if (dump->hq) memcpy(dump->hq + p * MI, hq, (size_t)MI);
                if (dump->hs) memcpy(dump->hs + p * (MI / BLK), hs, sizeof(float) * (MI / BLK));
                if (dump->htot) dump->htot[p] = ht;
            }
            free(h); free(hq); free(hs);
        }
    }
    if (c->gating == ORC_GATE_GEMMA)
        for (int s = 0; s < S; s++)
            orc_rmsnorm(out + (size_t)s * D, out + (size_t)s * D, w->post_ln, D, c->eps);

    if (dump) {
        if (dump->xin) memcpy(dump->xin, X, sizeof(float) * (size_t)S * D);
        if (dump->xq) memcpy(dump->xq, xq, (size_t)S * D);
        if (dump->xs) memcpy(dump->xs, xs, sizeof(float) * (size_t)S * (D / BLK));
        if (dump->xtot) memcpy(dump->xtot, xt, sizeof(float) * (size_t)S);
    }
    free(X); free(xq); free(xs); free(xt); free(offs); free(rows); free(rw); free(slot);
    return 0;
}

/* ------------------------------------------------- gemma around the MoE ---- */
void orc_dense_mlp(const orc_dense *dn, int D, float eps, const float *r, int S, float *h1) {
    const int DI = dn->DI;
    const int64_t gb = orc_tensor_bytes(ORC_FMT_Q40, DI, D);
    const uint8_t *G = dn->mlp, *U = dn->mlp + gb, *Dn = dn->mlp + 2 * gb;
    #pragma omp parallel for schedule(static)
    for (int s = 0; s < S; s++) {
        float *xn = (float *)malloc(sizeof(float) * (size_t)D);
        float *mlp = (float *)malloc(sizeof(float) * (size_t)DI);
        int8_t *xq = (int8_t *)malloc((size_t)(D > DI ? D : DI));
        float *sx = (float *)malloc(sizeof(float) * (size_t)((D > DI ? D : DI) / BLK));
        /* gemma4.c:1014-1020: rmsnorm, matvec(gate), matvec(up), gelu*up, matvec(down),
         * rmsnorm; every matvec quantises its input (gemma4.c:454-459) */
        orc_rmsnorm(xn, r + (size_t)s * D, dn->pre_ffn_ln, D, eps);
        orc_quant_act(xn, xq, sx, D);
        for (int o = 0; o < DI; o++) {
            float g = orc_q40_dot(G + (size_t)o * row_bytes(ORC_FMT_Q40, D), xq, sx, D);
            float u = orc_q40_dot(U + (size_t)o * row_bytes(ORC_FMT_Q40, D), xq, sx, D);
            mlp[o] = orc_act(ORC_ACT_GEGLU_TANH, g, u, 0.0f);
        }
        orc_quant_act(mlp, xq, sx, DI);
        float *h = h1 + (size_t)s * D;
        for (int o = 0; o < D; o++) h[o] = orc_q40_dot(Dn + (size_t)o * row_bytes(ORC_FMT_Q40, DI), xq, sx, DI);
        orc_rmsnorm(h, h, dn->post_ffn_ln1, D, eps);
        free(xn); free(mlp); free(xq); free(sx);
    }
}

int orc_gemma_ffn_block(const orc_cfg *c, const orc_weights *w, const orc_dense *dn, float *H, int S,
                        int *eidx, float *ewt) {
    const int D = c->D;
    if (c->gating != ORC_GATE_GEMMA || dn->DI % 64) return -1;
    float *res = (float *)malloc(sizeof(float) * (size_t)S * D + 4);
    float *h1 = (float *)malloc(sizeof(float) * (size_t)S * D + 4);
    float *h2 = (float *)malloc(sizeof(float) * (size_t)S * D + 4);
    int *uniq = (int *)malloc(sizeof(int) * (size_t)c->E);
    int nu = 0, rc;
    memcpy(res, H, sizeof(float) * (size_t)S * D);              /* gemma4.c:1008 */
    rc = orc_moe_layer(c, w, res, S, h2, eidx, ewt, uniq, &nu, NULL);
    if (rc == 0) {
        orc_dense_mlp(dn, D, c->eps, res, S, h1);
        /* gemma4.c:1022-1030 */
        for (int s = 0; s < S; s++) {
            float *t = h1 + (size_t)s * D, *hs = H + (size_t)s * D;
            const float *a = h2 + (size_t)s * D, *r = res + (size_t)s * D;
            for (int i = 0; i < D; i++) t[i] = t[i] + a[i];
            orc_rmsnorm(t, t, dn->post_ffn_ln, D, c->eps);
            for (int i = 0; i < D; i++) hs[i] = (r[i] + t[i]) * dn->layer_scalar;
        }
    }
    free(res); free(h1); free(h2); free(uniq);
    return rc;
}

void orc_embed_row(const uint8_t *table, int D, float embed_scale, int tok, float *h) {
    const uint8_t *row = table + (size_t)tok * row_bytes(ORC_FMT_Q40, D);
    for (int b = 0; b < D / BLK; b++) {
        const uint8_t *bp = row + (size_t)b * 18;
        float d = blk_scale(bp);
        for (int j = 0; j < 16; j++) {
            h[b * BLK + j] = d * (float)((bp[2 + j] & 15) - 8);
            h[b * BLK + j + 16] = d * (float)((bp[2 + j] >> 4) - 8);
        }
    }
    for (int i = 0; i < D; i++) h[i] *= embed_scale;
}

int orc_head(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
             const float *h, float *logits) {
    float *xn = (float *)malloc(sizeof(float) * (size_t)D);
    int8_t *xq = (int8_t *)malloc((size_t)D);
    float *sx = (float *)malloc(sizeof(float) * (size_t)(D / BLK));
    orc_rmsnorm(xn, h, fnorm, D, eps);
    orc_quant_act(xn, xq, sx, D);
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < V; o++) {
        float v = orc_q40_dot(table + (size_t)o * row_bytes(ORC_FMT_Q40, D), xq, sx, D);
        logits[o] = softcap > 0 ? tanhf(v / softcap) * softcap : v;
    }
    int am = 0;
    for (int i = 1; i < V; i++) if (logits[i] > logits[am]) am = i;
    free(xn); free(xq); free(sx);
    return am;
}

/* The k best of v[] to the front of idx[] (gemma4.c:1112-1131). Only the set that
 * ends in front matters to the caller, but where values tie at the boundary that set
 * depends on the exact steps, so they are kept: the seeded 64-bit LCG, the pivot
 * position it draws, the partition that moves strictly greater values left, and the
 * narrowing on the pivot's final place. */
static void flash_pick(const float *v, int *idx, int n, int k) {
    uint64_t g = 0x9e3779b97f4a7c15ULL;
    int lo = 0, hi = n - 1, t;
    while (lo < hi) {
        g = g * 6364136223846793005ULL + 1442695040888963407ULL;
        const int p = lo + (int)((g >> 33) % (uint64_t)(hi - lo + 1));
        const float pv = v[idx[p]];
        t = idx[p]; idx[p] = idx[hi]; idx[hi] = t;
        int st = lo;
        for (int i = lo; i < hi; i++)
            if (v[idx[i]] > pv) { t = idx[i]; idx[i] = idx[st]; idx[st] = t; st++; }
        t = idx[st]; idx[st] = idx[hi]; idx[hi] = t;
        if (st == k) break;
        if (st < k) lo = st + 1;
        else hi = st - 1;
    }
}

static int cmp_int(const void *a, const void *b) {
    const int x = *(const int *)a, y = *(const int *)b;
    return (x > y) - (x < y);
}

int orc_flash_head(const uint8_t *table, int V, int D, const float *fnorm, float eps, float softcap,
                   const uint8_t *cent, int NC, const int32_t *tmap, int CS, int NP,
                   const float *cscale, int scaled, const int32_t *force, int nforce,
                   const float *h, float *logits, int *sel) {
    if (NP < 1 || NP > NC || CS < 1) return -1;
    float *xn = (float *)malloc(sizeof(float) * (size_t)D);
    int8_t *xq = (int8_t *)malloc((size_t)D);
    float *sx = (float *)malloc(sizeof(float) * (size_t)(D / BLK));
    float *fsim = (float *)malloc(sizeof(float) * (size_t)NC);
    int *idx = (int *)malloc(sizeof(int) * (size_t)NC);
    orc_rmsnorm(xn, h, fnorm, D, eps);
    orc_quant_act(xn, xq, sx, D);
    const size_t rb = row_bytes(ORC_FMT_Q40, D);
    for (int i = 0; i < NC; i++) {
        fsim[i] = orc_q40_dot(cent + (size_t)i * rb, xq, sx, D);
        if (!scaled) fsim[i] *= cscale[i];
        idx[i] = i;
    }
    flash_pick(fsim, idx, NC, NP);
    for (int i = 0; i < V; i++) logits[i] = -INFINITY;
    for (int i = 0; i < NP + (nforce > 0); i++) {
        const int32_t *ids = i < NP ? tmap + (size_t)idx[i] * CS : force;
        const int n = i < NP ? CS : nforce;
        for (int j = 0; j < n; j++) {
            const int id = ids[j];
            if (id < 0 || id >= V) continue;           /* padding slot */
            const float v = orc_q40_dot(table + (size_t)id * rb, xq, sx, D);
            logits[id] = softcap > 0 ? tanhf(v / softcap) * softcap : v;
        }
    }
    int am = 0;
    for (int i = 1; i < V; i++) if (logits[i] > logits[am]) am = i;
    if (sel) {
        memcpy(sel, idx, sizeof(int) * (size_t)NP);
        qsort(sel, (size_t)NP, sizeof(int), cmp_int);
    }
    free(xn); free(xq); free(sx); free(fsim); free(idx);
    return am;
}
