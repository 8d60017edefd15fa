/* ref_kernels.c -- exported wrappers around the reference's header-only kernels.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile against /root/reference
 * (q40.h, tq2.h included in place, never copied) into oracle/_ref/libref_kernels.so,
 * with the reference's AVX2 flags, so the oracle restatement can be diffed against
 * the exact reference arithmetic.
 */
#include "q40.h"
#include "tq2.h"

float    ref_fp16_to_f32(uint16_t h) { return q40_fp16_to_f32(h); }
uint16_t ref_f32_to_fp16(float f) { return q40_f32_to_fp16(f); }
void ref_q40_quant_row(const float *w, uint8_t *d, int I) { q40_quant_row(w, d, I); }
void ref_q80_quant_row(const float *w, uint8_t *d, int I) { q80_quant_row(w, d, I); }
void ref_q40_dequant_row(const uint8_t *s, float *w, int I) { q40_dequant_row(s, w, I); }
void ref_q80_dequant_row(const uint8_t *s, float *w, int I) { q80_dequant_row(s, w, I); }
void ref_quant_act(const float *x, int8_t *q, float *s, int I) { q40_quant_act(x, q, s, I); }
float ref_tq2_quant_act(const float *x, int8_t *q, float *s, int I) { return tq2_quant_act(x, q, s, I); }
float ref_q40_dot(const uint8_t *w, const int8_t *q, const float *s, int I) { return q40_dot(w, q, s, I); }
float ref_q80_dot(const uint8_t *w, const int8_t *q, const float *s, int I) { return q80_dot(w, q, s, I); }
float ref_tq2_dot(const uint8_t *c, float a, const int8_t *q, const float *s, float t, int I) {
    return tq2_dot(c, a, q, s, t, I);
}
float ref_q40_dot_f32(const uint8_t *w, const float *x, int I) { return q40_dot_f32(w, x, I); }
float ref_q80_dot_f32(const uint8_t *w, const float *x, int I) { return q80_dot_f32(w, x, I); }
float ref_tq2_dot_f32(const uint8_t *c, float a, const float *x, int I) { return tq2_dot_f32(c, a, x, I); }
float ref_q4a_dot_f32(const uint8_t *w, const float *x, int I) { return q4a_dot_f32(w, x, I); }
void ref_tq2_dequant_row(const uint8_t *c, float a, float *w, int I) { tq2_dequant_row(c, a, w, I); }
int ref_simd_variant(void) {
#if defined(__AVX2__)
    return 2;
#elif defined(__ARM_NEON)
    return 1;
#else
    return 0;
#endif
}
