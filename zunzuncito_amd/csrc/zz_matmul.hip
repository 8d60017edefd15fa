// zz_matmul.hip -- the gpu.h matmul contract on gfx950: y[S,O] = W[O,I] x[S,I]
// with f32 activations and the weights in the reference's own byte layout
// (gpu.h:71-84). Numerically this is the *_dot_f32 path (q40.h:290-305,
// 443-455; tq2.h:235-252, 405-427): each block's partial is an exact-enough fp32
// sum of small-integer x f32 products scaled once, accumulated in fp32; the
// contract (gemma4.c:2361, maple.c:1813-1815) is relative error < 1e-4 against the
// double reference. Q4A's affine term m * sum(x) is a second per-half partial.
//
// One wave per (row, token); lanes stride the row's blocks.
#include "zz_common.h"
#include "zz_kernels.h"

__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) {
    return (uint16_t)(p[0] | (p[1] << 8));
}

__global__ __launch_bounds__(256) void zz_matmul_f32_kernel(int fmt, float *y, const uint8_t *W,
                                                            const float *x, int O, int I, int S) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), s = blockIdx.y, l = threadIdx.x & 63;
    if (row >= O) return;
    const float *xs = x + (size_t)s * I;
    float acc = 0.0f;
    if (fmt == ZZ_FMT_TQ2) {
        const float alpha = ((const float *)W)[row];
        const uint8_t *c = W + (size_t)O * 4 + (size_t)row * (I / 4);
        for (int g = l; g < I / 64; g += 64) {
            float p = 0.0f;
            for (int k = 0; k < 16; k++) {
                int byte = c[(size_t)g * 16 + k];
#pragma unroll
                for (int q = 0; q < 4; q++)
                    p = fmaf((float)(((byte >> (2 * q)) & 3) - 1), xs[g * 64 + 16 * q + k], p);
            }
            acc += p;
        }
        acc = zz_wave_sum(acc) * alpha;
    } else if (fmt == ZZ_FMT_Q4A) {
        // 64 weights in 36 bytes: fp16 d, fp16 m, then two halves of 16 bytes whose
        // low nibbles are w[j] and high nibbles w[j + 16] (tq2.h:269-282)
        const int ng = I / 64;
        const uint8_t *r = W + (size_t)row * ng * 36;
        for (int g = l; g < ng; g += 64) {
            const uint8_t *grp = r + (size_t)g * 36;
            const float *v = xs + g * 64;
            const float d = zz_h2f(ld_u16(grp)), m = zz_h2f(ld_u16(grp + 2));
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint8_t *nib = grp + 4 + 16 * h;
                const float *u = v + 32 * h;
                float p = 0.0f, t = 0.0f;
                for (int j = 0; j < 16; j++) {
                    p = fmaf((float)(nib[j] & 15), u[j], p);
                    p = fmaf((float)(nib[j] >> 4), u[j + 16], p);
                    t += u[j] + u[j + 16];
                }
                acc = fmaf(d, p, fmaf(m, t, acc));
            }
        }
        acc = zz_wave_sum(acc);
    } else {
        const int nb = I / ZZ_BLK, bb = fmt == ZZ_FMT_Q80 ? 34 : 18;
        const uint8_t *r = W + (size_t)row * nb * bb;
        for (int b = l; b < nb; b += 64) {
            const uint8_t *blk = r + (size_t)b * bb;
            const float *v = xs + b * ZZ_BLK;
            float p = 0.0f;
            if (fmt == ZZ_FMT_Q80) {
                for (int j = 0; j < ZZ_BLK; j++) p = fmaf((float)(int8_t)blk[2 + j], v[j], p);
            } else {
                for (int j = 0; j < 16; j++) {
                    p = fmaf((float)((blk[2 + j] & 15) - 8), v[j], p);
                    p = fmaf((float)((blk[2 + j] >> 4) - 8), v[j + 16], p);
                }
            }
            acc = fmaf(zz_h2f(ld_u16(blk)), p, acc);
        }
        acc = zz_wave_sum(acc);
    }
    if (l == 0) y[(size_t)s * O + row] = acc;
}

int zz_launch_matmul_f32(int fmt, float *y, const uint8_t *W, const float *x, int O, int I,
                         int S, hipStream_t st) {
    hipLaunchKernelGGL(zz_matmul_f32_kernel, dim3((O + 3) / 4, S), dim3(256), 0, st, fmt, y, W,
                       x, O, I, S);
    return hipGetLastError() == hipSuccess;
}
