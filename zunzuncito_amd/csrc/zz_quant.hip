// zz_quant.hip -- weight quantisers on gfx950: f32 rows -> q4_0 / q8_0 blocks in
// the reference's byte layout, bit-exact with q40_quant_row / q80_quant_row
// (q40.h:83-110, 332-348) for finite inputs. This is the converter step
// (tools/convert_*.py) run on the device, so resident expert tables can be built
// without a host round trip. One thread per 32-weight block.
#include "zz_common.h"
#include "zz_kernels.h"

// IEEE binary16 from binary32, round half to even, subnormals kept, signed zeros
// kept (q40.h:60-80 encodes mx/-8 = -0.0 of an all-zero block as 0x8000).
__device__ __forceinline__ uint16_t zz_f2h(float f) {
    uint32_t b = __float_as_uint(f);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t ex = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)ex - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t full = man | 0x800000u;
        int sh = 14 - e;
        uint32_t q = full >> sh, r = full & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (r > half || (r == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = man >> 13, r = man & 0x1fffu;
    uint32_t v = ((uint32_t)e << 10) | q;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) v++;
    if (v >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | v);
}

__global__ void zz_quant_q40_kernel(const float *w, uint8_t *dst, int64_t nblk) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const float *x = w + b * ZZ_BLK;
    float v[ZZ_BLK];
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < ZZ_BLK; j++) {
        v[j] = x[j];
        float a = fabsf(v[j]);
        if (a > amax) { amax = a; mx = v[j]; }     // first element of largest |x|
    }
    // an all-zero block has mx = +0 and the reference stores fp16(0/-8) = -0 (0x8000)
    uint16_t hd = amax == 0.0f ? (uint16_t)0x8000u : zz_f2h(mx / -8.0f);
    float d = zz_h2f(hd);
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t *o = dst + b * 18;
    o[0] = hd & 0xff;
    o[1] = hd >> 8;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int lo = (int)fmaf(v[j], id, 8.5f), hi = (int)fmaf(v[j + 16], id, 8.5f);
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        o[2 + j] = (uint8_t)(lo | (hi << 4));
    }
}

__global__ void zz_quant_q80_kernel(const float *w, uint8_t *dst, int64_t nblk) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const float *x = w + b * ZZ_BLK;
    float amax = 0.0f;
    for (int j = 0; j < ZZ_BLK; j++) amax = fmaxf(amax, fabsf(x[j]));
    uint16_t hd = zz_f2h(amax / 127.0f);
    float d = zz_h2f(hd), id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t *o = dst + b * 34;
    o[0] = hd & 0xff;
    o[1] = hd >> 8;
    for (int j = 0; j < ZZ_BLK; j++) {
        float q = rintf(x[j] * id);
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        o[2 + j] = (uint8_t)(int8_t)(int)q;
    }
}

int zz_launch_quantize(int fmt, const float *w, uint8_t *dst, int64_t nblk, hipStream_t st) {
    dim3 grid((unsigned)((nblk + 255) / 256));
    if (fmt == ZZ_FMT_Q40) hipLaunchKernelGGL(zz_quant_q40_kernel, grid, dim3(256), 0, st, w, dst, nblk);
    else if (fmt == ZZ_FMT_Q80) hipLaunchKernelGGL(zz_quant_q80_kernel, grid, dim3(256), 0, st, w, dst, nblk);
    else return 0;
    return hipGetLastError() == hipSuccess;
}
