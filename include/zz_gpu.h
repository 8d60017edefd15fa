/* zz_gpu.h -- the accelerator C ABI of the zunzuncito engines, implemented for
 * MI355X (gfx950) by libzzmoe.so.
 *
 * Same symbols, format codes and decline contract as the reference's gpu.h
 * (gpu.h:35-109), so an engine built against this header links against
 * libzzmoe.so instead of metal.o. Every entry point is fallible: 0 means "not
 * done, run the CPU path" and leaves every output untouched (gpu.h:31-33, 76-79;
 * maple.c:621-624 relies on that).
 *
 * Differences forced by a discrete GPU, all inside the same contract:
 *  - gpu_map() cannot wrap host pages without a copy (gpu.h:66-69 "NO copy" is a
 *    unified-memory property). It uploads the range into HBM when called and keeps
 *    a sampled fingerprint of it (the 8 bytes at every 256-byte step). The engines
 *    map each expert slot once, while it is still empty (gemma4.c:2051-2058,
 *    lfm25.c:1894, maple.c:1322, ling.c:1873), and then pread other experts into it
 *    (gemma4.c:484-491). gpu_matmul() therefore compares the tensor's samples with
 *    those of its last upload and, where the host bytes changed, uploads the tensor
 *    again before computing: an engine linked unchanged computes on the expert it
 *    just read. A rewrite that changes none of the sampled words is not seen (an
 *    expert record read over another differs in essentially all of them); mapping
 *    a range inside an existing mapping re-uploads it explicitly. A range that only
 *    overlaps older mappings replaces them (the host memory was reused).
 *  - gpu_matmul() copies x in and y out per call (PCIe), then runs a dequantising
 *    GEMV with f32 activations: the *_dot_f32 semantics (gpu.h:25-27), checked to
 *    < 1e-4 relative like gemma4.c:2315-2368.
 * The MoE-level path that keeps everything resident is in zz_moe.h.
 */
#ifndef ZZ_GPU_H
#define ZZ_GPU_H

#include <stdint.h>
#include <stddef.h>

/* gpu.h:49-52 */
#define GPU_FMT_Q40 1
#define GPU_FMT_Q80 2
#define GPU_FMT_TQ2 3
#define GPU_FMT_Q4A 4   /* gpu_matmul only: Maple's lm_head / FlashHead centroid format */

#ifdef __cplusplus
extern "C" {
#endif

/* gpu.h:61. 1 if a gfx950 device exists and the kernels load; safe to call always.
 * ZZ_DISABLE=1 in the environment makes it decline. */
int  gpu_init(void);
/* gpu.h:62. Releases every mapping, layer and stream. */
void gpu_shutdown(void);
/* gpu.h:63 */
int  gpu_ready(void);
/* gpu.h:64 */
const char *gpu_name(void);

/* gpu.h:69. Upload [p, p+n) into HBM (or re-upload an existing mapping of it). */
int  gpu_map(const void *p, size_t n);

/* gpu.h:74. y[S,O] = W[O,I] (q4_0) x[S,I] (f32), I % 32 == 0, W inside a mapping. */
int  gpu_q40_matmul(float *y, const uint8_t *W, const float *x, int O, int I, int S);

/* gpu.h:83-84. Any GPU_FMT_*. For TQ2, W is the whole tensor (alphas then code rows)
 * and I % 64 == 0; for Q4A (tq2.h:269-292), rows of I/64 groups of 36 bytes and
 * I % 64 == 0. */
int  gpu_matmul(int fmt, float *y, const uint8_t *W, const float *x, int O, int I, int S);

#ifdef __cplusplus
}
#endif

#endif /* ZZ_GPU_H */
